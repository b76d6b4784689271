"""GPU parity of the multi-token full-attention block (oq_attention_block_steps): m consecutive
tokens through one block, against the oracle's restatement of the reference block
(qwen35_block.cpp:607-756) applied token by token, as the reference's multi-token evaluation does
(src/runtime/qwen35_target_multi.cpp:14-25).

Per token, every traced stage is checked as tests/test_gpu_attention.py checks the single step,
from the device's own inputs to it: the cache before token t is the cache before the call with the
device's appended rows of the earlier tokens (the appended rows are checked bit for bit against the
token's traced key and value).  The call prepares every token's heads in one launch and attends for
all tokens in one launch, in chunks laid out for the last token; below 16 tokens its appended rows
are m single steps' bits and its outputs agree with theirs as the attention bar allows
(test_block_steps_equal_single_steps).
"""

import numpy as np
import pytest

import oracle
import oracle_amd
from test_gpu_attention import BLOCKS, CHAIN_TOL, THREADS, check_block_stages, f16

pytestmark = pytest.mark.gpu


# heads of 128 over 12000 cached rows: long chunks (an F16 cache's value rows four per load), and
# from 8192 rows several tokens per chunk workgroup
LONG = {"long128": (dict(embedding=512, q_heads=8, kv_heads=2, head_dim=128, ffn=512, rope_dim=64,
                         rope_sections=[11, 11, 10, 0], rope_base=1e6, eps=1e-6),
                    dict(q=12, k=12, v=12, out=12, gate=12, up=12, down=12), 12000)}


def inputs(name, m, seed):
    from golden.make_golden import attention_inputs
    d, types, cached = BLOCKS[name] if name in BLOCKS else LONG[name]
    w, vec, c, _ = attention_inputs(np.random.default_rng(seed), d, types, cached=cached)
    cache = oracle.KvCache(cached + m, d["kv_heads"], d["head_dim"], d["head_dim"])
    cache.keys[:cached] = c.keys[:cached]
    cache.values[:cached] = c.values[:cached]
    cache.length = cached
    xs = np.random.default_rng(seed + 1).standard_normal((m, d["embedding"])).astype(np.float32)
    positions = [(cached + t, cached + t, cached + t) for t in range(m)]
    if m > 2:
        positions[2] = (cached + 2, 7, 19)  # one multimodal position
    return d, w, vec, cache, xs, positions


def run_tokens(ctx, d, w, vec, c, positions, xs, trace=True, dtype="f32"):
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    hkv, D = d["kv_heads"], d["head_dim"]
    m, E = xs.shape
    cache = ctx.kv_cache(c.capacity, hkv, D, D, dtype=dtype)
    sizes = oracle.attention_trace_sizes(d)
    per = sum(sizes.values())
    bufs = []
    try:
        cache.load(c.keys[:c.length], c.values[:c.length], c.length)
        xb, yb = ctx.to_device(xs), ctx.alloc(m * E * 4)
        bufs += [xb, yb]
        tb = ctx.alloc(m * per * 4) if trace else None
        if tb is not None:
            bufs.append(tb)
        ctx.attention_block_steps(blk, cache, positions, xb, yb, tb)
        ctx.sync()
        traces = []
        if trace:
            flat = tb.download(np.float32, m * per).reshape(m, per)
            for t in range(m):
                tr, off = {}, 0
                for n, sz in sizes.items():
                    tr[n] = flat[t, off:off + sz]
                    off += sz
                traces.append(tr)
        keys, values = cache.download(hkv, D, D)
        return yb.download(np.float32, m * E).reshape(m, E), traces, keys, values, len(cache)
    finally:
        for b in bufs:
            b.free()
        cache.release()
        blk.release()


# OQ_ATTN_SHARE_MIN=0: workgroups serve as many tokens as their 8 query rows hold at any cache
# length (by default only from 8192 cached rows): 4 tokens per workgroup with 1 query head per KV
# head, 3 with 2, 2 with 4, 1 with 8 or 16
SHARE = [{}, {"OQ_ATTN_SHARE_MIN": "0"}]


@pytest.mark.parametrize("env", SHARE, ids=["default", "shared_rows"])
@pytest.mark.parametrize("name,m", [("rep1_d64", 4), ("mixed", 3), ("empty_rep8", 5), ("e2048", 2), ("rep16", 3),
                                    ("e8192", 2), ("e8448", 2), ("e4096", 2)])
def test_block_tokens_match_oracle(ctx, name, m, env):
    d, w, vec, c, xs, positions = inputs(name, m, 9100 + m)
    n0 = c.length
    with oracle_amd.launch_options(env):
        y, traces, keys, values, length = run_tokens(ctx, d, w, vec, c, positions, xs)
    assert length == n0 + m
    assert np.array_equal(keys[:n0], c.keys[:n0]) and np.array_equal(values[:n0], c.values[:n0])
    own = c.copy()
    for t in range(m):
        step = {"x": xs[t], "pos": positions[t], "y": y[t], "trace": traces[t], "keys0": keys, "values0": values,
                "len0": n0 + t, "keys1": keys, "values1": values, "len1": n0 + t + 1}
        check_block_stages(d, w, vec, step)
        y_o, _ = oracle.attention_block_step(d, w, vec, own, positions[t], xs[t], threads=THREADS)
        assert float(np.max(np.abs(y[t] - y_o))) <= CHAIN_TOL * float(np.max(np.abs(y_o))), t


def test_block_tokens_positions_in_device_memory(ctx):
    """Up to 32 tokens' positions travel in the preparation launch's arguments; beyond that they
    are copied to the device: 34 tokens, two of them at multimodal positions, the last one's past
    the first 32."""
    m = 34
    d, w, vec, c, xs, positions = inputs("rep1_d64", m, 9300)
    positions[33] = (c.length + 33, 5, 11)
    n0 = c.length
    y, traces, keys, values, length = run_tokens(ctx, d, w, vec, c, positions, xs)
    assert length == n0 + m
    for t in (0, 2, 31, 32, 33):
        step = {"x": xs[t], "pos": positions[t], "y": y[t], "trace": traces[t], "keys0": keys, "values0": values,
                "len0": n0 + t, "keys1": keys, "values1": values, "len1": n0 + t + 1}
        check_block_stages(d, w, vec, step)


# The matrix-core products' bound on rows that a few products lead (2^-10 of sum |w xhat| plus
# binary16-subnormal weights and F32 summation)
DOMINATED_TOL = 1.5e-3


@pytest.mark.parametrize("env", SHARE, ids=["default", "shared_rows"])
@pytest.mark.parametrize("name", ["e2048", "long128"])
def test_block_tokens_f16_cache(ctx, env, name):
    """m tokens over an F16 cache: each token's stages, its key and value appended rounded, and
    every later token attending over the rounded rows (e2048: heads of 256 over 1000 cached rows,
    with OQ_ATTN_SHARE_MIN=0 several tokens per workgroup; long128: heads of 128 over 12000)."""
    d, w, vec, c, xs, positions = inputs(name, 4, 9500)
    n0 = c.length
    with oracle_amd.launch_options(env):
        y, traces, keys, values, length = run_tokens(ctx, d, w, vec, c, positions, xs, dtype="f16")
    assert length == n0 + 4
    assert np.array_equal(keys[:n0], f16(c.keys[:n0])) and np.array_equal(values[:n0], f16(c.values[:n0]))
    for t in range(4):
        step = {"x": xs[t], "pos": positions[t], "y": y[t], "trace": traces[t], "keys0": keys, "values0": values,
                "len0": n0 + t, "keys1": keys, "values1": values, "len1": n0 + t + 1, "kv16": True}
        check_block_stages(d, w, vec, step)


@pytest.mark.parametrize("env", [{}, {"OQ_GEMM_MFMA": "0"}], ids=["matrix_cores", "integer_dots"])
def test_block_tokens_full_block_matrix_cores(ctx, env):
    """The hidden-4096 block (16 query heads over 4 KV heads of 256, FFN 12288) over 16 tokens after
    4000 cached ones: every projection takes the matrix-core path.  Tokens 0, 9 and 15 are checked
    stage by stage.  The down projection's input here is a saturated SwiGLU output (gate values far
    below zero on most tokens, so a few products lead each output): on matrix cores it is held to
    the f16 products' bound, DOMINATED_TOL, and with OQ_GEMM_MFMA=0 (integer dots at every m) the
    same call meets 1e-4 everywhere."""
    d, w, vec, c, xs, positions = inputs("e4096", 16, 9200)
    n0 = c.length
    with oracle_amd.launch_options(env):
        y, traces, keys, values, length = run_tokens(ctx, d, w, vec, c, positions, xs)
    assert length == n0 + 16 and np.all(np.isfinite(y))
    for t in (0, 9, 15):
        step = {"x": xs[t], "pos": positions[t], "y": y[t], "trace": traces[t], "keys0": keys, "values0": values,
                "len0": n0 + t, "keys1": keys, "values1": values, "len1": n0 + t + 1}
        check_block_stages(d, w, vec, step, proj_tol=None if env else {"ffn": DOMINATED_TOL})


@pytest.mark.parametrize("env", SHARE, ids=["default", "shared_rows"])
@pytest.mark.parametrize("m", [2, 4])
def test_block_tokens_trace_does_not_change_results(ctx, env, m):
    """The trace only adds stores: outputs and cache equal bit for bit with and without it."""
    d, w, vec, c, xs, positions = inputs("e2048", m, 9600)
    with oracle_amd.launch_options(env):
        y0, _, k0, v0, n0 = run_tokens(ctx, d, w, vec, c, positions, xs, trace=False)
        y1, _, k1, v1, n1 = run_tokens(ctx, d, w, vec, c, positions, xs, trace=True)
    assert n0 == n1 == c.length + m
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)


def test_block_steps_equal_single_steps(ctx):
    """Below 16 tokens the projections are the single step's per-stage kernels (OQ_BLOCK_FUSED=0)
    and the head preparation is the single step's arithmetic: the appended cache rows equal m single
    steps' bit for bit.  Attention sums over other chunk boundaries (the call's chunks are laid out
    for its last token), so the outputs agree within the wiring bound."""
    d, w, vec, c, xs, positions = inputs("rep1_d64", 4, 9300)
    y, _, keys, values, _ = run_tokens(ctx, d, w, vec, c, positions, xs, trace=False)
    hkv, D = d["kv_heads"], d["head_dim"]
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    cache = ctx.kv_cache(c.capacity, hkv, D, D)
    try:
        cache.load(c.keys[:c.length], c.values[:c.length], c.length)
        yb = ctx.alloc(d["embedding"] * 4)
        ys = []
        with oracle_amd.launch_options({"OQ_BLOCK_FUSED": "0"}):
            for t in range(len(xs)):
                xb = ctx.to_device(xs[t])
                ctx.attention_block_step(blk, cache, positions[t], xb, yb)
                ctx.sync()
                ys.append(yb.download(np.float32, d["embedding"]))
                xb.free()
        single = np.stack(ys)
        assert float(np.max(np.abs(single - y))) <= CHAIN_TOL * float(np.max(np.abs(single)))
        k1, v1 = cache.download(hkv, D, D)
        assert np.array_equal(k1, keys) and np.array_equal(v1, values)
        yb.free()
    finally:
        cache.release()
        blk.release()


def test_block_tokens_errors(ctx):
    d, w, vec, c, xs, positions = inputs("rep1_d64", 3, 9400)
    hkv, D = d["kv_heads"], d["head_dim"]
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    small = ctx.kv_cache(c.length + 2, hkv, D, D)
    try:
        small.load(c.keys[:c.length], c.values[:c.length], c.length)
        xb, yb = ctx.to_device(xs), ctx.alloc(xs.size * 4)
        with pytest.raises(oracle_amd.Overflow, match="KV cache capacity exceeded"):
            ctx.attention_block_steps(blk, small, positions, xb, yb)
        assert len(small) == c.length
        with pytest.raises(oracle_amd.InvalidArgument, match="token count must be non-zero"):
            ctx.attention_block_steps(blk, small, [], xb, yb)
        with pytest.raises(oracle_amd.InvalidArgument, match="sum to half the rotary dimension"):
            blk.desc.rope_sections[0] += 1
            ctx.attention_block_steps(blk, small, positions[:2], xb, yb)
        assert len(small) == c.length
        for b in (xb, yb):
            b.free()
    finally:
        small.release()
        blk.release()
