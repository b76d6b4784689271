"""GPU parity of the DeltaNet and attention blocks at shapes outside the fused kernels' widths.

The reference's blocks take any shape (reference_kernels.cpp:127-335, qwen35_block.cpp:406-756):
key and value widths of any size, a key width different from the value width in the attention
step, any number of query heads per KV head.  Shapes the fused and chunked kernels do not cover
run the per-stage launches with the any-shape delta rule and attention kernels; OQ_ANY_SHAPE=1
sends every shape there.  Checked here:

- the reference's own known-answer block and attention tests (tests/test_phase1e.cpp:92-186,
  tests/test_phase2c.cpp:182-310: embedding 4, key and value widths 1 and 2), on the device;
- seeded blocks at odd widths, stage by stage against the oracle (the bars of
  tests/test_gpu_deltanet.py and tests/test_gpu_attention.py), F32 and F16 caches, and the
  several-token calls, which run the single step token by token at these shapes;
- the any-shape delta rule gives the register-resident kernel's bits at the widths both take.
"""

import math

import numpy as np
import pytest

import oracle
import oracle_amd
from test_deltanet_oracle import _phase2c_block
from test_gpu_attention import (CHAIN_TOL, THREADS, attention_bar, check_attention, check_block_stages, f16,
                                run_block)
from test_gpu_deltanet import check_history, check_stages, run_gpu

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- DeltaNet

def test_deltanet_reference_known_answers(ctx, kat):
    """tests/test_phase2c.cpp:215-260 on the device: a zero output gate keeps the residual
    (y == x bit for bit), beta = sigmoid(0) = 0.5, the decay gate -log 2, the state takes a
    non-zero update and key heads repeat in tiled order."""
    e = kat["block"]["expect"]
    d, w, vec, hist, st, x = _phase2c_block(kat)
    steps, hist1, st1 = run_gpu(ctx, d, w, vec, hist, st, [x])
    tr = steps[0]["trace"]
    assert np.array_equal(steps[0]["y"], x) == e["output_equals_input"]
    assert abs(float(tr["beta_s"][0]) - e["beta_sigmoid0"]) <= e["tol"]
    assert abs(float(tr["log_decay"][0]) - e["gate0"]) <= e["tol"]
    assert np.any(st1 != 0.0) == e["state_after_nonzero"]
    v = tr["conv"][2 * d["key_heads"] * d["key_dim"]:]
    assert (np.sign(st1.reshape(-1)) * np.sign(v)).tolist() == e["q_predelta_signs"]
    check_stages(d, w, vec, steps[0], st1)
    check_history(steps[0], hist1)


def _deltanet_inputs(dims, types, seed):
    from golden.make_golden import block_inputs
    d = dict(dims, eps=1e-6)
    w, vec, hist, st, xs = block_inputs(np.random.default_rng(seed), d, types)
    return d, w, vec, hist, st, xs


KQ_IN = dict(qkv=12, z=12, beta=12, alpha=12, gate=12, up=12)
DN_SHAPES = {
    # key width 16, value width 48 (a partial 32-column chunk); the out projection's rows of 192
    # on q8_0
    "dk16_dv48": (dict(embedding=256, key_heads=2, value_heads=4, key_dim=16, value_dim=48, conv_kernel=3, ffn=512),
                  dict(KQ_IN, out=8, down=14)),
    # key width 256, two value heads of 128
    "dk256": (dict(embedding=512, key_heads=1, value_heads=2, key_dim=256, value_dim=128, conv_kernel=4, ffn=512),
              dict(KQ_IN, out=12, down=12)),
    # value width 32 and a 20-tap convolution (beyond the fused in-projection's 16)
    "dv32_k20": (dict(embedding=256, key_heads=2, value_heads=8, key_dim=128, value_dim=32, conv_kernel=20, ffn=256),
                 dict(KQ_IN, out=14, down=12)),
    # widths 5 and 3, F32 / F16 / BF16 rows of 8
    "tiny": (dict(embedding=8, key_heads=1, value_heads=2, key_dim=5, value_dim=3, conv_kernel=2, ffn=8),
             dict(qkv=0, z=1, beta=30, alpha=0, out=0, gate=1, up=0, down=30)),
}


@pytest.mark.parametrize("name", list(DN_SHAPES))
def test_deltanet_any_shape_matches_oracle(ctx, name):
    dims, types = DN_SHAPES[name]
    print(f"deltanet any shape {name}", flush=True)
    d, w, vec, hist, st, xs = _deltanet_inputs(dims, types, 7100)
    steps, hist1, st1 = run_gpu(ctx, d, w, vec, hist, st, xs)
    for i, step in enumerate(steps):
        after = steps[i + 1]["state0"] if i + 1 < len(steps) else st1
        check_stages(d, w, vec, step, after)
    check_history(steps[-1], hist1)


@pytest.mark.parametrize("name", ["dk16_dv48", "tiny"])
def test_deltanet_any_shape_tokens_equal_steps(ctx, name):
    """oq_deltanet_steps at these shapes runs the single step token by token: outputs, traces,
    state and history equal three single steps bit for bit."""
    dims, types = DN_SHAPES[name]
    d, w, vec, hist, st, xs = _deltanet_inputs(dims, types, 7200)
    steps, hist1, st1 = run_gpu(ctx, d, w, vec, hist, st, xs)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    sizes = oracle.deltanet_trace_sizes(d)
    per = sum(sizes.values())
    m, E = xs.shape
    bufs = []
    try:
        hb, sb, xb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(np.ascontiguousarray(xs))
        yb, tb = ctx.alloc(m * E * 4), ctx.alloc(m * per * 4)
        bufs = [hb, sb, xb, yb, tb]
        ctx.deltanet_steps(blk, m, hb, sb, xb, yb, tb)
        ctx.sync()
        y = yb.download(np.float32, m * E).reshape(m, E)
        flat = tb.download(np.float32, m * per).reshape(m, per)
        for t, step in enumerate(steps):
            assert np.array_equal(y[t].view(np.uint32), step["y"].view(np.uint32)), t
            want = np.concatenate([step["trace"][n] for n in sizes])
            assert np.array_equal(flat[t].view(np.uint32), want.view(np.uint32)), t
        assert np.array_equal(sb.download(np.float32, st.size).reshape(st.shape), st1)
        assert np.array_equal(hb.download(np.float32, hist.size).reshape(hist.shape), hist1)
    finally:
        for b in bufs:
            b.free()
        blk.release()


SMALL_FAST = dict(embedding=1024, key_heads=2, value_heads=4, key_dim=128, value_dim=128, conv_kernel=4, ffn=1536)


@pytest.mark.parametrize("dims", [
    SMALL_FAST,
    dict(SMALL_FAST, key_dim=64, value_dim=64, value_heads=8, key_heads=4),
    dict(SMALL_FAST, key_dim=32, value_dim=192, key_heads=4),
], ids=["dk128_dv128", "dk64_dv64", "dk32_dv192"])
def test_delta_any_kernel_equals_register_kernel(ctx, dims):
    """At the widths the register-resident delta rule takes, the any-shape kernel (OQ_ANY_SHAPE=1)
    gives its bits: both schedules run one launch per stage (OQ_BLOCK_FUSED=0), so outputs,
    state and history of three steps are equal bit for bit."""
    d, w, vec, hist, st, xs = _deltanet_inputs(dims, dict(KQ_IN, out=14, down=12), 7300)
    runs = []
    for env in ({"OQ_BLOCK_FUSED": "0"}, {"OQ_BLOCK_FUSED": "0", "OQ_ANY_SHAPE": "1"}):
        with oracle_amd.launch_options(env):
            runs.append(run_gpu(ctx, d, w, vec, hist, st, xs))
    (s_a, h_a, st_a), (s_b, h_b, st_b) = runs
    for a, b in zip(s_a, s_b):
        assert np.array_equal(a["y"].view(np.uint32), b["y"].view(np.uint32))
        assert np.array_equal(a["trace"]["rec"].view(np.uint32), b["trace"]["rec"].view(np.uint32))
    assert np.array_equal(st_a.view(np.uint32), st_b.view(np.uint32))
    assert np.array_equal(h_a, h_b)


# ---------------------------------------------------------------- attention step

def test_attention_reference_known_answers(ctx, kat):
    """tests/test_phase1e.cpp:92-186 on the device: two query heads over one KV head of width 2;
    the first step returns the one value row, the second weighs both rows by
    e^(1/sqrt 2) : 1, and a third step overflows the two-row cache."""
    a = kat["attention"]
    cache = ctx.kv_cache(a["capacity"], a["kv_heads"], a["key_dim"], a["value_dim"])
    s0, s1 = a["steps"]
    bufs = []
    try:
        out = ctx.alloc(4 * 4)
        bufs.append(out)
        results = []
        for s in (s0, s1):
            q, k, v = (ctx.to_device(np.array(s[n], np.float32)) for n in ("q", "k", "v"))
            bufs += [q, k, v]
            ctx.attention_step(q, a["q_heads"], k, v, cache, out)
            results.append(out.download(np.float32, 4))
        assert len(cache) == 2
        assert np.allclose(results[0], s0["expected"], atol=a["tol"], rtol=0)
        e = math.exp(1.0 / math.sqrt(2.0))
        p_new = e / (1.0 + e)
        p_old = 1.0 - p_new
        assert abs(results[1][0] - (p_old * 2 + p_new * 4)) <= a["tol"]
        assert abs(results[1][1] - (p_old * 3 + p_new * 5)) <= a["tol"]
        assert np.array_equal(results[1][:2], results[1][2:])
        with pytest.raises(oracle_amd.Overflow, match="KV cache capacity exceeded"):
            ctx.attention_step(bufs[-3], a["q_heads"], bufs[-2], bufs[-1], cache, out)
        assert len(cache) == 2
    finally:
        for b in bufs:
            b.free()
        cache.release()


ANY_STEPS = [(2, 1, 2, 2, 1), (4, 2, 96, 48, 300), (6, 3, 32, 80, 1000), (257, 1, 64, 64, 50), (3, 1, 8192, 16, 5),
             (8, 2, 128, 128, 700)]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("hq,hkv,dk,dv,T", ANY_STEPS, ids=[f"h{a}_{b}_k{c}_v{d}_T{t}" for a, b, c, d, t in ANY_STEPS])
def test_attention_step_any_shape(ctx, hq, hkv, dk, dv, T, dtype):
    """The any-shape kernels against the oracle within 1e-4 of sum_t p_t |v_t|; the new rows are
    appended (rounded to nearest even over an F16 cache).  The last case is a width the chunked
    kernels take, run here with OQ_ANY_SHAPE=1."""
    print(f"attention any shape hq={hq} hkv={hkv} dk={dk} dv={dv} T={T} {dtype}", flush=True)
    rng = np.random.default_rng(2000 + T + hq + dk)
    keys = rng.standard_normal((T, hkv, dk)).astype(np.float32)
    values = rng.standard_normal((T, hkv, dv)).astype(np.float32)
    q = (2.0 * rng.standard_normal((hq, dk)) / math.sqrt(max(1.0, dk / 64))).astype(np.float32)
    stored_k, stored_v = (f16(keys), f16(values)) if dtype == "f16" else (keys, values)
    ref = oracle.KvCache(T + 1, hkv, dk, dv)
    ref.keys[:T - 1] = stored_k[:T - 1]
    ref.values[:T - 1] = stored_v[:T - 1]
    ref.length = T - 1
    want = oracle.attention_step(q, stored_k[T - 1], stored_v[T - 1], ref)
    cache = ctx.kv_cache(T + 1, hkv, dk, dv, dtype=dtype)
    bufs = [ctx.to_device(q), ctx.to_device(keys[T - 1]), ctx.to_device(values[T - 1]), ctx.alloc(hq * dv * 4)]
    env = {"OQ_ANY_SHAPE": "1"} if dk == dv == 128 else {}
    try:
        cache.load(keys[:T - 1], values[:T - 1], T - 1)
        with oracle_amd.launch_options(env):
            ctx.attention_step(bufs[0], hq, bufs[1], bufs[2], cache, bufs[3])
        got = bufs[3].download(np.float32, hq * dv).reshape(hq, dv)
        check_attention(got, want, attention_bar(q, stored_k, stored_v, T), f"T={T}")
        assert len(cache) == T
        k_dev, v_dev = cache.download(hkv, dk, dv)
        assert np.array_equal(k_dev[:T], stored_k) and np.array_equal(v_dev[:T], stored_v)
    finally:
        for b in bufs:
            b.free()
        cache.release()


# ---------------------------------------------------------------- attention block

def test_attention_block_reference_known_answers(ctx, kat):
    """tests/test_phase2c.cpp:284-310 on the device: embedding 4, two query heads over one KV
    head of width 2, F32 projections; y = x + 0.5 x[2 + i % 2] / sqrt(7.5 + eps) and one cache
    row after the step."""
    b = kat["attention_block"]
    d = b["dims"]
    E, Hq, Hkv, D, F = d["embedding"], d["q_heads"], d["kv_heads"], d["head_dim"], d["ffn"]

    def mat(rows, cols, ones):
        m = np.zeros((rows, cols), np.float32)
        for r, c in ones:
            m[r, c] = 1.0
        return (0, m.ravel().view(np.uint8))

    w = {"q": mat(2 * Hq * D, E, b["q_ones"]), "k": mat(Hkv * D, E, b["k_ones"]), "v": mat(Hkv * D, E, b["v_ones"]),
         "out": (0, np.eye(E, dtype=np.float32).ravel().view(np.uint8)), "gate": mat(F, E, []),
         "up": mat(F, E, []), "down": mat(E, F, [])}
    vec = {"input_norm": np.ones(E, np.float32), "q_norm": np.ones(D, np.float32), "k_norm": np.ones(D, np.float32),
           "post_norm": np.ones(E, np.float32)}
    x = np.array(b["input"], np.float32)
    c = oracle.KvCache(4, Hkv, D, D)
    steps = run_block(ctx, d, w, vec, c, [(0, 0, 0)], [x])
    inv = 1.0 / math.sqrt(7.5 + d["eps"])
    expected = [x[i] + 0.5 * x[2 + i % 2] * inv for i in range(E)]
    assert np.allclose(steps[0]["y"], expected, atol=b["tol"], rtol=0)
    assert steps[0]["len1"] == b["cache_after"]
    assert np.allclose(steps[0]["trace"]["gate_s"], 0.5)
    check_block_stages(d, w, vec, steps[0])


ANY_BLOCKS = {
    # heads of 80 (rotation over 32), the out projection's rows of 320 on q8_0
    "d80": (dict(embedding=512, q_heads=4, kv_heads=2, head_dim=80, ffn=512, rope_dim=32,
                 rope_sections=[6, 5, 5, 0], rope_base=1e6, eps=1e-6),
            dict(q=12, k=12, v=12, out=8, gate=12, up=12, down=12), 40),
    # heads of 512, three query heads per KV head
    "d512_rep3": (dict(embedding=256, q_heads=6, kv_heads=2, head_dim=512, ffn=256, rope_dim=64,
                       rope_sections=[11, 11, 10, 0], rope_base=1e7, eps=1e-6),
                  dict(q=12, k=14, v=12, out=12, gate=12, up=12, down=14), 300),
    # heads of 32 from an empty cache, F32 / F16 rows
    "d32_empty": (dict(embedding=96, q_heads=2, kv_heads=1, head_dim=32, ffn=64, rope_dim=32,
                       rope_sections=[8, 4, 4, 0], rope_base=1e4, eps=1e-6),
                  dict(q=0, k=1, v=0, out=30, gate=0, up=1, down=0), 0),
}


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("name", list(ANY_BLOCKS))
def test_attention_block_any_shape(ctx, name, dtype):
    from golden.make_golden import attention_inputs
    d, types, cached = ANY_BLOCKS[name]
    print(f"attention block any shape {name} {dtype}", flush=True)
    w, vec, c, xs = attention_inputs(np.random.default_rng(4343), d, types, cached=cached)
    if dtype == "f16":
        c.keys[:] = f16(c.keys)
        c.values[:] = f16(c.values)
    positions = [(cached + i, cached + i, cached + i) for i in range(2)] + [(cached + 2, 7, 19)]
    steps = run_block(ctx, d, w, vec, c, positions, xs, dtype=dtype)
    for st in steps:
        check_block_stages(d, w, vec, st)
    if dtype == "f32":
        own = c.copy()
        for st in steps:
            y, _ = oracle.attention_block_step(d, w, vec, own, st["pos"], st["x"], threads=THREADS)
            assert float(np.max(np.abs(st["y"] - y))) <= CHAIN_TOL * float(np.max(np.abs(y)))


def test_attention_block_any_shape_forced(ctx):
    """A block of heads of 128 on the any-shape kernels (OQ_ANY_SHAPE=1), stage by stage."""
    from test_gpu_attention import BLOCKS
    from golden.make_golden import attention_inputs
    d, types, cached = BLOCKS["mixed"]
    w, vec, c, xs = attention_inputs(np.random.default_rng(4444), d, types, cached=cached)
    positions = [(cached + i, cached + i, cached + i) for i in range(3)]
    with oracle_amd.launch_options({"OQ_ANY_SHAPE": "1"}):
        steps = run_block(ctx, d, w, vec, c, positions, xs)
    for st in steps:
        check_block_stages(d, w, vec, st)


@pytest.mark.parametrize("name", ["d80", "d32_empty"])
def test_attention_block_any_shape_tokens_equal_steps(ctx, name):
    """oq_attention_block_steps at these shapes runs the single step token by token: outputs,
    traces and cache rows equal three single steps bit for bit."""
    from golden.make_golden import attention_inputs
    d, types, cached = ANY_BLOCKS[name]
    w, vec, c, xs = attention_inputs(np.random.default_rng(4545), d, types, cached=cached)
    positions = [(cached + i, cached + i, cached + i) for i in range(2)] + [(cached + 2, 7, 19)]
    steps = run_block(ctx, d, w, vec, c, positions, xs)
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    hkv, D = d["kv_heads"], d["head_dim"]
    cache = ctx.kv_cache(c.capacity, hkv, D, D)
    sizes = oracle.attention_trace_sizes(d)
    per = sum(sizes.values())
    m, E = xs.shape
    bufs = []
    try:
        cache.load(c.keys[:c.length], c.values[:c.length], c.length)
        xb, yb, tb = ctx.to_device(np.ascontiguousarray(xs)), ctx.alloc(m * E * 4), ctx.alloc(m * per * 4)
        bufs = [xb, yb, tb]
        ctx.attention_block_steps(blk, cache, positions, xb, yb, tb)
        ctx.sync()
        y = yb.download(np.float32, m * E).reshape(m, E)
        flat = tb.download(np.float32, m * per).reshape(m, per)
        for t, st in enumerate(steps):
            assert np.array_equal(y[t].view(np.uint32), st["y"].view(np.uint32)), t
            want = np.concatenate([st["trace"][n] for n in sizes])
            assert np.array_equal(flat[t].view(np.uint32), want.view(np.uint32)), t
        keys, values = cache.download(hkv, D, D)
        assert np.array_equal(keys, steps[-1]["keys1"]) and np.array_equal(values, steps[-1]["values1"])
    finally:
        for b in bufs:
            b.free()
        cache.release()
        blk.release()
