"""GPU parity of the full-attention decode path against the oracle's restatement of the
reference (reference_kernels.cpp:77-195, qwen35_block.cpp:607-756) on identical seeded inputs.

- RoPE (oq_rope): within 2^-21 of |a| + |b| of the rotated pair (cos and sin in double on the
  device, from glibc in the reference; the F32 rotation itself is the reference's), exact for
  almost every element;
- attention (oq_attention_step): |out - ref| <= 1e-4 * sum_t p_t |v_t| per output (F32 chunked
  sums against the reference's double dot products and token-order F32 sum); the appended cache
  rows bit for bit;
- the block (oq_attention_block_step) stage by stage, each stage from the device's own inputs to
  it as in the DeltaNet block tests, and end to end as a wiring check.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-4     # attention outputs, normalised by sum_t p_t |v_t|
TOL = 1e-4          # projections, normalised by sum |w xhat|
STAGE_TOL = 2e-6    # elementwise / per-head stages, relative to the stage's max |value|
CHAIN_TOL = 5e-2    # end-to-end y, relative to max |y| (wiring check)
THREADS = min(16, oracle.default_threads())
KQ = (12, 13, 14)


@pytest.fixture(scope="module")
def ctx():
    c = oracle_amd.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def attn_golden():
    from conftest import GOLDEN
    with np.load(GOLDEN / "ref_attention.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def attention_bar(q, keys, values, length):
    """sum_t p_t |v_t| per output [Hq][D] in float64 (q [Hq][D], keys/values [T][Hkv][D])."""
    hq, d = q.shape
    hkv = keys.shape[1]
    rep = hq // hkv
    out = np.empty((hq, values.shape[2]))
    for h in range(hq):
        k = keys[:length, h // rep].astype(np.float64)
        s = k @ q[h].astype(np.float64) / math.sqrt(d)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ np.abs(values[:length, h // rep].astype(np.float64))
    return out


def check_attention(got, want, bar, what):
    err = float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(bar, 1e-30)))
    assert err <= ATTN_TOL, f"{what}: normalised error {err:.3e}"
    return err


# ---------------------------------------------------------------- RoPE

def rope_close(got, want, x, half):
    a = np.abs(x[:, :half]) + np.abs(x[:, half:2 * half])
    scale = np.concatenate([a, a, np.abs(x[:, 2 * half:])], axis=1)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 2.0 ** -21 * scale + 1e-30), float(np.max(err / (scale + 1e-30)))
    return float(np.mean(got == want))


def test_rope_matches_reference_fixture(ctx, attn_golden):
    """Bit for bit: a single-position rotation of up to 128 frequency pairs takes its cos / sin
    from the host, computed as apply_qwen35_rope computes them (reference_kernels.cpp:105-115),
    and rotates in the reference's F32 operations."""
    g = attn_golden
    x = g["rope_in"]
    buf = ctx.alloc(x.nbytes)
    try:
        for name in ("text", "mm", "far"):
            buf.upload(x)
            ctx.rope(buf, x.shape[0], x.shape[1], 64, [11, 11, 10, 0], 1e7, tuple(int(v) for v in g[f"rope_{name}_pos"]))
            got = buf.download(np.float32, x.size).reshape(x.shape)
            assert np.array_equal(got.view(np.uint32), g[f"rope_{name}_bits"]), name
    finally:
        buf.free()


def test_rope_known_answers_and_sizes(ctx, kat):
    r = kat["rope"]
    for spec in (r, kat["mrope"]):
        x = np.array([spec["head"]], np.float32)
        buf = ctx.to_device(x)
        ctx.rope(buf, 1, x.shape[1], spec["rotary_dim"], spec["sections"], spec["base"], spec["position"])
        got = buf.download(np.float32, x.size)
        buf.free()
        want = oracle.rope(x, spec["rotary_dim"], spec["sections"], spec["base"], spec["position"])[0]
        assert np.allclose(got, want, atol=spec["tol"], rtol=0)
    rng = np.random.default_rng(3)
    # up to 128 frequency pairs: the host's table, bit-exact; 256 pairs (rotary dimension 512): the
    # device's double-precision angles, within 2^-21 of the pair (>= 99 % bit-exact)
    for n, hd, rd, sec in ((3, 128, 128, [22, 21, 21, 0]), (40, 256, 64, [11, 11, 10, 0]), (1, 2, 2, [1, 0, 0, 0]),
                           (7, 96, 48, [8, 8, 8, 0]), (2, 512, 512, [86, 85, 85, 0])):
        x = rng.standard_normal((n, hd)).astype(np.float32)
        pos = (int(rng.integers(0, 300000)), int(rng.integers(0, 64)), int(rng.integers(0, 64)))
        buf = ctx.to_device(x)
        ctx.rope(buf, n, hd, rd, sec, 1e6, pos)
        got = buf.download(np.float32, x.size).reshape(x.shape)
        buf.free()
        want = oracle.rope(x, rd, sec, 1e6, pos)
        if rd // 2 <= 128:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, hd, rd)
        else:
            assert rope_close(got, want, x, rd // 2) >= 0.99


def test_rope_errors(ctx):
    buf = ctx.alloc(64)
    try:
        for rd, sec, base, msg in ((0, [0, 0, 0, 0], 1.0, "RoPE dimension must be non-zero, even, and within head width"),
                                   (6, [3, 0, 0, 0], 1.0, "RoPE dimension must be non-zero, even, and within head width"),
                                   (4, [2, 0, 0, 0], -1.0, "RoPE frequency base must be positive and finite"),
                                   (4, [3, -1, 0, 0], 1.0, "RoPE dimension sections must be non-negative"),
                                   (4, [1, 0, 0, 0], 1.0, "RoPE dimension sections must sum to half the rotary dimension")):
            with pytest.raises(oracle_amd.InvalidArgument, match=msg):
                ctx.rope(buf, 1, 4, rd, sec, base, (1, 1, 1))
    finally:
        buf.free()


# ---------------------------------------------------------------- attention step

def test_attention_step_matches_reference_fixture(ctx, attn_golden):
    g = attn_golden
    steps, hq, d = g["attn_q"].shape
    hkv = g["attn_k"].shape[1]
    cache = ctx.kv_cache(16, hkv, d, d)
    qb, kb, vb, ob = ctx.alloc(hq * d * 4), ctx.alloc(hkv * d * 4), ctx.alloc(hkv * d * 4), ctx.alloc(hq * d * 4)
    try:
        for i in range(steps):
            qb.upload(g["attn_q"][i])
            kb.upload(g["attn_k"][i])
            vb.upload(g["attn_v"][i])
            ctx.attention_step(qb, hq, kb, vb, cache, ob)
            got = ob.download(np.float32, hq * d).reshape(hq, d)
            assert len(cache) == i + 1
            bar = attention_bar(g["attn_q"][i], g["attn_k"][:i + 1], g["attn_v"][:i + 1], i + 1)
            check_attention(got, g["attn_y_bits"][i].view(np.float32), bar, f"step {i}")
        keys, values = cache.download(hkv, d, d)
        assert np.array_equal(keys[:steps], g["attn_k"]) and np.array_equal(values[:steps], g["attn_v"])
        assert not np.any(keys[steps:]) and not np.any(values[steps:])
    finally:
        for b in (qb, kb, vb, ob):
            b.free()
        cache.release()


# (q_heads, kv_heads, head_dim, tokens after the step): group sizes 1-8, chunk edges, long caches;
# groups above 8 query heads run as equal subgroups of at most 8: 16 (two of 8), 12 (two of 6),
# 9 (three of 3), 11 (a prime: eleven single heads)
CASES = [(8, 2, 256, 1), (8, 2, 256, 17), (16, 4, 256, 4097), (8, 2, 256, 20000), (8, 1, 128, 777),
         (4, 4, 64, 300), (6, 2, 128, 301), (24, 4, 256, 3000), (16, 2, 256, 50), (16, 4, 256, 65537),
         (32, 2, 256, 4097), (16, 1, 256, 1), (24, 2, 128, 301), (18, 2, 64, 300), (11, 1, 64, 77)]


@pytest.mark.parametrize("hq,hkv,d,T", CASES, ids=[f"h{a}_{b}_d{c}_T{t}" for a, b, c, t in CASES])
def test_attention_step_sizes(ctx, hq, hkv, d, T):
    print(f"attention step hq={hq} hkv={hkv} d={d} T={T}", flush=True)
    rng = np.random.default_rng(1000 + T + hq)
    keys = rng.standard_normal((T, hkv, d)).astype(np.float32)
    values = rng.standard_normal((T, hkv, d)).astype(np.float32)
    q = (2.0 * rng.standard_normal((hq, d))).astype(np.float32)
    ref_cache = oracle.KvCache(T + 1, hkv, d, d)
    ref_cache.keys[:T - 1] = keys[:T - 1]
    ref_cache.values[:T - 1] = values[:T - 1]
    ref_cache.length = T - 1
    want = oracle.attention_step(q, keys[T - 1], values[T - 1], ref_cache)
    cache = ctx.kv_cache(T + 1, hkv, d, d)
    bufs = [ctx.to_device(q), ctx.to_device(keys[T - 1]), ctx.to_device(values[T - 1]), ctx.alloc(hq * d * 4)]
    try:
        cache.load(keys[:T - 1], values[:T - 1], T - 1)
        ctx.attention_step(bufs[0], hq, bufs[1], bufs[2], cache, bufs[3])
        got = bufs[3].download(np.float32, hq * d).reshape(hq, d)
        check_attention(got, want, attention_bar(q, keys, values, T), f"T={T}")
        assert len(cache) == T
        k_dev, v_dev = cache.download(hkv, d, d)
        assert np.array_equal(k_dev[T - 1], keys[T - 1]) and np.array_equal(v_dev[T - 1], values[T - 1])
        assert np.array_equal(k_dev[:T - 1], keys[:T - 1])
    finally:
        for b in bufs:
            b.free()
        cache.release()


def f16(a):
    """The value an F16 cache stores for F32 elements (round to nearest even)."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


# long chunks of rows of 128 and 256 load several value rows per instruction (4 and 2): 65537 and
# 4097 rows over 4 KV heads, 20000 over 2 and 30001 over one (16 query heads: two subgroups)
F16_CASES = [(8, 2, 256, 1), (16, 4, 256, 4097), (8, 1, 128, 777), (4, 4, 64, 300), (6, 2, 128, 301),
             (32, 2, 256, 4097), (16, 4, 256, 65537), (8, 2, 128, 20000), (16, 1, 128, 30001)]


@pytest.mark.parametrize("hq,hkv,d,T", F16_CASES, ids=[f"h{a}_{b}_d{c}_T{t}" for a, b, c, t in F16_CASES])
def test_attention_step_f16_cache(ctx, hq, hkv, d, T):
    """An F16 cache: loaded and appended rows are the F32 rows rounded to nearest even (bit for
    bit), and attention runs over the stored rows, the new token's included, within the same bar
    as over an F32 cache."""
    print(f"attention step f16 cache hq={hq} hkv={hkv} d={d} T={T}", flush=True)
    rng = np.random.default_rng(2000 + T + hq)
    keys = rng.standard_normal((T, hkv, d)).astype(np.float32)
    values = rng.standard_normal((T, hkv, d)).astype(np.float32)
    q = (2.0 * rng.standard_normal((hq, d))).astype(np.float32)
    k16, v16 = f16(keys), f16(values)
    ref_cache = oracle.KvCache(T + 1, hkv, d, d)
    ref_cache.keys[:T - 1] = k16[:T - 1]
    ref_cache.values[:T - 1] = v16[:T - 1]
    ref_cache.length = T - 1
    want = oracle.attention_step(q, k16[T - 1], v16[T - 1], ref_cache)
    cache = ctx.kv_cache(T + 1, hkv, d, d, dtype="f16")
    bufs = [ctx.to_device(q), ctx.to_device(keys[T - 1]), ctx.to_device(values[T - 1]), ctx.alloc(hq * d * 4)]
    try:
        cache.load(keys[:T - 1], values[:T - 1], T - 1)
        ctx.attention_step(bufs[0], hq, bufs[1], bufs[2], cache, bufs[3])
        got = bufs[3].download(np.float32, hq * d).reshape(hq, d)
        check_attention(got, want, attention_bar(q, k16, v16, T), f"T={T}")
        assert len(cache) == T
        k_dev, v_dev = cache.download(hkv, d, d)
        assert np.array_equal(k_dev[:T], k16) and np.array_equal(v_dev[:T], v16)
        assert not np.any(k_dev[T:]) and not np.any(v_dev[T:])
    finally:
        for b in bufs:
            b.free()
        cache.release()


def test_kv_cache_f16_rounding_and_errors(ctx):
    """Loaded rows round to nearest even, ties included, subnormal and overflowing values too;
    reset zeroes the binary16 arrays; an element type other than F32 / F16 is refused."""
    vals = np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, -70000.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25,
                     2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 0.1, -1e-7, 1234.5678], np.float32)
    rows = np.tile(vals, 8).reshape(2, 1, 64)
    cache = ctx.kv_cache(4, 1, 64, 64, dtype="f16")
    try:
        cache.load(rows, -rows, 2)
        k, v = cache.download(1, 64, 64)
        assert np.array_equal(k[:2].view(np.uint32), f16(rows).view(np.uint32))
        assert np.array_equal(v[:2].view(np.uint32), f16(-rows).view(np.uint32))
        cache.reset()
        k, v = cache.download(1, 64, 64)
        assert len(cache) == 0 and not np.any(k) and not np.any(v)
    finally:
        cache.release()
    h = C.c_void_p()
    rc = ctx.lib.oq_kv_cache_create_typed(ctx.h, 4, 1, 64, 64, 8, C.byref(h))
    assert rc == -1 and b"KV cache element type must be F32 or F16" in ctx.lib.oq_last_error(ctx.h)
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.kv_cache(4, 1, 64, 64, dtype="q8_0")


def test_attention_step_errors(ctx):
    cache = ctx.kv_cache(2, 2, 64, 64)
    q, k, v, o = ctx.alloc(6 * 64 * 4), ctx.alloc(2 * 64 * 4), ctx.alloc(2 * 64 * 4), ctx.alloc(6 * 64 * 4)
    try:
        with pytest.raises(oracle_amd.InvalidArgument, match="causal_attention_step dimensions are incompatible"):
            ctx.attention_step(q, 3, k, v, cache, o)
        cache.load(np.zeros((2, 2, 64), np.float32), np.zeros((2, 2, 64), np.float32), 2)
        with pytest.raises(oracle_amd.Overflow, match="KV cache capacity exceeded"):
            ctx.attention_step(q, 6, k, v, cache, o)
        assert len(cache) == 2
        with pytest.raises(oracle_amd.InvalidArgument, match="KV cache truncate must not grow state"):
            cache.truncate(3)
        cache.truncate(1)
        assert len(cache) == 1
        cache.reset()
        assert len(cache) == 0
        keys, values = cache.download(2, 64, 64)
        assert not np.any(keys) and not np.any(values)
        with pytest.raises(oracle_amd.InvalidArgument, match="KV cache capacity must be non-zero"):
            ctx.kv_cache(0, 1, 64, 64)
        # key rows wider than the any-shape kernels' LDS row (other widths: tests/test_gpu_any_shape.py)
        wide = ctx.kv_cache(4, 1, 8193, 64)
        try:
            with pytest.raises(oracle_amd.InvalidArgument, match="attention device path needs key_dim <= 8192"):
                ctx.attention_step(q, 1, k, v, wide, o)
            assert len(wide) == 0
        finally:
            wide.release()
    finally:
        for b in (q, k, v, o):
            b.free()
        cache.release()


# ---------------------------------------------------------------- the block

def run_block(ctx, d, w, vec, cache_np, positions, xs, dtype="f32"):
    """Device steps; per step: y, trace and the cache arrays before the step."""
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    hkv, D = d["kv_heads"], d["head_dim"]
    cache = ctx.kv_cache(cache_np.capacity, hkv, D, D, dtype=dtype)
    try:
        cache.load(cache_np.keys, cache_np.values, cache_np.length)
        sizes = oracle.attention_trace_sizes(d)
        tb = ctx.alloc(sum(sizes.values()) * 4)
        yb = ctx.alloc(d["embedding"] * 4)
        steps = []
        for x, pos in zip(xs, positions):
            k0, v0 = cache.download(hkv, D, D)
            n0 = len(cache)
            xb = ctx.to_device(x)
            ctx.attention_block_step(blk, cache, pos, xb, yb, tb)
            ctx.sync()
            flat = tb.download(np.float32, sum(sizes.values()))
            tr, off = {}, 0
            for n, sz in sizes.items():
                tr[n] = flat[off:off + sz]
                off += sz
            k1, v1 = cache.download(hkv, D, D)
            steps.append({"x": x, "pos": pos, "y": yb.download(np.float32, d["embedding"]), "trace": tr,
                          "keys0": k0, "values0": v0, "len0": n0, "keys1": k1, "values1": v1, "len1": len(cache),
                          "kv16": dtype == "f16"})
            xb.free()
        tb.free()
        yb.free()
        return steps
    finally:
        cache.release()
        blk.release()


def project(w, name, inp, rows, cols):
    t, data = w[name]
    xhat = oracle.dequantize_q8k(oracle.quantize_q8k(inp), cols) if t in KQ else inp
    y = oracle.storage_matvec(t, rows, cols, data, xhat, threads=THREADS)
    return y, oracle.matvec_stats(t, rows, cols, data, xhat, threads=THREADS)[1]


def close(name, got, want, worst):
    scale = float(np.max(np.abs(want))) or 1.0
    worst[name] = float(np.max(np.abs(got.astype(np.float64) - want))) / scale
    assert worst[name] <= STAGE_TOL, f"{name}: error {worst[name]:.3e} of scale"


def check_block_stages(d, w, vec, step, proj_tol=None):
    """Every traced stage of one block step from the device's inputs to it; proj_tol maps a
    projection's trace name to a bound other than TOL."""
    E, F, Hq, Hkv, D, eps = (d[k] for k in ("embedding", "ffn", "q_heads", "kv_heads", "head_dim", "eps"))
    Q, KV = Hq * D, Hkv * D
    g, x = step["trace"], step["x"]
    worst = {}
    normed = oracle.rms_norm_rows(x, vec["input_norm"], E, eps)
    projections = {"qfull": ("q", normed, 2 * Q, E), "k": ("k", normed, KV, E), "v": ("v", normed, KV, E),
                   "branch": ("out", g["gated"], E, Q), "gate": ("gate", g["post"], F, E),
                   "up": ("up", g["post"], F, E), "ffn": ("down", g["act"], E, F)}
    for n, (wn, inp, rows, cols) in projections.items():
        y, norm = project(w, wn, inp, rows, cols)
        worst[n] = float(np.max(np.abs(g[n].astype(np.float64) - y) / np.maximum(norm, 1e-30)))
        assert worst[n] <= (proj_tol or {}).get(n, TOL), f"{n}: normalised error {worst[n]:.3e}"
    qf = g["qfull"].reshape(Hq, 2 * D)
    rd, sec, base = d["rope_dim"], d["rope_sections"], d["rope_base"]
    qn = oracle.rms_norm_rows(qf[:, :D].reshape(-1), vec["q_norm"], D, eps).reshape(Hq, D)
    kn = oracle.rms_norm_rows(g["k"], vec["k_norm"], D, eps).reshape(Hkv, D)
    close("qcur", g["qcur"], oracle.rope(qn, rd, sec, base, step["pos"]).reshape(-1), worst)
    close("kcur", g["kcur"], oracle.rope(kn, rd, sec, base, step["pos"]).reshape(-1), worst)
    n0 = step["len0"]
    c = oracle.KvCache(step["keys0"].shape[0], Hkv, D, D)
    c.keys[:] = step["keys0"]
    c.values[:] = step["values0"]
    c.length = n0
    q = g["qcur"].reshape(Hq, D)
    # the new token's rows as the cache stores them (an F16 cache: rounded to nearest even)
    knew, vnew = g["kcur"].reshape(Hkv, D), g["v"].reshape(Hkv, D)
    if step.get("kv16"):
        knew, vnew = f16(knew), f16(vnew)
    att = oracle.attention_step(q, knew, vnew, c)
    bar = attention_bar(q, c.keys, c.values, n0 + 1)
    worst["pregate"] = check_attention(g["pregate"].reshape(Hq, D), att, bar, "pregate")
    gs = np.array([oracle.sigmoid(v) for v in qf[:, D:].reshape(-1)], np.float32)
    close("gate_s", g["gate_s"], gs, worst)
    close("gated", g["gated"], g["pregate"] * g["gate_s"], worst)
    close("resid", g["resid"], x + g["branch"], worst)
    close("post", g["post"], oracle.rms_norm_rows(g["resid"], vec["post_norm"], E, eps), worst)
    close("act", g["act"], np.array([oracle.silu(a) for a in g["gate"]], np.float32) * g["up"], worst)
    close("y", step["y"], g["resid"] + g["ffn"], worst)
    # the append: row n0 holds the rotated key and the value; nothing else changed
    assert step["len1"] == n0 + 1
    assert np.array_equal(step["keys1"][n0].reshape(-1), knew.reshape(-1))
    assert np.array_equal(step["values1"][n0].reshape(-1), vnew.reshape(-1))
    assert np.array_equal(step["keys1"][:n0], step["keys0"][:n0])
    return worst


def test_attention_block_reference_fixture_stages(ctx, attn_golden):
    """The committed kq block case (q4_K / q6_K projections, one multimodal position)."""
    from golden.make_golden import ATTN_KQ_DIMS, ATTN_POSITIONS
    g = attn_golden
    d = ATTN_KQ_DIMS
    w = {n: (int(g[f"kq_t_{n}"][0]), g[f"kq_w_{n}"]) for n in oracle.ATTN_WEIGHTS}
    vec = {n: g[f"kq_v_{n}"] for n in oracle.ATTN_VECTORS}
    c = oracle.KvCache(*g["kq_keys0"].shape, g["kq_values0"].shape[2])
    c.keys[:] = g["kq_keys0"]
    c.values[:] = g["kq_values0"]
    c.length = int(g["kq_length0"][0])
    steps = run_block(ctx, d, w, vec, c, ATTN_POSITIONS, g["kq_x"])
    for i, st in enumerate(steps):
        check_block_stages(d, w, vec, st)
        want = g["kq_y_bits"][i].view(np.float32)
        assert float(np.max(np.abs(st["y"] - want))) <= CHAIN_TOL * float(np.max(np.abs(want)))


BLOCKS = {
    # the 2B checkpoint's attention geometry (8 query heads over 2 KV heads of 256, MRoPE 64)
    "e2048": (dict(embedding=2048, q_heads=8, kv_heads=2, head_dim=256, ffn=6144, rope_dim=64,
                   rope_sections=[11, 11, 10, 0], rope_base=1e7, eps=1e-6),
              dict(q=12, k=12, v=12, out=14, gate=12, up=12, down=14), 1000),
    # hidden 4096: 16 query heads over 4 KV heads
    "e4096": (dict(embedding=4096, q_heads=16, kv_heads=4, head_dim=256, ffn=12288, rope_dim=64,
                   rope_sections=[11, 11, 10, 0], rope_base=1e7, eps=1e-6),
              dict(q=12, k=12, v=12, out=12, gate=12, up=12, down=12), 4000),
    # mixed storage types: the unfused projection path
    "mixed": (dict(embedding=512, q_heads=4, kv_heads=2, head_dim=128, ffn=1024, rope_dim=32,
                   rope_sections=[6, 5, 5, 0], rope_base=1e6, eps=1e-6),
              dict(q=13, k=8, v=0, out=14, gate=13, up=1, down=8), 37),
    # from an empty cache (the first step's only token is the new one), 8 query heads per KV head,
    # rotation over the whole head
    "empty_rep8": (dict(embedding=512, q_heads=8, kv_heads=1, head_dim=128, ffn=1024, rope_dim=128,
                        rope_sections=[22, 21, 21, 0], rope_base=1e6, eps=1e-6),
                   dict(q=12, k=12, v=12, out=14, gate=12, up=12, down=12), 0),
    # one query head per KV head, heads of 64 rotated whole, 16-token chunks: the first step's
    # new token closes a full chunk, the next two open one
    "rep1_d64": (dict(embedding=256, q_heads=4, kv_heads=4, head_dim=64, ffn=512, rope_dim=64,
                      rope_sections=[11, 11, 10, 0], rope_base=1e4, eps=1e-6),
                 dict(q=12, k=12, v=12, out=12, gate=12, up=12, down=14), 47),
    # 32 query heads over 2 KV heads of 256 (two subgroups of 8 per KV head)
    "rep16": (dict(embedding=1024, q_heads=32, kv_heads=2, head_dim=256, ffn=1024, rope_dim=64,
                   rope_sections=[11, 11, 10, 0], rope_base=1e7, eps=1e-6),
              dict(q=12, k=12, v=12, out=14, gate=12, up=12, down=12), 500),
    # long activation rows: the streamed q / k / v projection walks each row in two units (8192)
    # or three with a partial last one (8448 = 33 super-blocks)
    "e8192": (dict(embedding=8192, q_heads=4, kv_heads=2, head_dim=64, ffn=512, rope_dim=64,
                   rope_sections=[11, 11, 10, 0], rope_base=1e6, eps=1e-6),
              dict(q=12, k=12, v=12, out=12, gate=12, up=12, down=12), 20),
    "e8448": (dict(embedding=8448, q_heads=4, kv_heads=2, head_dim=64, ffn=512, rope_dim=64,
                   rope_sections=[11, 11, 10, 0], rope_base=1e6, eps=1e-6),
              dict(q=12, k=12, v=12, out=14, gate=12, up=12, down=12), 20),
}


@pytest.mark.parametrize("name", list(BLOCKS))
def test_attention_block_stages(ctx, name):
    from golden.make_golden import attention_inputs
    d, types, cached = BLOCKS[name]
    print(f"attention block {name} cached={cached}", flush=True)
    w, vec, c, xs = attention_inputs(np.random.default_rng(4242), d, types, cached=cached)
    positions = [(cached + i, cached + i, cached + i) for i in range(2)] + [(cached + 2, 7, 19)]
    steps = run_block(ctx, d, w, vec, c, positions, xs)
    own = c.copy()
    for st in steps:
        check_block_stages(d, w, vec, st)
        y, _ = oracle.attention_block_step(d, w, vec, own, st["pos"], st["x"], threads=THREADS)
        assert float(np.max(np.abs(st["y"] - y))) <= CHAIN_TOL * float(np.max(np.abs(y)))


@pytest.mark.parametrize("name", ["e2048", "rep1_d64", "rep16"])
def test_attention_block_f16_cache(ctx, name):
    """The block over an F16 cache: every stage as over an F32 cache, the attention against the
    oracle over the stored (rounded) rows, the appended key and value rounded to nearest even."""
    from golden.make_golden import attention_inputs
    d, types, cached = BLOCKS[name]
    w, vec, c, xs = attention_inputs(np.random.default_rng(4343), d, types, cached=cached)
    positions = [(cached + i, cached + i, cached + i) for i in range(2)] + [(cached + 2, 7, 19)]
    steps = run_block(ctx, d, w, vec, c, positions, xs, dtype="f16")
    for st in steps:
        check_block_stages(d, w, vec, st)
        # the loaded rows, rounded on the device as numpy rounds them
        assert np.array_equal(st["keys0"][:cached], f16(c.keys[:cached]))
        assert np.array_equal(st["values0"][:cached], f16(c.values[:cached]))


@pytest.mark.parametrize("name", ["e2048", "rep1_d64"])
def test_attention_block_trace_does_not_change_results(ctx, name):
    """Without a trace the block skips the stores only the trace reads (qcur / kcur, the pre-gate
    output, sigmoid(gate), the raw residual and gate/up rows): y and the cache must be the same
    bits."""
    from golden.make_golden import attention_inputs
    d, types, cached = BLOCKS[name]
    w, vec, c, xs = attention_inputs(np.random.default_rng(77), d, types, cached=cached)
    hkv, D = d["kv_heads"], d["head_dim"]
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    caches, bufs = [], []
    try:
        tb = ctx.alloc(sum(oracle.attention_trace_sizes(d).values()) * 4)
        bufs.append(tb)
        runs = []
        for traced in (True, False):
            cache = ctx.kv_cache(c.capacity, hkv, D, D)
            caches.append(cache)
            cache.load(c.keys, c.values, c.length)
            yb = ctx.alloc(d["embedding"] * 4)
            bufs.append(yb)
            ys = []
            for i, x in enumerate(xs[:2]):
                xb = ctx.to_device(x)
                pos = (cached + i, cached + i, cached + i)
                if traced:
                    ctx.attention_block_step(blk, cache, pos, xb, yb, tb)
                else:
                    ctx.attention_block_step(blk, cache, pos, xb, yb)
                ctx.sync()
                ys.append(yb.download(np.float32, d["embedding"]))
                xb.free()
            runs.append((ys, *cache.download(hkv, D, D)))
        (y_t, k_t, v_t), (y_n, k_n, v_n) = runs
        for a, b in zip(y_t, y_n):
            assert np.array_equal(a, b)
        assert np.array_equal(k_t, k_n) and np.array_equal(v_t, v_n)
    finally:
        for b in bufs:
            b.free()
        for cache in caches:
            cache.release()
        blk.release()


def test_attention_block_errors(ctx):
    from golden.make_golden import ATTN_KQ_DIMS, ATTN_KQ_TYPES, attention_inputs
    d = dict(ATTN_KQ_DIMS)
    w, vec, c, xs = attention_inputs(np.random.default_rng(5), d, ATTN_KQ_TYPES)
    blk = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    wrong = ctx.kv_cache(4, 2, 64, 64)
    full = ctx.kv_cache(1, 1, 64, 64)
    xb, yb = ctx.to_device(xs[0]), ctx.alloc(d["embedding"] * 4)
    try:
        with pytest.raises(oracle_amd.InvalidArgument, match="cache dimensions do not match the manifest"):
            ctx.attention_block_step(blk, wrong, (0, 0, 0), xb, yb)
        full.load(np.zeros((1, 1, 64), np.float32), np.zeros((1, 1, 64), np.float32), 1)
        with pytest.raises(oracle_amd.Overflow, match="KV cache capacity exceeded"):
            ctx.attention_block_step(blk, full, (0, 0, 0), xb, yb)
        blk.desc.rope_sections[0] = 7
        with pytest.raises(oracle_amd.InvalidArgument, match="sum to half the rotary dimension"):
            ctx.attention_block_step(blk, full, (0, 0, 0), xb, yb)
        assert len(full) == 1
    finally:
        xb.free()
        yb.free()
        wrong.release()
        full.release()
        blk.release()


def test_attention_steps_refused_under_capture(ctx):
    """The KV cache's length advances on the host when a step is issued, so a captured step would
    replay over a stale length: both attention entry points refuse a capture, and the cache is
    left as it was."""
    cache = ctx.kv_cache(4, 1, 64, 64)
    q, k, v = (ctx.to_device(np.ones((1, 64), np.float32)) for _ in range(3))
    o = ctx.alloc(64 * 4)
    heads = ctx.to_device(np.ones((1, 64), np.float32))
    try:
        ctx.capture_begin()
        try:
            ctx.rope(heads, 1, 64, 64, (32, 0, 0, 0), 10000.0, (1, 1, 1))
            with pytest.raises(oracle_amd.InvalidArgument, match="cannot be captured"):
                ctx.attention_step(q, 1, k, v, cache, o)
        finally:
            g = ctx.capture_end()
        g.destroy()
        assert len(cache) == 0
        ctx.attention_step(q, 1, k, v, cache, o)
        ctx.sync()
        assert len(cache) == 1
        assert np.array_equal(o.download(np.float32, 64), np.ones(64, np.float32))
    finally:
        for b in (q, k, v, o, heads):
            b.free()
        cache.release()


def test_attention_cache_of_another_context(ctx):
    """A cache is ordered by its own context's stream (reset, load): another context's step is
    refused."""
    other = oracle_amd.Context(0)
    q, k, v = (ctx.to_device(np.ones((1, 64), np.float32)) for _ in range(3))
    o = ctx.alloc(64 * 4)
    try:
        cache = other.kv_cache(4, 1, 64, 64)
        try:
            with pytest.raises(oracle_amd.InvalidArgument, match="belongs to another context"):
                ctx.attention_step(q, 1, k, v, cache, o)
            assert len(cache) == 0
        finally:
            cache.release()
    finally:
        for b in (q, k, v, o):
            b.free()
        other.close()


def test_caller_stream_capture_is_refused(ctx):
    """A caller capturing the context's stream with its own hipStreamBeginCapture is seen too:
    uploads, KV cache creation and attention steps refuse it, as under oq_capture_begin."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    stream = C.c_void_p(ctx.lib.oq_context_stream(ctx.h))
    cache = ctx.kv_cache(4, 1, 64, 64)
    q, k, v = (ctx.to_device(np.ones((1, 64), np.float32)) for _ in range(3))
    o = ctx.alloc(64 * 4)
    data = synth.q4_k(np.random.default_rng(3), 4, 256)
    try:
        assert hip.hipStreamBeginCapture(stream, 2) == 0  # hipStreamCaptureModeRelaxed
        try:
            with pytest.raises(oracle_amd.InvalidArgument, match="during graph capture"):
                ctx.upload(12, 256, 4, data)
            with pytest.raises(oracle_amd.InvalidArgument, match="during graph capture"):
                ctx.kv_cache(4, 1, 64, 64)
            with pytest.raises(oracle_amd.InvalidArgument, match="cannot be captured"):
                ctx.attention_step(q, 1, k, v, cache, o)
        finally:
            graph = C.c_void_p()
            assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
            if graph.value:
                hip.hipGraphDestroy(graph)
        w = ctx.upload(12, 256, 4, data)  # eager again
        w.release()
        assert len(cache) == 0
    finally:
        for b in (q, k, v, o):
            b.free()
        cache.release()
