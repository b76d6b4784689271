"""Pins of the oracle's full-attention restatement (oracle/oracle.c), CPU only.

- the reference's own known answers for RoPE / MRoPE and for the KV cache with attention
  (reference tests/test_phase1e.cpp:92-186) and for the attention block
  (tests/test_phase2c.cpp:182-213, :284-310);
- bit-for-bit equality with the reference's compiled apply_qwen35_rope and
  causal_attention_step (reference_kernels.cpp:77-195) on seeded inputs through the committed
  fixtures (tests/golden/ref_attention.npz) and, where oracle/_ref is built, live;
- the whole attention block (qwen35_block.cpp:607-756): bit-for-bit equality with the
  reference's execute_qwen35_attention_block_reference over three steps after five cached
  tokens, one of them at a multimodal position; K-quant projections through the reference's
  matvec override bridge with the oracle's own projection outputs;
- what the mathematics fixes: rotations keep each pair's norm, position 0 is the identity, one
  cached token returns its value, equal keys average the values, query head h reads KV head
  h / (q_heads / kv_heads).
"""
import math

import numpy as np
import pytest

import oracle

GOLDEN_ATTN = "ref_attention.npz"
LIVE = pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference (oracle/_ref) not built here")


@pytest.fixture(scope="module")
def attn_golden():
    from conftest import GOLDEN
    with np.load(GOLDEN / GOLDEN_ATTN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------- RoPE

def test_rope_known_answers(kat):
    r = kat["rope"]
    out = oracle.rope(np.array([r["head"]], np.float32), r["rotary_dim"], r["sections"], r["base"], r["position"])[0]
    c, s = math.cos(1.0), math.sin(1.0)
    x = r["head"]
    expected = [x[0] * c - x[2] * s, x[1] * c - x[3] * s, x[2] * c + x[0] * s, x[3] * c + x[1] * s]
    assert np.allclose(out, expected, atol=r["tol"], rtol=0)
    assert abs(float(np.sum(out.astype(np.float64) ** 2)) - r["norm"]) <= 1e-5
    m = kat["mrope"]
    out = oracle.rope(np.array([m["head"]], np.float32), m["rotary_dim"], m["sections"], m["base"], m["position"])[0]
    expected = [math.cos(1), math.cos(2), math.cos(3), math.sin(1), math.sin(2), math.sin(3)]
    assert np.allclose(out, expected, atol=m["tol"], rtol=0)


def test_rope_matches_reference_fixtures(attn_golden):
    g = attn_golden
    for name in ("text", "mm", "far"):
        out = oracle.rope(g["rope_in"], 64, [11, 11, 10, 0], 1e7, tuple(int(v) for v in g[f"rope_{name}_pos"]))
        assert np.array_equal(out.view(np.uint32), g[f"rope_{name}_bits"]), name


def test_rope_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    # position 0: every angle is 0, cos 1 and sin 0 -- the identity, bit for bit
    assert np.array_equal(oracle.rope(x, 64, [11, 11, 10, 0], 1e7, (0, 0, 0)), x)
    # each rotated pair keeps its norm; dimensions past the rotary width are untouched
    y = oracle.rope(x, 64, [11, 11, 10, 0], 1e7, (1234, 99, 7))
    n0 = x[:, :32].astype(np.float64) ** 2 + x[:, 32:64].astype(np.float64) ** 2
    n1 = y[:, :32].astype(np.float64) ** 2 + y[:, 32:64].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-6, atol=1e-6)
    assert np.array_equal(y[:, 64:], x[:, 64:])
    # frequency 0 turns by the temporal coordinate itself (inverse frequency 1)
    e = np.zeros((1, 128), np.float32)
    e[0, 0] = 1.0
    z = oracle.rope(e, 64, [11, 11, 10, 0], 1e7, (3, 0, 0))
    assert z[0, 0] == np.float32(math.cos(3.0)) and z[0, 32] == np.float32(math.sin(3.0))


@pytest.mark.parametrize("args,message", [
    ((0, [0, 0, 0, 0]), "RoPE dimension must be non-zero, even, and within head width"),
    ((3, [1, 0, 0, 0]), "RoPE dimension must be non-zero, even, and within head width"),
    ((10, [5, 0, 0, 0]), "RoPE dimension must be non-zero, even, and within head width"),
    ((4, [-1, 3, 0, 0]), "RoPE dimension sections must be non-negative"),
    ((4, [1, 0, 0, 0]), "RoPE dimension sections must sum to half the rotary dimension"),
])
def test_rope_errors(args, message):
    rd, sec = args
    with pytest.raises(oracle.OracleError, match=message):
        oracle.rope(np.zeros((1, 8), np.float32), rd, sec, 1.0, (1, 1, 1))
    with pytest.raises(oracle.OracleError, match="RoPE frequency base must be positive and finite"):
        oracle.rope(np.zeros((1, 8), np.float32), 4, [2, 0, 0, 0], float("inf"), (1, 1, 1))
    if oracle.ref_available():
        with pytest.raises(oracle.OracleError, match=message):
            oracle.rope(np.zeros((1, 8), np.float32), rd, sec, 1.0, (1, 1, 1), reference=True)


@LIVE
def test_rope_matches_live_reference():
    rng = np.random.default_rng(77)
    x = rng.standard_normal((6, 256)).astype(np.float32)
    for pos in ((0, 0, 0), (1, 1, 1), (4095, 17, 3), (2 ** 40, 5, 2 ** 20)):
        for rd, sec in ((64, [11, 11, 10, 0]), (256, [40, 40, 40, 8]), (2, [1, 0, 0, 0])):
            a = oracle.rope(x, rd, sec, 1e7, pos)
            b = oracle.rope(x, rd, sec, 1e7, pos, reference=True)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (pos, rd)


# ---------------------------------------------------------------- attention step

def test_attention_known_answers(kat):
    a = kat["attention"]
    cache = oracle.KvCache(a["capacity"], a["kv_heads"], a["key_dim"], a["value_dim"])
    s0, s1 = a["steps"]
    out = oracle.attention_step(np.reshape(s0["q"], (2, 2)), np.reshape(s0["k"], (1, 2)),
                                np.reshape(s0["v"], (1, 2)), cache)
    assert cache.length == 1
    assert np.allclose(out.ravel(), s0["expected"], atol=a["tol"], rtol=0)
    out = oracle.attention_step(np.reshape(s1["q"], (2, 2)), np.reshape(s1["k"], (1, 2)),
                                np.reshape(s1["v"], (1, 2)), cache)
    e = math.exp(1.0 / math.sqrt(2.0))
    p_new = e / (1.0 + e)
    p_old = 1.0 - p_new
    assert abs(out[0, 0] - (p_old * 2 + p_new * 4)) <= a["tol"]
    assert abs(out[0, 1] - (p_old * 3 + p_new * 5)) <= a["tol"]
    with pytest.raises(oracle.OracleError, match="KV cache capacity exceeded"):
        oracle.attention_step(np.reshape(s1["q"], (2, 2)), np.reshape(s1["k"], (1, 2)), np.reshape(s1["v"], (1, 2)),
                              cache)
    assert cache.length == 2


def test_attention_matches_reference_fixture(attn_golden):
    g = attn_golden
    cache = oracle.KvCache(16, 2, 256, 256)
    for i in range(g["attn_q"].shape[0]):
        out = oracle.attention_step(g["attn_q"][i], g["attn_k"][i], g["attn_v"][i], cache)
        assert np.array_equal(out.view(np.uint32), g["attn_y_bits"][i]), f"step {i}"


def test_attention_invariants():
    rng = np.random.default_rng(6)
    # one token: every query head returns its KV head's value
    cache = oracle.KvCache(8, 2, 16, 24)
    k = rng.standard_normal((2, 16)).astype(np.float32)
    v = rng.standard_normal((2, 24)).astype(np.float32)
    out = oracle.attention_step(rng.standard_normal((6, 16)).astype(np.float32), k, v, cache)
    assert np.array_equal(out, v[[0, 0, 0, 1, 1, 1]])  # heads 0-2 read KV head 0, heads 3-5 KV head 1
    # equal keys: the average of the values
    cache = oracle.KvCache(8, 1, 16, 8)
    k = rng.standard_normal((1, 16)).astype(np.float32)
    vs = [rng.standard_normal((1, 8)).astype(np.float32) for _ in range(4)]
    for v in vs:
        out = oracle.attention_step(rng.standard_normal((2, 16)).astype(np.float32), k, v, cache)
    assert np.allclose(out[0], np.mean(np.concatenate(vs), axis=0), rtol=1e-6, atol=1e-6)
    # the softmax against a float64 evaluation
    cache = oracle.KvCache(40, 2, 32, 32)
    for _ in range(33):
        q = rng.standard_normal((4, 32)).astype(np.float32)
        out = oracle.attention_step(q, rng.standard_normal((2, 32)).astype(np.float32),
                                    rng.standard_normal((2, 32)).astype(np.float32), cache)
    K = cache.keys[:33].astype(np.float64)
    V = cache.values[:33].astype(np.float64)
    for h in range(4):
        s = K[:, h // 2] @ q[h].astype(np.float64) / math.sqrt(32)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ V[:, h // 2]
        assert np.allclose(out[h], ref, rtol=0, atol=1e-5 * np.abs(V[:, h // 2]).max())


def test_attention_dimension_errors():
    cache = oracle.KvCache(4, 2, 8, 8)
    with pytest.raises(oracle.OracleError, match="causal_attention_step dimensions are incompatible"):
        oracle.attention_step(np.zeros((3, 8), np.float32), np.zeros((2, 8), np.float32),
                              np.zeros((2, 8), np.float32), cache)
    assert cache.length == 0


@LIVE
def test_attention_matches_live_reference():
    rng = np.random.default_rng(78)
    for hq, hkv, dk, dv in ((8, 2, 256, 256), (16, 4, 128, 64), (3, 3, 64, 128)):
        c1 = oracle.KvCache(70, hkv, dk, dv)
        c2 = oracle.KvCache(70, hkv, dk, dv)
        for t in range(70):
            q = (3 * rng.standard_normal((hq, dk))).astype(np.float32)
            k = rng.standard_normal((hkv, dk)).astype(np.float32)
            v = rng.standard_normal((hkv, dv)).astype(np.float32)
            a = oracle.attention_step(q, k, v, c1)
            b = oracle.attention_step(q, k, v, c2, reference=True)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (hq, hkv, t)
        assert np.array_equal(c1.keys, c2.keys) and np.array_equal(c1.values, c2.values)


# ---------------------------------------------------------------- attention block

def _attn_case(g, case):
    from golden.make_golden import ATTN_KQ_DIMS, ATTN_PLAIN_DIMS
    dims = ATTN_PLAIN_DIMS if case == "plain" else ATTN_KQ_DIMS
    w = {n: (int(g[f"{case}_t_{n}"][0]), g[f"{case}_w_{n}"]) for n in oracle.ATTN_WEIGHTS}
    vec = {n: g[f"{case}_v_{n}"] for n in oracle.ATTN_VECTORS}
    cache = oracle.KvCache(*g[f"{case}_keys0"].shape, g[f"{case}_values0"].shape[2])
    cache.keys[:] = g[f"{case}_keys0"]
    cache.values[:] = g[f"{case}_values0"]
    cache.length = int(g[f"{case}_length0"][0])
    return dims, w, vec, cache


PROJ = {"q": "qfull", "k": "k", "v": "v", "out": "branch", "gate": "gate", "up": "up", "down": "ffn"}


@pytest.mark.parametrize("case", ["plain", "kq"])
def test_attention_block_matches_reference_fixtures(attn_golden, case):
    from golden.make_golden import ATTN_POSITIONS
    g = attn_golden
    dims, w, vec, cache = _attn_case(g, case)
    for i, x in enumerate(g[f"{case}_x"]):
        y, tr = oracle.attention_block_step(dims, w, vec, cache, ATTN_POSITIONS[i], x, threads=2)
        assert np.array_equal(y.view(np.uint32), g[f"{case}_y_bits"][i]), f"step {i}: y"
        flat = np.concatenate([tr[n] for n in oracle.ATTN_TRACE])
        assert np.array_equal(flat.view(np.uint32), g[f"{case}_trace_bits"][i]), f"step {i}: trace"
        if case == "kq":
            proj = np.concatenate([tr[PROJ[n]] for n in oracle.ATTN_WEIGHTS])
            assert np.array_equal(proj.view(np.uint32), g[f"{case}_proj_bits"][i])
    assert np.array_equal(cache.keys.view(np.uint32), g[f"{case}_keys_bits"])
    assert np.array_equal(cache.values.view(np.uint32), g[f"{case}_values_bits"])


def test_attention_block_known_answers(kat):
    b = kat["attention_block"]
    d = b["dims"]
    E, Hq, D, F = d["embedding"], d["q_heads"], d["head_dim"], d["ffn"]

    def mat(rows, cols, ones):
        m = np.zeros((rows, cols), np.float32)
        for r, c in ones:
            m[r, c] = 1.0
        return (0, m.ravel().view(np.uint8))

    w = {"q": mat(2 * Hq * D, E, b["q_ones"]), "k": mat(d["kv_heads"] * D, E, b["k_ones"]),
         "v": mat(d["kv_heads"] * D, E, b["v_ones"]), "out": (0, np.eye(E, dtype=np.float32).ravel().view(np.uint8)),
         "gate": mat(F, E, []), "up": mat(F, E, []), "down": mat(E, F, [])}
    vec = {"input_norm": np.ones(E, np.float32), "q_norm": np.ones(D, np.float32), "k_norm": np.ones(D, np.float32),
           "post_norm": np.ones(E, np.float32)}
    x = np.array(b["input"], np.float32)
    inv = 1.0 / math.sqrt(7.5 + d["eps"])
    expected = [x[i] + 0.5 * x[2 + i % 2] * inv for i in range(E)]
    runs = [("oracle", oracle.attention_block_step)]
    if oracle.ref_available():
        runs.append(("reference", oracle.ref_attention_block))
    for name, fn in runs:
        cache = oracle.KvCache(4, d["kv_heads"], D, D)
        y, tr = fn(d, w, vec, cache, (0, 0, 0), x)
        assert np.allclose(y, expected, atol=b["tol"], rtol=0), name
        assert cache.length == b["cache_after"]
        assert np.allclose(tr["gate_s"], 0.5) and tr["gated"].shape == (Hq * D,)


@LIVE
@pytest.mark.parametrize("types", [
    dict(q=0, k=0, v=0, out=0, gate=0, up=0, down=0),
    dict(q=8, k=30, v=1, out=8, gate=1, up=30, down=8),
    dict(q=12, k=13, v=14, out=12, gate=14, up=12, down=13),
], ids=["f32", "mixed", "kquant_overrides"])
def test_attention_block_matches_live_reference(types):
    from golden.make_golden import attention_inputs
    dims = dict(embedding=256, q_heads=8, kv_heads=2, head_dim=64, ffn=512, rope_dim=32,
                rope_sections=[6, 5, 5, 0], rope_base=1e7, eps=1e-6)
    w, vec, cache, xs = attention_inputs(np.random.default_rng(101), dims, types, cached=9)
    kq = any(t in (12, 13, 14) for t in types.values())
    c2 = cache.copy()
    for i, x in enumerate(xs):
        pos = (9 + i, 9 + i, 9 + i) if i < 2 else (40, 2, 3)
        y, tr = oracle.attention_block_step(dims, w, vec, cache, pos, x, threads=2)
        ov = {n: tr[PROJ[n]] for n in oracle.ATTN_WEIGHTS} if kq else None
        y_r, tr_r = oracle.ref_attention_block(dims, w, vec, c2, pos, x, overrides=ov)
        assert np.array_equal(y.view(np.uint32), y_r.view(np.uint32))
        for n in oracle.ATTN_TRACE:
            assert np.array_equal(tr[n].view(np.uint32), tr_r[n].view(np.uint32)), n
    assert np.array_equal(cache.keys, c2.keys) and np.array_equal(cache.values, c2.values)
