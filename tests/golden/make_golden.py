"""Write the golden vectors under tests/golden/.

1. ref_kat.json -- the reference's own known-answer fixtures for the quantized path
   (tests/test_phase2a.cpp:50-106,132-289 of the reference): block recipes and the values the
   reference asserts for them.  They are restated here as data (bytes in hex, expected floats).
2. ref_random.npz -- seeded random rows run through the reference's own decoder and matvec,
   compiled from its sources into oracle/_ref/libref.so (oracle/Makefile).  Q4_K has no
   reference decoder; its vectors are the reference's Q5_K results on the same blocks with an
   all-zero fifth-bit plane, which GGML's Q4_K format must reproduce exactly.

3. ref_deltanet.npz -- seeded random inputs run through the reference's own causal depthwise
   convolution step and gated delta rule step (src/runtime/reference_kernels.cpp:197-335,
   compiled into the same library), several steps in a row with the state carried.

4. ref_block.npz -- seeded Gated DeltaNet decode blocks run through the reference's own
   execute_qwen35_recurrent_block_reference (src/runtime/qwen35_block.cpp:406-605) on in-memory
   tensor views, as the reference's block test drives it (tests/test_phase2c.cpp:72-213), three
   steps with the state and convolution history carried:
   - "plain": projections stored as F32, F16, BF16 and Q8_0 (the reference multiplies them with
     the F32 activation, as the oracle does), no overrides;
   - "kq": q4_K projections with a q6_K output projection; the reference's matvec override
     bridge (Qwen35MatvecOverrides) takes the oracle's projection outputs, so every other stage
     is the reference's own arithmetic.

Run from the repository root after `make -C oracle all ref`:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402
from oracle_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def u16le(v: int) -> list[int]:
    return [v & 0xFF, v >> 8]


def kat() -> dict:
    # Q5_K: d = 0.5 (0x3800), dmin = 0.25 (0x3400), scales bytes {2,2,2,2,3,3,3,3,0x32 x4},
    # qh = 0xFF x32, qs = 0x21 x128 -> 16.25 (low nibbles) / 17.25 (high nibbles)
    q5 = u16le(0x3800) + u16le(0x3400) + [2, 2, 2, 2, 3, 3, 3, 3, 0x32, 0x32, 0x32, 0x32] + [0xFF] * 32 + [0x21] * 128
    q5_second = q5[:16] + [0] * 160  # qh and qs cleared -> every element -0.75
    # Q6_K: ql = 0x21 x128, qh = 0xFF x64, sc = 2 x16, d = 0.5 -> 17 (lower 64) / 18 (upper 64)
    q6 = [0x21] * 128 + [0xFF] * 64 + [0x02] * 16 + u16le(0x3800)
    q8_quants = [0, 1, -1, 127, -128, 2, -2, 3, -3, 4, -4, 5, -5, 6, -6, 7,
                 -7, 8, -8, 9, -9, 10, -10, 11, -11, 12, -12, 13, -13, 14, -14, 15]
    q8 = u16le(0x3C00) + [q & 0xFF for q in q8_quants]
    q8_second = u16le(0x3800) + [10] * 32
    q8_second_row = u16le(0x3800) + [4] * 32
    hexs = lambda b: bytes(b).hex()  # noqa: E731
    return {
        "source": "reference tests/test_phase2a.cpp (known-answer fixtures of the quantized path)",
        "f16": [[0x3C00, 1.0], [0xC000, -2.0], [0x0001, 2.0 ** -24]],
        "f16_special": {"inf": 0x7C00, "nan": 0x7E00, "neg_zero": 0x8000},
        "bf16": [[0x3F80, 1.0], [0xC000, -2.0]],
        "f16_row": {"bits": [0x3C00, 0xC000, 0x4200, 0x0000], "expected": [1.0, -2.0, 3.0, 0.0]},
        "bf16_row": {"bits": [0x3F80, 0xC000, 0x4040, 0x0000], "expected": [1.0, -2.0, 3.0, 0.0]},
        "q5_k": {"block": hexs(q5), "low": 16.25, "high": 17.25, "dot_ones": 4288.0,
                 "dot_ones_two_blocks": 8576.0},
        "q5_k_matvec": {"rows": [hexs(q5), hexs(q5_second)], "expected": [4288.0, -192.0]},
        "q6_k": {"block": hexs(q6), "lower": 17.0, "upper": 18.0, "dot_ones": 4480.0},
        "q8_0": {"block": hexs(q8), "expected": q8_quants, "dot_ones": 14.0},
        "q8_0_two_blocks": {"blocks": hexs(q8 + q8_second), "at3": 127.0, "at32": 5.0, "at63": 5.0},
        "q8_0_matvec": {"rows": [hexs(q8), hexs(q8_second_row)], "expected": [14.0, 64.0]},
        # reference tests/test_phase1e.cpp:188-245 and tests/test_phase2c.cpp:265-285
        "ssm": {"conv": {"taps": [1.0, 2.0, 3.0], "inputs": [1.0, 2.0], "expected": [3.0, 8.0]},
                "delta": {"q": [1.0, 0.0], "k": [1.0, 0.0], "v": [2.0],
                          "steps": [{"beta": 0.5, "log_decay": 0.0, "expected": 0.7071067811865476, "tol": 2e-6},
                                    {"beta": 1.0, "log_decay_of": 0.5, "expected": 1.4142135623730951, "tol": 3e-6}],
                          "eps": 1e-12},
                "delta_eps": {"q": [1e-4, 0.0], "k": [1e-4, 0.0], "v": [2.0], "beta": 1.0, "log_decay": 0.0,
                              "eps": 1e-6, "expected": 1.4142135623730951, "tol": 2e-6}},
        # reference tests/test_phase2c.cpp: manifest :49-71, recurrent block weights :146-181 (all
        # F32; unlisted matrices are zero), assertions :215-260
        "block": {"dims": {"embedding": 4, "key_heads": 2, "value_heads": 4, "key_dim": 1, "value_dim": 1,
                           "conv_kernel": 2, "ffn": 4, "eps": 1e-6},
                  "input": [1.0, -2.0, 3.0, 4.0],
                  "qkv_ones": [[0, 0], [1, 1], [2, 0], [3, 1], [4, 0], [5, 1], [6, 2], [7, 3]],
                  "conv_tap_one": 1, "dt_bias": [0.0, 0.0, 0.0, 0.0], "decay": [-1.0, -1.0, -1.0, -1.0],
                  "out": "identity", "norms": "ones",
                  "expect": {"output_equals_input": True, "beta_sigmoid0": 0.5, "gate0": -0.6931471805599453,
                             "tol": 1e-6, "q_predelta_signs": [1, -1, 1, -1], "state_before_zero": True,
                             "state_after_nonzero": True}},
        # reference tests/test_phase1e.cpp:92-142 (RoPE, MRoPE) and :144-186 (KV cache + attention)
        "rope": {"head": [1.0, 2.0, 3.0, 4.0], "position": [1, 1, 1], "rotary_dim": 4, "sections": [2, 0, 0, 0],
                 "base": 1.0, "expected_of": "1cos1-3sin1, 2cos1-4sin1, 3cos1+1sin1, 4cos1+2sin1",
                 "norm": 30.0, "tol": 1e-6},
        "mrope": {"head": [1.0, 1.0, 1.0, 0.0, 0.0, 0.0], "position": [1, 2, 3], "rotary_dim": 6,
                  "sections": [1, 1, 1, 0], "base": 1.0,
                  "expected_of": "cos1 cos2 cos3 sin1 sin2 sin3", "tol": 1e-6},
        "attention": {"capacity": 2, "kv_heads": 1, "key_dim": 2, "value_dim": 2, "q_heads": 2,
                      "steps": [{"q": [1.0, 0.0, 1.0, 0.0], "k": [1.0, 0.0], "v": [2.0, 3.0],
                                 "expected": [2.0, 3.0, 2.0, 3.0]},
                                {"q": [0.0, 1.0, 0.0, 1.0], "k": [0.0, 1.0], "v": [4.0, 5.0],
                                 "expected_of": "p_new = e^(1/sqrt2) / (1 + e^(1/sqrt2)); p_old 2 + p_new 4, "
                                                "p_old 3 + p_new 5"}],
                      "tol": 1e-6, "third_step": "overflow"},
        # reference tests/test_phase2c.cpp: manifest :44-71, attention block weights :182-213 (all
        # F32, MLP zero), assertions :284-310
        "attention_block": {"dims": {"embedding": 4, "q_heads": 2, "kv_heads": 1, "head_dim": 2, "ffn": 4,
                                     "rope_dim": 2, "rope_sections": [1, 0, 0, 0], "rope_base": 10000.0,
                                     "eps": 1e-6},
                            "input": [1.0, 2.0, 3.0, 4.0],
                            "q_ones": [[0, 0], [1, 1], [4, 2], [5, 3]], "k_ones": [[0, 0], [1, 1]],
                            "v_ones": [[0, 2], [1, 3]], "out": "identity", "norms": "ones",
                            "expected_of": "x[i] + 0.5 * x[2 + i % 2] / sqrt(7.5 + eps)", "tol": 1e-5,
                            "cache_after": 1},
    }


def random_vectors() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}
    rows, cols = 4, 512
    cases = {
        "q5_k": (13, synth.q5_k(rng, rows, cols)),
        "q6_k": (14, synth.q6_k(rng, rows, cols)),
        "q8_0": (8, synth.q8_0(rng, rows, cols)),
        # raw random bytes with finite, moderate scales: every quant bit pattern is reachable
        "q5_k_raw": (13, None),
        "q6_k_raw": (14, None),
        "q8_0_raw": (8, None),
    }
    for name, (t, data) in list(cases.items()):
        if data is None:
            rb = synth.row_bytes(t, cols)
            data = np.frombuffer(rng.bytes(rows * rb), dtype=np.uint8).copy()
            blk = {13: 176, 14: 210, 8: 34}[t]
            view = data.reshape(-1, blk)
            dpos = {13: [0, 2], 14: [208], 8: [0]}[t]
            for p in dpos:  # finite f16 scales in [2^-15, 2^-1), sign random
                e = rng.integers(0, 15, view.shape[0]).astype(np.uint16)
                bits = (rng.integers(0, 2, view.shape[0]).astype(np.uint16) << 15) | (e << 10) | \
                    rng.integers(0, 1024, view.shape[0]).astype(np.uint16)
                view[:, p:p + 2] = bits.astype("<u2").view(np.uint8).reshape(-1, 2)
        cases[name] = (t, data)
    x = rng.standard_normal(cols, dtype=np.float32)
    out["x"] = x
    for name, (t, data) in cases.items():
        dec = np.stack([oracle.ref_decode_row(t, cols, data.reshape(rows, -1)[r]) for r in range(rows)])
        y = oracle.ref_storage_matvec(t, rows, cols, data, x)
        out[f"{name}_type"] = np.array([t])
        out[f"{name}_bytes"] = data
        out[f"{name}_decoded_bits"] = dec.view(np.uint32)
        out[f"{name}_matvec_bits"] = y.view(np.uint32)
    # Q4_K via the Q5_K decoder with qh = 0 (the same 144-byte block without the qh plane)
    q5 = synth.q5_k(rng, rows, cols).reshape(-1, 176)
    q5[:, 16:48] = 0
    q5 = q5.reshape(-1)
    q4 = np.concatenate([q5.reshape(-1, 176)[:, :16], q5.reshape(-1, 176)[:, 48:]], axis=1).reshape(-1)
    out["q4_k_bytes"] = q4
    out["q4_k_decoded_bits"] = np.stack(
        [oracle.ref_decode_row(13, cols, q5.reshape(rows, -1)[r]) for r in range(rows)]).view(np.uint32)
    out["q4_k_matvec_bits"] = oracle.ref_storage_matvec(13, rows, cols, q5, x).view(np.uint32)
    # F16 / BF16 / F32 rows, all bit patterns of f16 included once
    f16_bits = np.arange(65536, dtype=np.uint16)
    out["f16_all_bits"] = f16_bits
    out["f16_all_decoded_bits"] = oracle.ref_decode_row(1, 65536, f16_bits.view(np.uint8)).view(np.uint32)
    out["bf16_sample_bits"] = rng.integers(0, 65536, 4096, dtype=np.uint16)
    out["bf16_sample_decoded_bits"] = oracle.ref_decode_row(30, 4096, out["bf16_sample_bits"].view(np.uint8)).view(np.uint32)
    return out


def deltanet_vectors() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261202)
    out: dict[str, np.ndarray] = {}
    channels, kernel, steps = 24, 4, 3
    hist = rng.standard_normal((channels, kernel)).astype(np.float32)
    taps = rng.standard_normal(channels * kernel).astype(np.float32)
    out["conv_taps"] = taps
    out["conv_history0"] = hist.copy()
    xs = rng.standard_normal((steps, channels)).astype(np.float32)
    out["conv_inputs"] = xs
    outs = [oracle.ref_conv_step(hist, taps, xs[i]) for i in range(steps)]
    out["conv_outputs_bits"] = np.stack(outs).view(np.uint32)
    out["conv_history_bits"] = hist.view(np.uint32)
    heads, dk, dv = 3, 16, 8
    state = (0.1 * rng.standard_normal((heads, dk, dv))).astype(np.float32)
    out["delta_state0"] = state.copy()
    q = rng.standard_normal((steps, heads, dk)).astype(np.float32)
    k = rng.standard_normal((steps, heads, dk)).astype(np.float32)
    v = rng.standard_normal((steps, heads, dv)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (steps, heads)).astype(np.float32)
    log_decay = (-rng.uniform(0.0, 2.0, (steps, heads))).astype(np.float32)
    for n, a in (("q", q), ("k", k), ("v", v), ("beta", beta), ("log_decay", log_decay)):
        out[f"delta_{n}"] = a
    outs = [oracle.ref_gated_delta_step(q[i], k[i], v[i], beta[i], log_decay[i], state, 1e-6) for i in range(steps)]
    out["delta_outputs_bits"] = np.stack(outs).view(np.uint32)
    out["delta_state_bits"] = state.view(np.uint32)
    return out


BLOCK_PLAIN_DIMS = dict(embedding=64, key_heads=2, value_heads=4, key_dim=8, value_dim=16, conv_kernel=4,
                        ffn=96, eps=1e-6)
BLOCK_KQ_DIMS = dict(embedding=256, key_heads=1, value_heads=2, key_dim=32, value_dim=128, conv_kernel=4,
                     ffn=256, eps=1e-6)
# storage type per projection (0 f32, 1 f16, 30 bf16, 8 q8_0, 12 q4_K, 14 q6_K)
BLOCK_PLAIN_TYPES = dict(qkv=8, z=1, beta=30, alpha=0, out=8, gate=0, up=1, down=8)
BLOCK_KQ_TYPES = dict(qkv=12, z=12, beta=12, alpha=12, out=14, gate=12, up=12, down=12)


def block_inputs(rng: np.random.Generator, dims: dict, types: dict):
    """Seeded block inputs: (weights {name: (type, bytes)}, vectors, conv history, state, xs[3])."""
    E, F = dims["embedding"], dims["ffn"]
    Hk, Hv, dk, dv, K = (dims[k] for k in ("key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel"))
    C, V = 2 * Hk * dk + Hv * dv, Hv * dv
    shapes = {"qkv": (C, E), "z": (V, E), "beta": (Hv, E), "alpha": (Hv, E), "out": (E, V), "gate": (F, E),
              "up": (F, E), "down": (E, F)}
    w = {}
    for n, (rows, cols) in shapes.items():
        t = types[n]
        if t in (12, 13, 14, 8):
            w[n] = (t, synth.weights(t, rng, rows, cols))
        else:
            vals = (0.05 * rng.standard_normal(rows * cols)).astype(np.float32)
            if t == 0:
                data = vals.view(np.uint8)
            elif t == 1:
                data = vals.astype(np.float16).view(np.uint8)
            else:  # bf16: the upper half of the F32 pattern
                data = (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
            w[n] = (t, data.copy())
    vec = {
        "input_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
        "conv_weight": (0.5 * rng.standard_normal(C * K)).astype(np.float32),
        "dt_bias": rng.standard_normal(Hv).astype(np.float32),
        "decay": (-np.exp(0.5 * rng.standard_normal(Hv))).astype(np.float32),
        "out_norm": (1.0 + 0.1 * rng.standard_normal(dv)).astype(np.float32),
        "post_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
    }
    hist = rng.standard_normal((C, K)).astype(np.float32)
    state = (0.01 * rng.standard_normal((Hv, dk, dv))).astype(np.float32)
    xs = rng.standard_normal((3, E)).astype(np.float32)
    return w, vec, hist, state, xs


def block_vectors() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for case, dims, types, seed in (("plain", BLOCK_PLAIN_DIMS, BLOCK_PLAIN_TYPES, 20261203),
                                    ("kq", BLOCK_KQ_DIMS, BLOCK_KQ_TYPES, 20261204)):
        w, vec, hist, state, xs = block_inputs(np.random.default_rng(seed), dims, types)
        for n, (t, data) in w.items():
            out[f"{case}_w_{n}"] = data
            out[f"{case}_t_{n}"] = np.array([t])
        for n, v in vec.items():
            out[f"{case}_v_{n}"] = v
        out[f"{case}_history0"] = hist.copy()
        out[f"{case}_state0"] = state.copy()
        out[f"{case}_x"] = xs
        out[f"{case}_ffn"] = np.array([dims["ffn"]])
        ys, traces, projs = [], [], []
        oh, os_ = hist.copy(), state.copy()
        for i in range(xs.shape[0]):
            overrides = None
            if case == "kq":
                # the oracle's projections of this step (its own state carried alongside)
                _, tr = oracle.deltanet_step(dims, w, vec, oh, os_, xs[i], threads=1, trace=True)
                overrides = {"qkv": tr["qkv"], "z": tr["z"], "beta": tr["beta"], "alpha": tr["alpha"],
                             "out": tr["branch"], "gate": tr["gate"], "up": tr["up"], "down": tr["ffn"]}
                projs.append(np.concatenate([overrides[n] for n in oracle.DN_WEIGHTS]))
            y, tr = oracle.ref_recurrent_block(dims, w, vec, hist, state, xs[i], overrides=overrides)
            ys.append(y)
            traces.append(np.concatenate([tr[n] for n in oracle.DN_TRACE]))
        out[f"{case}_y_bits"] = np.stack(ys).view(np.uint32)
        out[f"{case}_trace_bits"] = np.stack(traces).view(np.uint32)
        out[f"{case}_history_bits"] = hist.view(np.uint32)
        out[f"{case}_state_bits"] = state.view(np.uint32)
        if projs:
            out[f"{case}_proj_bits"] = np.stack(projs).view(np.uint32)
    return out


ATTN_PLAIN_DIMS = dict(embedding=64, q_heads=4, kv_heads=2, head_dim=32, ffn=96, rope_dim=16,
                       rope_sections=[3, 3, 2, 0], rope_base=10000.0, eps=1e-6)
ATTN_KQ_DIMS = dict(embedding=256, q_heads=4, kv_heads=1, head_dim=64, ffn=256, rope_dim=32,
                    rope_sections=[6, 5, 5, 0], rope_base=1e7, eps=1e-6)
ATTN_PLAIN_TYPES = dict(q=8, k=1, v=0, out=8, gate=0, up=1, down=8)
ATTN_KQ_TYPES = dict(q=12, k=12, v=12, out=14, gate=12, up=12, down=12)
# positions (temporal, height, width) of the three block steps after five cached tokens; the last
# one multimodal
ATTN_POSITIONS = ((5, 5, 5), (6, 6, 6), (7, 3, 11))


def _weight(rng, t, rows, cols):
    if t in (12, 13, 14, 8):
        return t, synth.weights(t, rng, rows, cols)
    vals = (0.05 * rng.standard_normal(rows * cols)).astype(np.float32)
    if t == 0:
        data = vals.view(np.uint8)
    elif t == 1:
        data = vals.astype(np.float16).view(np.uint8)
    else:
        data = (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    return t, data.copy()


def attention_inputs(rng: np.random.Generator, dims: dict, types: dict, cached: int = 5):
    """Seeded attention-block inputs: (weights, vectors, cache with `cached` tokens, xs[3])."""
    E, F, Hq, Hkv, D = (dims[k] for k in ("embedding", "ffn", "q_heads", "kv_heads", "head_dim"))
    Q, KV = Hq * D, Hkv * D
    shapes = {"q": (2 * Q, E), "k": (KV, E), "v": (KV, E), "out": (E, Q), "gate": (F, E), "up": (F, E),
              "down": (E, F)}
    w = {n: _weight(rng, types[n], r, c) for n, (r, c) in shapes.items()}
    vec = {
        "input_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
        "q_norm": (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32),
        "k_norm": (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32),
        "post_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
    }
    cache = oracle.KvCache(cached + 4, Hkv, D, D)
    cache.keys[:cached] = rng.standard_normal((cached, Hkv, D)).astype(np.float32)
    cache.values[:cached] = rng.standard_normal((cached, Hkv, D)).astype(np.float32)
    cache.length = cached
    xs = rng.standard_normal((3, E)).astype(np.float32)
    return w, vec, cache, xs


def attention_vectors() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    # RoPE and the attention step alone, 8 query heads over 2 KV heads of 256 (the 2B model's
    # attention geometry), 12 steps from an empty cache
    rng = np.random.default_rng(20261205)
    heads = rng.standard_normal((16, 256)).astype(np.float32)
    out["rope_in"] = heads
    for name, pos in (("text", (37, 37, 37)), ("mm", (37, 4, 19)), ("far", (262143, 262143, 262143))):
        out[f"rope_{name}_pos"] = np.array(pos, dtype=np.uint64)
        out[f"rope_{name}_bits"] = oracle.rope(heads, 64, [11, 11, 10, 0], 1e7, pos, reference=True).view(np.uint32)
    cache = oracle.KvCache(16, 2, 256, 256)
    qs = rng.standard_normal((12, 8, 256)).astype(np.float32)
    ks = rng.standard_normal((12, 2, 256)).astype(np.float32)
    vs = rng.standard_normal((12, 2, 256)).astype(np.float32)
    ys = [oracle.attention_step(qs[i], ks[i], vs[i], cache, reference=True) for i in range(12)]
    out["attn_q"], out["attn_k"], out["attn_v"] = qs, ks, vs
    out["attn_y_bits"] = np.stack(ys).view(np.uint32)
    for case, dims, types, seed in (("plain", ATTN_PLAIN_DIMS, ATTN_PLAIN_TYPES, 20261206),
                                    ("kq", ATTN_KQ_DIMS, ATTN_KQ_TYPES, 20261207)):
        w, vec, cache, xs = attention_inputs(np.random.default_rng(seed), dims, types)
        for n, (t, data) in w.items():
            out[f"{case}_w_{n}"] = data
            out[f"{case}_t_{n}"] = np.array([t])
        for n, v in vec.items():
            out[f"{case}_v_{n}"] = v
        out[f"{case}_keys0"] = cache.keys.copy()
        out[f"{case}_values0"] = cache.values.copy()
        out[f"{case}_length0"] = np.array([cache.length])
        out[f"{case}_x"] = xs
        ys, traces, projs = [], [], []
        own = cache.copy()
        for i in range(xs.shape[0]):
            overrides = None
            if case == "kq":
                # the oracle's projections of this step (its own cache carried alongside)
                _, tr = oracle.attention_block_step(dims, w, vec, own, ATTN_POSITIONS[i], xs[i], threads=1)
                overrides = {"q": tr["qfull"], "k": tr["k"], "v": tr["v"], "out": tr["branch"], "gate": tr["gate"],
                             "up": tr["up"], "down": tr["ffn"]}
                projs.append(np.concatenate([overrides[n] for n in oracle.ATTN_WEIGHTS]))
            y, tr = oracle.ref_attention_block(dims, w, vec, cache, ATTN_POSITIONS[i], xs[i], overrides=overrides)
            ys.append(y)
            traces.append(np.concatenate([tr[n] for n in oracle.ATTN_TRACE]))
        out[f"{case}_y_bits"] = np.stack(ys).view(np.uint32)
        out[f"{case}_trace_bits"] = np.stack(traces).view(np.uint32)
        out[f"{case}_keys_bits"] = cache.keys.view(np.uint32)
        out[f"{case}_values_bits"] = cache.values.view(np.uint32)
        if projs:
            out[f"{case}_proj_bits"] = np.stack(projs).view(np.uint32)
    return out


def main() -> None:
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libref.so is not built: run `make -C oracle ref` first")
    (OUT / "ref_kat.json").write_text(json.dumps(kat(), indent=1) + "\n")
    np.savez_compressed(OUT / "ref_random.npz", **random_vectors())
    np.savez_compressed(OUT / "ref_deltanet.npz", **deltanet_vectors())
    np.savez_compressed(OUT / "ref_block.npz", **block_vectors())
    np.savez_compressed(OUT / "ref_attention.npz", **attention_vectors())
    print("wrote", OUT / "ref_kat.json", OUT / "ref_random.npz", OUT / "ref_deltanet.npz", OUT / "ref_block.npz",
          OUT / "ref_attention.npz")


if __name__ == "__main__":
    main()
