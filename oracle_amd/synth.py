"""Seeded synthetic GGML tensors and activations for the quantized matrix workloads.

Distributions (per workload definition):
  q8_0 : d = fp16(|N(0, 0.02)| / 127), q ~ U{-127..127}
  q4_K : d, dmin = fp16(|N(0, 0.02)| / 63); 8 scales and 8 mins ~ U{0..63} packed in GGML's
         12-byte K-quant form; 4-bit q ~ U{0..15}
  q5_K : as q4_K with a fifth bit ~ U{0,1} (32-byte qh plane)
  q6_K : d = fp16(|N(0, 0.02)| / 63); sc ~ U{-32..31} (int8); 6-bit q ~ U{0..63} split into the
         ql (low nibble) and qh (two high bits) planes
  activations x ~ N(0, 1) in F32
numpy's PCG64 generator makes every stream reproducible from its seed on any platform.
"""
from __future__ import annotations

import numpy as np

Q4_K, Q5_K, Q6_K, Q8_0 = 12, 13, 14, 8


def _f16_bits(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint16)


def _u16_bytes(bits: np.ndarray) -> np.ndarray:
    return bits.astype("<u2").view(np.uint8).reshape(-1, 2)


def pack_scale_min_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of the K-quant 6-bit (scale, min) unpack: (nb, 8) x2 -> (nb, 12) bytes.
    Pairs 0..3 occupy the low six bits of bytes 0..3 / 4..7; pairs 4..7 keep their low nibbles
    in bytes 8..11 (scale low, min high) and their top two bits in bits 6..7 of bytes 0..7."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    p = np.empty((sc.shape[0], 12), dtype=np.uint8)
    p[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    p[:, 4:8] = mn[:, 0:4] | ((mn[:, 4:8] >> 4) << 6)
    p[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return p


def _scale(rng: np.random.Generator, nb: int, div: float) -> np.ndarray:
    return _f16_bits(np.abs(rng.normal(0.0, 0.02, nb)) / div)


def q4_k(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    assert cols % 256 == 0
    nb = rows * cols // 256
    d = _u16_bytes(_scale(rng, nb, 63.0))
    dmin = _u16_bytes(_scale(rng, nb, 63.0))
    sc = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    qs = np.frombuffer(rng.bytes(nb * 128), dtype=np.uint8).reshape(nb, 128)
    return np.concatenate([d, dmin, pack_scale_min_k4(sc, mn), qs], axis=1).reshape(-1)


def q5_k(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    assert cols % 256 == 0
    nb = rows * cols // 256
    d = _u16_bytes(_scale(rng, nb, 63.0))
    dmin = _u16_bytes(_scale(rng, nb, 63.0))
    sc = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    qh = np.frombuffer(rng.bytes(nb * 32), dtype=np.uint8).reshape(nb, 32)
    qs = np.frombuffer(rng.bytes(nb * 128), dtype=np.uint8).reshape(nb, 128)
    return np.concatenate([d, dmin, pack_scale_min_k4(sc, mn), qh, qs], axis=1).reshape(-1)


def q6_k(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    assert cols % 256 == 0
    nb = rows * cols // 256
    ql = np.frombuffer(rng.bytes(nb * 128), dtype=np.uint8).reshape(nb, 128)
    qh = np.frombuffer(rng.bytes(nb * 64), dtype=np.uint8).reshape(nb, 64)
    sc = rng.integers(-32, 32, (nb, 16), dtype=np.int8).view(np.uint8)
    d = _u16_bytes(_scale(rng, nb, 63.0))
    return np.concatenate([ql, qh, sc, d], axis=1).reshape(-1)


def q8_0(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    assert cols % 32 == 0
    nb = rows * cols // 32
    d = _u16_bytes(_scale(rng, nb, 127.0))
    q = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    return np.concatenate([d, q], axis=1).reshape(-1)


def weights(type_id: int, rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    gen = {Q4_K: q4_k, Q5_K: q5_k, Q6_K: q6_k, Q8_0: q8_0}[type_id]
    return gen(rng, rows, cols)


def activations(rng: np.random.Generator, m: int, k: int) -> np.ndarray:
    return rng.standard_normal((m, k), dtype=np.float32)


def row_bytes(type_id: int, cols: int) -> int:
    per = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34)}[type_id]
    return cols // per[0] * per[1]


# Gated DeltaNet decode block (Qwen3.5-style recurrent layer, batch 1).  Projections use the
# distributions above (q/k/v/z/beta/alpha and the FFN in q4_K, the output projection in q6_K);
# the recurrent state is F32 ~ N(0, 0.01) (standard deviation), the convolution history and
# input x ~ N(0, 1); norm weights 1 + N(0, 0.1); conv taps N(0, 0.5); dt_bias ~ N(0, 1);
# decay = -exp(N(0, 0.5)) < 0, so every head's state decay exp(softplus(.) * decay) is in (0, 1).
DELTANET_DIMS = {"embedding": 4096, "key_heads": 32, "value_heads": 32, "key_dim": 128, "value_dim": 128,
                 "conv_kernel": 4, "ffn": 12288, "eps": 1e-6}


def deltanet_block(rng: np.random.Generator, dims: dict | None = None):
    """(dims, weights {name: (type, bytes)}, vectors {name: F32}, conv_history, state, x)."""
    d = dict(DELTANET_DIMS if dims is None else dims)
    E, F = d["embedding"], d["ffn"]
    Hk, Hv, dk, dv, K = d["key_heads"], d["value_heads"], d["key_dim"], d["value_dim"], d["conv_kernel"]
    C, V = 2 * Hk * dk + Hv * dv, Hv * dv
    shapes = {"qkv": (Q4_K, C, E), "z": (Q4_K, V, E), "beta": (Q4_K, Hv, E), "alpha": (Q4_K, Hv, E),
              "out": (Q6_K, E, V), "gate": (Q4_K, F, E), "up": (Q4_K, F, E), "down": (Q4_K, E, F)}
    w = {n: (t, weights(t, rng, rows, cols)) for n, (t, rows, cols) in shapes.items()}
    vec = {
        "input_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
        "conv_weight": (0.5 * rng.standard_normal(C * K)).astype(np.float32),
        "dt_bias": rng.standard_normal(Hv).astype(np.float32),
        "decay": (-np.exp(0.5 * rng.standard_normal(Hv))).astype(np.float32),
        "out_norm": (1.0 + 0.1 * rng.standard_normal(dv)).astype(np.float32),
        "post_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
    }
    conv_history = rng.standard_normal((C, K)).astype(np.float32)
    state = (0.01 * rng.standard_normal((Hv, dk, dv))).astype(np.float32)
    x = rng.standard_normal(E).astype(np.float32)
    return d, w, vec, conv_history, state, x


# hidden 4096, 16 query heads over 4 KV heads of 256 (MRoPE over 64 dimensions), FFN 12288
ATTENTION_DIMS = dict(embedding=4096, q_heads=16, kv_heads=4, head_dim=256, ffn=12288, rope_dim=64,
                      rope_sections=[11, 11, 10, 0], rope_base=1e7, eps=1e-6)


def attention_block(rng: np.random.Generator, dims: dict | None = None, cached: int = 4096):
    """(dims, weights {name: (type, bytes)}, vectors {name: F32}, keys, values, x): q4_K
    projections (out and down q6_K / q4_K as in the DeltaNet block) and `cached` tokens of keys
    and values [cached][kv_heads][head_dim]."""
    d = dict(ATTENTION_DIMS if dims is None else dims)
    E, F, Hq, Hkv, D = d["embedding"], d["ffn"], d["q_heads"], d["kv_heads"], d["head_dim"]
    Q, KV = Hq * D, Hkv * D
    shapes = {"q": (Q4_K, 2 * Q, E), "k": (Q4_K, KV, E), "v": (Q4_K, KV, E), "out": (Q6_K, E, Q),
              "gate": (Q4_K, F, E), "up": (Q4_K, F, E), "down": (Q4_K, E, F)}
    w = {n: (t, weights(t, rng, rows, cols)) for n, (t, rows, cols) in shapes.items()}
    vec = {
        "input_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
        "q_norm": (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32),
        "k_norm": (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32),
        "post_norm": (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32),
    }
    keys = rng.standard_normal((cached, Hkv, D)).astype(np.float32)
    values = rng.standard_normal((cached, Hkv, D)).astype(np.float32)
    x = rng.standard_normal(E).astype(np.float32)
    return d, w, vec, keys, values, x
