"""ORACLE -- test infrastructure, not product code.

ctypes view of the CPU restatement (liboracle.so, built from oracle.c) and, where it was built
from the reference's own sources, of the reference's quantized path (_ref/libref.so).  Only the
tests, the smoke check and the CPU-baseline leg of the benchmark use this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libref.so"
REFERENCE_TREE = Path("/root/reference")

_P = C.c_void_p
_U64 = C.c_uint64
_U32 = C.c_uint32
_F = C.POINTER(C.c_float)
_D = C.POINTER(C.c_double)

_ORC_SIGS = [
    ("orc_last_error", C.c_char_p, []),
    ("orc_type_layout", C.c_int, [_U32, C.POINTER(_U64), C.POINTER(_U64), C.POINTER(C.c_int), C.POINTER(C.c_char_p)]),
    ("orc_row_byte_size", C.c_int, [_U64, _U32, C.POINTER(_U64)]),
    ("orc_f16_to_f32", C.c_float, [C.c_uint16]),
    ("orc_bf16_to_f32", C.c_float, [C.c_uint16]),
    ("orc_check_row", C.c_int, [_U32, _U64, _U64]),
    ("orc_decode_row", C.c_int, [_U32, _U64, _P, _U64, _P]),
    ("orc_storage_dot", C.c_int, [_U32, _U64, _P, _U64, _P, _F]),
    ("orc_storage_matvec", C.c_int, [_U32, _U64, _U64, _P, _U64, _P, _P]),
    ("orc_storage_matvec_mt", C.c_int, [_U32, _U64, _U64, _P, _U64, _P, _P, C.c_int]),
    ("orc_storage_matmul_mt", C.c_int, [_U32, _U64, _U64, _P, _U64, _U64, _P, _P, C.c_int]),
    ("orc_storage_dot_stats", C.c_int, [_U32, _U64, _P, _U64, _P, _D, _D]),
    ("orc_storage_matvec_stats", C.c_int, [_U32, _U64, _U64, _P, _U64, _P, _P, _P, C.c_int]),
    ("orc_quantize_row_q8_k", C.c_int, [_P, _U64, _P]),
    ("orc_dequantize_row_q8_k", C.c_int, [_P, _U64, _P]),
    ("orc_vec_dot_q8_k", C.c_int, [_U32, _U64, _P, _P, _F]),
    ("orc_fnv1a64", _U64, [_P, _U64]),
    ("orc_sigmoid", C.c_float, [C.c_float]),
    ("orc_softplus", C.c_float, [C.c_float]),
    ("orc_silu", C.c_float, [C.c_float]),
    ("orc_rms_norm_rows", C.c_int, [_P, _P, _U64, _U64, C.c_float, _P]),
    ("orc_conv_step", C.c_int, [_P, _P, _U64, _U64, _P, _P, C.c_int]),
    ("orc_gated_delta_step", C.c_int, [_P, _P, _P, _P, _P, _U64, _U64, _U64, C.c_float, _P, _P]),
    ("orc_deltanet_trace_size", _U64, [_P]),
    ("orc_deltanet_step", C.c_int, [_P, _P, _P, _P, _P, _P, C.c_int]),
    ("orc_rope", C.c_int, [_P, _U64, _U64, _U64, _P, C.c_float, _P]),
    ("orc_attention_step", C.c_int, [_P, _U64, _P, _P, _P, _P]),
    ("orc_attention_trace_size", _U64, [_P]),
    ("orc_attention_block_step", C.c_int, [_P, _P, _P, _P, _P, _P, C.c_int]),
]

_REF_SIGS = [
    ("ref_last_error", C.c_char_p, []),
    ("ref_f16_to_f32", C.c_float, [C.c_uint16]),
    ("ref_bf16_to_f32", C.c_float, [C.c_uint16]),
    ("ref_type_layout", C.c_int, [_U32, C.POINTER(_U64), C.POINTER(_U64), C.POINTER(C.c_int), C.c_char_p, C.c_int]),
    ("ref_row_byte_size", C.c_int, [_U64, _U32, C.POINTER(_U64)]),
    ("ref_decode_row", C.c_int, [_U32, _U64, _P, _U64, _P, _U64]),
    ("ref_storage_dot", C.c_int, [_U32, _U64, _P, _U64, _P, _U64, _F]),
    ("ref_storage_matvec", C.c_int, [_U32, _U64, _U64, _P, _U64, _P, _U64, _P, _U64]),
    ("ref_mapped_tensor_matvec", C.c_int, [_U32, _U64, _U64, _P, _U64, _P, _U64, _P, _U64]),
    ("ref_storage_matvec_rows", C.c_int, [_U32, _U64, _P, _U64, _U64, _U64, _P, _P]),
    ("ref_conv_step", C.c_int, [_U64, _U64, _P, _P, _P, _P, C.c_int]),
    ("ref_gated_delta_step", C.c_int, [_U64, _U64, _U64, _P, _P, _P, _P, _P, C.c_float, _P, _P]),
    ("ref_recurrent_block", C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    ("ref_block_trace_value", C.c_int64, [C.c_char_p, _P, _U64]),
    ("ref_gguf_open", C.c_int, [C.c_char_p, C.POINTER(_U64)]),
    ("ref_rope", C.c_int, [_P, _U64, _U64, _U64, _P, C.c_float, _P]),
    ("ref_attention_step", C.c_int, [_P, _U64, _P, _P, _P, _P]),
    ("ref_attention_block", C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    ("ref_gguf_tensor", C.c_int, [_U64, C.c_char_p, C.c_int, C.POINTER(_U32), C.POINTER(_U32), C.POINTER(_U64),
                                  C.POINTER(_U64), C.POINTER(_U64)]),
]


class OracleError(Exception):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def build(reference: bool = True) -> None:
    """Compile liboracle.so and, when the reference tree is present, _ref/libref.so."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if reference and REFERENCE_TREE.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF={REFERENCE_TREE}"], check=True)


def _bind(path: Path, sigs) -> C.CDLL:
    lib = C.CDLL(str(path))
    for name, res, args in sigs:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_orc = None
_ref = None


def lib() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORACLE_LIB.exists():
            build(reference=False)
        _orc = _bind(ORACLE_LIB, _ORC_SIGS)
    return _orc


def ref_available() -> bool:
    return REF_LIB.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} not built (needs the reference tree at build time)")
        _ref = _bind(REF_LIB, _REF_SIGS)
    return _ref


def _ptr(a: np.ndarray):
    return a.ctypes.data if a.size else None


def _chk(rc: int, which: C.CDLL, err_fn: str) -> None:
    if rc != 0:
        raise OracleError(rc, getattr(which, err_fn)().decode(errors="replace"))


# ---------------------------------------------------------------- restatement wrappers

def decode_row(type_id: int, n: int, data: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    _chk(lib().orc_decode_row(type_id, n, _ptr(d), d.nbytes, _ptr(out)), lib(), "orc_last_error")
    return out


def decode_matrix(type_id: int, cols: int, rows: int, data: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8).reshape(rows, -1)
    return np.stack([decode_row(type_id, cols, d[r]) for r in range(rows)])


def storage_dot(type_id: int, n: int, data: np.ndarray, x: np.ndarray) -> float:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = C.c_float()
    _chk(lib().orc_storage_dot(type_id, n, _ptr(d), d.nbytes, _ptr(xv), C.byref(out)), lib(), "orc_last_error")
    return out.value


def storage_matvec(type_id: int, rows: int, cols: int, data: np.ndarray, x: np.ndarray,
                   threads: int = 1) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    if threads <= 1:
        rc = lib().orc_storage_matvec(type_id, rows, cols, _ptr(d), d.nbytes, _ptr(xv), _ptr(y))
    else:
        rc = lib().orc_storage_matvec_mt(type_id, rows, cols, _ptr(d), d.nbytes, _ptr(xv), _ptr(y), threads)
    _chk(rc, lib(), "orc_last_error")
    return y


def storage_matmul(type_id: int, rows: int, cols: int, data: np.ndarray, x: np.ndarray,
                   threads: int = 1) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    m = xv.size // cols
    y = np.empty((m, rows), dtype=np.float32)
    _chk(lib().orc_storage_matmul_mt(type_id, rows, cols, _ptr(d), d.nbytes, m, _ptr(xv), _ptr(y), threads),
         lib(), "orc_last_error")
    return y


def matvec_stats(type_id: int, rows: int, cols: int, data: np.ndarray, x: np.ndarray,
                 threads: int = 8) -> tuple[np.ndarray, np.ndarray]:
    """(double-precision dot, sum |w x|) per row, the tolerance normaliser."""
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    dot = np.empty(rows, dtype=np.float64)
    ab = np.empty(rows, dtype=np.float64)
    _chk(lib().orc_storage_matvec_stats(type_id, rows, cols, _ptr(d), d.nbytes, _ptr(xv), _ptr(dot), _ptr(ab),
                                        threads), lib(), "orc_last_error")
    return dot, ab


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(xv.size // 256 * 292, dtype=np.uint8)
    _chk(lib().orc_quantize_row_q8_k(_ptr(xv), xv.size, _ptr(out)), lib(), "orc_last_error")
    return out


def dequantize_q8k(blocks: np.ndarray, k: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(k, dtype=np.float32)
    _chk(lib().orc_dequantize_row_q8_k(_ptr(b), k, _ptr(out)), lib(), "orc_last_error")
    return out


def vec_dot_q8k(type_id: int, k: int, wrow: np.ndarray, q8k: np.ndarray) -> float:
    w = np.ascontiguousarray(wrow, dtype=np.uint8)
    q = np.ascontiguousarray(q8k, dtype=np.uint8)
    out = C.c_float()
    _chk(lib().orc_vec_dot_q8_k(type_id, k, _ptr(w), _ptr(q), C.byref(out)), lib(), "orc_last_error")
    return out.value


def fnv1a64(data) -> int:
    a = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), dtype=np.uint8))
    return int(lib().orc_fnv1a64(_ptr(a), a.nbytes))


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def check_row(type_id: int, n: int, nbytes: int) -> int:
    return lib().orc_check_row(type_id, n, nbytes)


def row_byte_size(n: int, type_id: int) -> int:
    out = C.c_uint64()
    _chk(lib().orc_row_byte_size(n, type_id, C.byref(out)), lib(), "orc_last_error")
    return out.value


# ---------------------------------------------------------------- compiled-reference wrappers

def ref_decode_row(type_id: int, n: int, data: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    _chk(ref().ref_decode_row(type_id, n, _ptr(d), d.nbytes, _ptr(out), n), ref(), "ref_last_error")
    return out


def ref_storage_dot(type_id: int, n: int, data: np.ndarray, x: np.ndarray) -> float:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = C.c_float()
    _chk(ref().ref_storage_dot(type_id, n, _ptr(d), d.nbytes, _ptr(xv), xv.size, C.byref(out)), ref(),
         "ref_last_error")
    return out.value


def ref_storage_matvec(type_id: int, rows: int, cols: int, data: np.ndarray, x: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    _chk(ref().ref_storage_matvec(type_id, rows, cols, _ptr(d), d.nbytes, _ptr(xv), xv.size, _ptr(y), rows),
         ref(), "ref_last_error")
    return y


def ref_storage_matvec_threads(type_id: int, rows: int, cols: int, data: np.ndarray, x: np.ndarray,
                               threads: int) -> np.ndarray:
    """The reference's reference_storage_dot over row ranges on `threads` host threads (ctypes
    releases the GIL for the call), for timing its CPU path on several cores."""
    from concurrent.futures import ThreadPoolExecutor
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    rb = d.nbytes // rows
    bounds = [rows * i // threads for i in range(threads + 1)]

    def run(i):
        return ref().ref_storage_matvec_rows(type_id, cols, _ptr(d), rb, bounds[i], bounds[i + 1], _ptr(xv), _ptr(y))

    with ThreadPoolExecutor(max_workers=threads) as pool:
        codes = list(pool.map(run, range(threads)))
    for c in codes:
        _chk(c, ref(), "ref_last_error")
    return y


def ref_conv_step(history: np.ndarray, weights: np.ndarray, x: np.ndarray, apply_silu: bool = False) -> np.ndarray:
    """One step of the reference's causal depthwise convolution; updates `history` in place."""
    ch, kern = history.shape
    w = np.ascontiguousarray(weights, dtype=np.float32)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(ch, dtype=np.float32)
    _chk(ref().ref_conv_step(ch, kern, _ptr(history), _ptr(w), _ptr(xv), _ptr(out), int(apply_silu)), ref(),
         "ref_last_error")
    return out


def ref_gated_delta_step(q, k, v, beta, log_decay, state: np.ndarray, eps: float) -> np.ndarray:
    """One step of the reference's gated delta rule; updates `state` [H][dk][dv] in place."""
    heads, dk, dv = state.shape
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, beta, log_decay)]
    out = np.empty((heads, dv), dtype=np.float32)
    _chk(ref().ref_gated_delta_step(heads, dk, dv, *[_ptr(a) for a in arrs], eps, _ptr(state), _ptr(out)), ref(),
         "ref_last_error")
    return out


def ref_status(fn: str, *args) -> int:
    return getattr(ref(), fn)(*args)


def default_threads() -> int:
    """Host threads for the oracle's parallel loops: the process's CPU share -- OMP_NUM_THREADS
    when the environment sets it, else the CPUs this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return os.cpu_count() or 1


# ---------------------------------------------------------------- greedy token

def greedy_token(logits: np.ndarray) -> tuple[int, float]:
    """Greedy sampling at temperature 0 (src/runtime/sampler.cpp:22-44): ValueError for an
    empty vector, a NaN, or a maximum that is not finite; otherwise the first index holding the
    maximum (strict '>' in index order, as also src/runtime/qwen35_mtp.cpp:300-308) and its value.
    numpy's argmax returns the first occurrence of the maximum."""
    logits = np.asarray(logits, np.float32)
    if logits.size == 0:
        raise ValueError("cannot sample an empty logits vector")
    if np.isnan(logits).any():
        raise ValueError("logits contain NaN")
    i = int(np.argmax(logits))
    if not np.isfinite(logits[i]):
        raise ValueError("logits contain no finite candidates")
    return i, float(logits[i])



# ---------------------------------------------------------------- Gated DeltaNet block

def sigmoid(v: float) -> float:
    return lib().orc_sigmoid(v)


def softplus(v: float) -> float:
    return lib().orc_softplus(v)


def silu(v: float) -> float:
    return lib().orc_silu(v)


def rms_norm_rows(x: np.ndarray, weight: np.ndarray, width: int, eps: float) -> np.ndarray:
    xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(xv)
    _chk(lib().orc_rms_norm_rows(_ptr(xv), _ptr(w), xv.size, width, eps, _ptr(out)), lib(), "orc_last_error")
    return out


def conv_step(history: np.ndarray, weights: np.ndarray, x: np.ndarray, apply_silu: bool = False) -> np.ndarray:
    """Restated causal depthwise convolution step; updates `history` [channels][kernel] in place."""
    ch, kern = history.shape
    w = np.ascontiguousarray(weights, dtype=np.float32)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(ch, dtype=np.float32)
    _chk(lib().orc_conv_step(_ptr(xv), _ptr(w), ch, kern, _ptr(history), _ptr(out), int(apply_silu)), lib(),
         "orc_last_error")
    return out


def gated_delta_step(q, k, v, beta, log_decay, state: np.ndarray, eps: float) -> np.ndarray:
    """Restated gated delta rule step; updates `state` [H][dk][dv] in place."""
    heads, dk, dv = state.shape
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, beta, log_decay)]
    out = np.empty((heads, dv), dtype=np.float32)
    _chk(lib().orc_gated_delta_step(*[_ptr(a) for a in arrs], heads, dk, dv, eps, _ptr(state), _ptr(out)), lib(),
         "orc_last_error")
    return out


class _DNBlock(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim",
                                          "conv_kernel", "ffn")] + [("eps", C.c_float)] + \
               [(n + "_type", C.c_uint32) for n in ("qkv", "z", "beta", "alpha", "out", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("qkv", "z", "beta", "alpha", "out", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("input_norm", "conv_weight", "dt_bias", "decay", "out_norm", "post_norm")]


DN_WEIGHTS = ("qkv", "z", "beta", "alpha", "out", "gate", "up", "down")
DN_VECTORS = ("input_norm", "conv_weight", "dt_bias", "decay", "out_norm", "post_norm")
DN_TRACE = ("qkv", "z", "beta", "alpha", "conv", "rec", "gated", "branch", "resid", "post", "gate", "up", "act", "ffn",
            "beta_s", "log_decay")


def deltanet_trace_sizes(dims: dict) -> dict:
    C_ = 2 * dims["key_heads"] * dims["key_dim"] + dims["value_heads"] * dims["value_dim"]
    V = dims["value_heads"] * dims["value_dim"]
    E, F, Hv = dims["embedding"], dims["ffn"], dims["value_heads"]
    return dict(zip(DN_TRACE, (C_, V, Hv, Hv, C_, V, V, E, E, E, F, F, F, E, Hv, Hv)))


def deltanet_step(dims: dict, weights: dict, vectors: dict, conv_history: np.ndarray, state: np.ndarray,
                  x: np.ndarray, threads: int | None = None, trace: bool = False):
    """Restated recurrent block step.  weights[name] = (ggml type, uint8 bytes); vectors[name] = F32;
    conv_history and state are updated in place.  Returns y (and the intermediates when trace)."""
    b = _DNBlock()
    for k_ in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel", "ffn"):
        setattr(b, k_, int(dims[k_]))
    b.eps = float(dims["eps"])
    keep = []
    for n in DN_WEIGHTS:
        t, data = weights[n]
        a = np.ascontiguousarray(data, dtype=np.uint8)
        keep.append(a)
        setattr(b, n + "_type", int(t))
        setattr(b, n, a.ctypes.data)
    for n in DN_VECTORS:
        a = np.ascontiguousarray(vectors[n], dtype=np.float32)
        keep.append(a)
        setattr(b, n, a.ctypes.data)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(int(dims["embedding"]), dtype=np.float32)
    tr = np.empty(int(lib().orc_deltanet_trace_size(C.byref(b))), dtype=np.float32) if trace else None
    _chk(lib().orc_deltanet_step(C.byref(b), _ptr(conv_history), _ptr(state), _ptr(xv), _ptr(y),
                                 _ptr(tr) if trace else None, threads or default_threads()), lib(), "orc_last_error")
    if not trace:
        return y
    out, off = {}, 0
    for n, sz in deltanet_trace_sizes(dims).items():
        out[n] = tr[off:off + sz]
        off += sz
    return y, out


class _RefDNBlock(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim",
                                          "conv_kernel", "ffn")] + [("eps", C.c_float)] + \
               [("types", C.c_uint32 * 8), ("weights", C.c_void_p * 8)] + \
               [(n, C.c_void_p) for n in DN_VECTORS]


def ref_recurrent_block(dims: dict, weights: dict, vectors: dict, conv_history: np.ndarray, state: np.ndarray,
                        x: np.ndarray, overrides: dict | None = None):
    """The reference's own recurrent block (execute_qwen35_recurrent_block_reference) on in-memory
    views.  Same arguments as deltanet_step; overrides maps projection names (DN_WEIGHTS) to F32
    outputs that replace the reference's matvec for that projection.  conv_history and state are
    updated in place.  Returns (y, trace dict with the fields of deltanet_step)."""
    b = _RefDNBlock()
    for k_ in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel", "ffn"):
        setattr(b, k_, int(dims[k_]))
    b.eps = float(dims["eps"])
    keep = []
    for i, n in enumerate(DN_WEIGHTS):
        t, data = weights[n]
        a = np.ascontiguousarray(data, dtype=np.uint8)
        keep.append(a)
        b.types[i] = int(t)
        b.weights[i] = a.ctypes.data
    for n in DN_VECTORS:
        a = np.ascontiguousarray(vectors[n], dtype=np.float32)
        keep.append(a)
        setattr(b, n, a.ctypes.data)
    ov = None
    if overrides:
        ov = (C.c_void_p * 8)()
        for i, n in enumerate(DN_WEIGHTS):
            if n in overrides:
                a = np.ascontiguousarray(overrides[n], dtype=np.float32)
                keep.append(a)
                ov[i] = a.ctypes.data
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(int(dims["embedding"]), dtype=np.float32)
    sizes = deltanet_trace_sizes(dims)
    tr = np.empty(sum(sizes.values()), dtype=np.float32)
    _chk(ref().ref_recurrent_block(C.byref(b), _ptr(conv_history), _ptr(state), _ptr(xv), _ptr(y), _ptr(tr),
                                   ov), ref(), "ref_last_error")
    out, off = {}, 0
    for n, sz in sizes.items():
        out[n] = tr[off:off + sz]
        off += sz
    return y, out


def ref_block_trace_value(name: str) -> np.ndarray:
    """A named trace tensor of the last ref_recurrent_block call (the reference's own names)."""
    n = int(ref().ref_block_trace_value(name.encode(), None, 0))
    if n < 0:
        raise KeyError(name)
    out = np.empty(n, dtype=np.float32)
    ref().ref_block_trace_value(name.encode(), _ptr(out), n)
    return out


def ref_gguf_tensors(path) -> list[dict]:
    """The tensor table the reference's MappedGgufModel builds for a GGUF file (raises OracleError
    with the reference's message when it rejects the file)."""
    n = C.c_uint64()
    _chk(ref().ref_gguf_open(str(path).encode(), C.byref(n)), ref(), "ref_last_error")
    out = []
    for i in range(n.value):
        name = C.create_string_buffer(512)
        t, nd, off, nb = C.c_uint32(), C.c_uint32(), C.c_uint64(), C.c_uint64()
        dims = (C.c_uint64 * 4)()
        _chk(ref().ref_gguf_tensor(i, name, 512, C.byref(t), C.byref(nd), dims, C.byref(off), C.byref(nb)), ref(),
             "ref_last_error")
        out.append({"name": name.value.decode(), "type": t.value, "dims": list(dims[:nd.value]),
                    "absolute_offset": off.value, "nbytes": nb.value})
    return out


# ---------------------------------------------------------------- full-attention decode

class KvCache:
    """KV cache in the reference's layout (hybrid_cache.cpp:131-207): keys [capacity][kv_heads][key_dim],
    values [capacity][kv_heads][value_dim], F32, `length` tokens stored."""

    def __init__(self, capacity: int, kv_heads: int, key_dim: int, value_dim: int):
        self.keys = np.zeros((capacity, kv_heads, key_dim), dtype=np.float32)
        self.values = np.zeros((capacity, kv_heads, value_dim), dtype=np.float32)
        self.length = 0

    @property
    def capacity(self) -> int:
        return self.keys.shape[0]

    def copy(self) -> "KvCache":
        c = KvCache(*self.keys.shape, self.values.shape[2])
        c.keys[:] = self.keys
        c.values[:] = self.values
        c.length = self.length
        return c

    def _struct(self):
        s = _KvCacheStruct()
        s.capacity, s.kv_heads, s.key_dim = self.keys.shape
        s.value_dim = self.values.shape[2]
        s.length = self.length
        s.keys = self.keys.ctypes.data
        s.values = self.values.ctypes.data
        return s


class _KvCacheStruct(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("capacity", "kv_heads", "key_dim", "value_dim", "length")] + \
               [("keys", C.c_void_p), ("values", C.c_void_p)]


def _rope_args(sections, position):
    sec = (C.c_int32 * 4)(*[int(v) for v in sections])
    pos = (C.c_uint64 * 3)(*[int(v) for v in position])
    return sec, pos


def rope(heads: np.ndarray, rotary_dim: int, sections, base: float, position, reference: bool = False) -> np.ndarray:
    """apply_qwen35_rope on a copy of heads [n][head_dim]; position = (temporal, height, width)."""
    out = np.array(heads, dtype=np.float32, order="C", copy=True)
    sec, pos = _rope_args(sections, position)
    lb, fn, err = (ref(), "ref_rope", "ref_last_error") if reference else (lib(), "orc_rope", "orc_last_error")
    _chk(getattr(lb, fn)(_ptr(out), out.shape[0], out.shape[1], int(rotary_dim), sec, float(base), pos), lb, err)
    return out


def attention_step(q: np.ndarray, k: np.ndarray, v: np.ndarray, cache: KvCache, reference: bool = False) -> np.ndarray:
    """causal_attention_step: appends k [kv_heads][key_dim] and v to `cache` (in place) and returns
    the output [q_heads][value_dim] of q [q_heads][key_dim]."""
    qv, kv, vv = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    out = np.empty((qv.shape[0], cache.values.shape[2]), dtype=np.float32)
    st = cache._struct()
    lb, fn, err = (ref(), "ref_attention_step", "ref_last_error") if reference else \
        (lib(), "orc_attention_step", "orc_last_error")
    _chk(getattr(lb, fn)(_ptr(qv), qv.shape[0], _ptr(kv), _ptr(vv), C.byref(st), _ptr(out)), lb, err)
    cache.length = int(st.length)
    return out


ATTN_WEIGHTS = ("q", "k", "v", "out", "gate", "up", "down")
ATTN_VECTORS = ("input_norm", "q_norm", "k_norm", "post_norm")
ATTN_TRACE = ("qfull", "k", "v", "qcur", "kcur", "pregate", "gate_s", "gated", "branch", "resid", "post", "gate", "up",
              "act", "ffn")
ATTN_DIMS = ("embedding", "q_heads", "kv_heads", "head_dim", "ffn", "rope_dim")


class _AttnBlock(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ATTN_DIMS] + \
               [("rope_sections", C.c_int32 * 4), ("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n + "_type", C.c_uint32) for n in ATTN_WEIGHTS] + \
               [(n, C.c_void_p) for n in ATTN_WEIGHTS] + \
               [(n, C.c_void_p) for n in ATTN_VECTORS]


class _RefAttnBlock(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ATTN_DIMS] + \
               [("rope_sections", C.c_int32 * 4), ("rope_base", C.c_float), ("eps", C.c_float)] + \
               [("types", C.c_uint32 * 7), ("weights", C.c_void_p * 7)] + \
               [(n, C.c_void_p) for n in ATTN_VECTORS]


def attention_trace_sizes(dims: dict) -> dict:
    Q = dims["q_heads"] * dims["head_dim"]
    KV = dims["kv_heads"] * dims["head_dim"]
    E, F = dims["embedding"], dims["ffn"]
    return dict(zip(ATTN_TRACE, (2 * Q, KV, KV, Q, KV, Q, Q, Q, E, E, E, F, F, F, E)))


def _attn_struct(cls, dims, weights, vectors, keep, ref_layout):
    b = cls()
    for n in ATTN_DIMS:
        setattr(b, n, int(dims[n]))
    for i, v in enumerate(dims["rope_sections"]):
        b.rope_sections[i] = int(v)
    b.rope_base = float(dims["rope_base"])
    b.eps = float(dims["eps"])
    for i, n in enumerate(ATTN_WEIGHTS):
        t, data = weights[n]
        a = np.ascontiguousarray(data, dtype=np.uint8)
        keep.append(a)
        if ref_layout:
            b.types[i] = int(t)
            b.weights[i] = a.ctypes.data
        else:
            setattr(b, n + "_type", int(t))
            setattr(b, n, a.ctypes.data)
    for n in ATTN_VECTORS:
        a = np.ascontiguousarray(vectors[n], dtype=np.float32)
        keep.append(a)
        setattr(b, n, a.ctypes.data)
    return b


def _split_trace(dims, tr):
    out, off = {}, 0
    for n, sz in attention_trace_sizes(dims).items():
        out[n] = tr[off:off + sz]
        off += sz
    return out


def attention_block_step(dims: dict, weights: dict, vectors: dict, cache: KvCache, position, x: np.ndarray,
                         threads: int | None = None):
    """Restated attention block step (dims: ATTN_DIMS + rope_sections, rope_base, eps; weights[name] =
    (ggml type, uint8 bytes)).  Appends to `cache` in place.  Returns (y, trace dict)."""
    keep = []
    b = _attn_struct(_AttnBlock, dims, weights, vectors, keep, False)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(int(dims["embedding"]), dtype=np.float32)
    tr = np.empty(int(lib().orc_attention_trace_size(C.byref(b))), dtype=np.float32)
    st = cache._struct()
    pos = (C.c_uint64 * 3)(*[int(v) for v in position])
    _chk(lib().orc_attention_block_step(C.byref(b), C.byref(st), pos, _ptr(xv), _ptr(y), _ptr(tr),
                                        threads or default_threads()), lib(), "orc_last_error")
    cache.length = int(st.length)
    return y, _split_trace(dims, tr)


def ref_attention_block(dims: dict, weights: dict, vectors: dict, cache: KvCache, position, x: np.ndarray,
                        overrides: dict | None = None):
    """The reference's own attention block (execute_qwen35_attention_block_reference) on in-memory
    views; same arguments as attention_block_step, overrides maps ATTN_WEIGHTS names to F32
    projection outputs.  Appends to `cache` in place.  Returns (y, trace dict)."""
    keep = []
    b = _attn_struct(_RefAttnBlock, dims, weights, vectors, keep, True)
    ov = None
    if overrides:
        ov = (C.c_void_p * 7)()
        for i, n in enumerate(ATTN_WEIGHTS):
            if n in overrides:
                a = np.ascontiguousarray(overrides[n], dtype=np.float32)
                keep.append(a)
                ov[i] = a.ctypes.data
    xv = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(int(dims["embedding"]), dtype=np.float32)
    tr = np.empty(sum(attention_trace_sizes(dims).values()), dtype=np.float32)
    st = cache._struct()
    pos = (C.c_uint64 * 3)(*[int(v) for v in position])
    _chk(ref().ref_attention_block(C.byref(b), C.byref(st), pos, _ptr(xv), _ptr(y), _ptr(tr), ov), ref(),
         "ref_last_error")
    cache.length = int(st.length)
    return y, _split_trace(dims, tr)
