"""ctypes binding of liboq.so (include/oq.h).

The library is built in-tree by oracle_amd/build.py.  Loading never falls back to anything:
a missing or unloadable liboq.so raises immediately.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liboq.so"

OQ_OK = 0
OQ_INVALID_ARGUMENT = -1
OQ_OUT_OF_RANGE = -2
OQ_OVERFLOW = -3
OQ_UNSUPPORTED_TYPE = -4
OQ_DEVICE_ERROR = -5
OQ_OUT_OF_MEMORY = -6
OQ_LOGIC_ERROR = -7
OQ_RUNTIME_ERROR = -8

# (name, restype, argtypes) for every entry point declared in include/oq.h
_P = C.c_void_p
_U64 = C.c_uint64
_U32 = C.c_uint32
SIGNATURES = [
    ("oq_type_layout", C.c_int, [_U32, C.POINTER(_U64), C.POINTER(_U64), C.POINTER(C.c_int), C.POINTER(C.c_char_p)]),
    ("oq_row_byte_size", C.c_int, [_U64, _U32, C.POINTER(_U64)]),
    ("oq_type_supported", C.c_int, [_U32]),
    ("oq_context_create", C.c_int, [C.c_int, C.POINTER(_P)]),
    ("oq_context_destroy", None, [_P]),
    ("oq_last_error", C.c_char_p, [_P]),
    ("oq_synchronize", C.c_int, [_P]),
    ("oq_context_stream", _P, [_P]),
    ("oq_reload_options", None, []),
    ("oq_device_alloc", C.c_int, [_P, _U64, C.POINTER(_P)]),
    ("oq_device_free", C.c_int, [_P, _P]),
    ("oq_copy_to_device", C.c_int, [_P, _P, _P, _U64]),
    ("oq_copy_to_host", C.c_int, [_P, _P, _P, _U64]),
    ("oq_copy_device", C.c_int, [_P, _P, _P, _U64]),
    ("oq_weight_upload", C.c_int, [_P, _U32, _U64, _U64, _P, _U64, C.POINTER(_P)]),
    ("oq_weight_upload_device", C.c_int, [_P, _U32, _U64, _U64, _P, _U64, C.POINTER(_P)]),
    ("oq_weight_release", None, [_P]),
    ("oq_weight_info", C.c_int, [_P, C.POINTER(_U32), C.POINTER(_U64), C.POINTER(_U64), C.POINTER(_U64)]),
    ("oq_model_validate", C.c_int, [_U64, _P, _U64]),
    ("oq_model_upload", C.c_int, [_P, _P, _U64, _P, _U64, C.POINTER(_P)]),
    ("oq_model_release", None, [_P]),
    ("oq_model_tensor_count", _U64, [_P]),
    ("oq_model_find", C.c_int, [_P, C.c_char_p, C.POINTER(_U64)]),
    ("oq_model_tensor", C.c_int, [_P, _U64, _P]),
    ("oq_model_device_bytes", _U64, [_P]),
    ("oq_dequantize_rows", C.c_int, [_P, _P, _U64, _U64, _P]),
    ("oq_quantize_q8k", C.c_int, [_P, _P, _U64, _U64, _P]),
    ("oq_argmax", C.c_int, [_P, _P, _U64, _P, _P]),
    ("oq_matvec", C.c_int, [_P, _P, _P, _P]),
    ("oq_matvec_argmax", C.c_int, [_P, _P, _P, _P, _P, _P]),
    ("oq_matvec_q8k", C.c_int, [_P, _P, _P, _P]),
    ("oq_matmul", C.c_int, [_P, _P, _U64, _P, _P]),
    ("oq_matmul_q8k", C.c_int, [_P, _P, _U64, _P, _P]),
    ("oq_deltanet_step", C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    ("oq_deltanet_steps", C.c_int, [_P, _P, _U64, _P, _P, _P, _P, _P]),
    ("oq_deltanet_step_noalloc", C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    ("oq_deltanet_noalloc_capacity", _U64, []),
    ("oq_kv_cache_create", C.c_int, [_P, _U64, _U64, _U64, _U64, C.POINTER(_P)]),
    ("oq_kv_cache_create_typed", C.c_int, [_P, _U64, _U64, _U64, _U64, C.c_uint32, C.POINTER(_P)]),
    ("oq_kv_cache_type", C.c_uint32, [_P]),
    ("oq_kv_cache_release", None, [_P]),
    ("oq_kv_cache_size", _U64, [_P]),
    ("oq_kv_cache_capacity", _U64, [_P]),
    ("oq_kv_cache_reset", C.c_int, [_P]),
    ("oq_kv_cache_truncate", C.c_int, [_P, _U64]),
    ("oq_kv_cache_arrays", C.c_int, [_P, C.POINTER(_P), C.POINTER(_P)]),
    ("oq_kv_cache_load", C.c_int, [_P, _P, _P, _U64]),
    ("oq_rope", C.c_int, [_P, _P, _U64, _U64, _U64, _P, C.c_float, _P]),
    ("oq_attention_step", C.c_int, [_P, _P, _U64, _P, _P, _P, _P]),
    ("oq_attention_block_step", C.c_int, [_P, _P, _P, _P, _P, _P, _P]),
    ("oq_attention_block_steps", C.c_int, [_P, _P, _P, _U64, _P, _P, _P, _P]),
    ("oq_timer_start", C.c_int, [_P]),
    ("oq_timer_stop", C.c_int, [_P, C.POINTER(C.c_float)]),
    ("oq_capture_begin", C.c_int, [_P]),
    ("oq_capture_end", C.c_int, [_P, C.POINTER(_P)]),
    ("oq_graph_launch", C.c_int, [_P, _P]),
    ("oq_graph_destroy", None, [_P]),
]



class DeltaNetBlock(C.Structure):
    """oq_deltanet_block (include/oq.h)."""
    _fields_ = [(n, C.c_uint64) for n in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim",
                                          "conv_kernel", "ffn")] + [("eps", C.c_float)] + \
               [(n, C.c_void_p) for n in ("qkv", "z", "beta", "alpha", "out", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("input_norm", "conv_weight", "dt_bias", "decay", "out_norm", "post_norm")]


class AttentionBlock(C.Structure):
    """oq_attention_block (include/oq.h)."""
    _fields_ = [(n, C.c_uint64) for n in ("embedding", "q_heads", "kv_heads", "head_dim", "ffn", "rope_dim")] + \
               [("rope_sections", C.c_int32 * 4), ("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n, C.c_void_p) for n in ("q", "k", "v", "out", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("input_norm", "q_norm", "k_norm", "post_norm")]


class TensorDesc(C.Structure):
    """oq_tensor_desc (include/oq.h)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("offset", C.c_uint64)]


class ModelTensorInfo(C.Structure):
    """oq_model_tensor_info (include/oq.h)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("nbytes", C.c_uint64), ("weight", C.c_void_p), ("data_dev", C.c_void_p)]


_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load liboq.so and attach prototypes; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python oracle_amd/build.py` "
            "(or __graft_entry__.build()); there is no fallback path")
    lib = C.CDLL(str(LIB_PATH))
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return [name for name, _, _ in SIGNATURES]
