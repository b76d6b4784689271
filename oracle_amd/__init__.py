"""oracle_amd -- MI355X (gfx950) quantized-weight matrix path.

Python view of liboq.so's C ABI (include/oq.h), used by the tests and the benchmark.  The
production host side is the C++20 adapter in oracle_amd/host/, which mirrors the reference's
oracle::backend::cpu quantized functions.  Errors surface as the reference's exception kinds:

    std::invalid_argument -> InvalidArgument (ValueError)
    std::out_of_range     -> OutOfRange (IndexError)
    std::overflow_error   -> Overflow (OverflowError)
    std::runtime_error    -> UnsupportedType (RuntimeError)   [unregistered / ragged type]
    std::logic_error      -> LogicError
    HIP failures          -> DeviceError / DeviceOutOfMemory
"""
from __future__ import annotations

import contextlib
import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import _lib

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q8_K = 15
TYPE_BF16 = 30
QK_K = 256
Q8K_BLOCK_BYTES = 292


class OqError(Exception):
    code = 0


class InvalidArgument(OqError, ValueError):
    code = _lib.OQ_INVALID_ARGUMENT


class OutOfRange(OqError, IndexError):
    code = _lib.OQ_OUT_OF_RANGE


class Overflow(OqError, OverflowError):
    code = _lib.OQ_OVERFLOW


class UnsupportedType(OqError, RuntimeError):
    code = _lib.OQ_UNSUPPORTED_TYPE


class DeviceError(OqError, RuntimeError):
    code = _lib.OQ_DEVICE_ERROR


class DeviceOutOfMemory(DeviceError):
    code = _lib.OQ_OUT_OF_MEMORY


class LogicError(OqError):
    code = _lib.OQ_LOGIC_ERROR


_BY_CODE = {cls.code: cls for cls in (InvalidArgument, OutOfRange, Overflow, UnsupportedType,
                                      DeviceError, DeviceOutOfMemory, LogicError)}


def _check(rc: int, ctx_handle=None) -> None:
    if rc == _lib.OQ_OK:
        return
    lib = _lib.load()
    msg = lib.oq_last_error(ctx_handle).decode(errors="replace")
    raise _BY_CODE.get(rc, OqError)(msg)


@contextlib.contextmanager
def launch_options(env: dict):
    """Run a block with the given OQ_* launch options set (they select alternative kernel
    schedules; the library reads them once per oq_reload_options), restoring them afterwards."""
    lib = _lib.load()
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    lib.oq_reload_options()
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        lib.oq_reload_options()


# ---------------------------------------------------------------- registry

@dataclass(frozen=True)
class GgmlTypeLayout:
    """Mirror of oracle::model::GgmlTypeLayout (include/oracle/model/ggml_type.hpp:9-15)."""
    type: int
    name: str
    block_elements: int
    bytes_per_block: int
    quantized: bool


def ggml_type_layout(type_id: int) -> GgmlTypeLayout | None:
    """ggml_type_layout (src/model/ggml_type.cpp:69-75): None for unknown/removed ids."""
    lib = _lib.load()
    be, bpb, q = C.c_uint64(), C.c_uint64(), C.c_int()
    name = C.c_char_p()
    if lib.oq_type_layout(type_id, C.byref(be), C.byref(bpb), C.byref(q), C.byref(name)) != 0:
        return None
    return GgmlTypeLayout(type_id, name.value.decode(), be.value, bpb.value, bool(q.value))


def ggml_row_byte_size(row_elements: int, type_id: int) -> int:
    """ggml_row_byte_size (src/model/ggml_type.cpp:77-94), same error kinds."""
    lib = _lib.load()
    out = C.c_uint64()
    _check(lib.oq_row_byte_size(row_elements, type_id, C.byref(out)))
    return out.value


def type_supported(type_id: int) -> bool:
    return bool(_lib.load().oq_type_supported(type_id))


# ---------------------------------------------------------------- device objects

class DeviceBuffer:
    """Device (HBM) allocation owned by a Context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        ctx._call(ctx.lib.oq_device_alloc, ctx.h, self.nbytes, C.byref(p))
        self.ptr = p.value

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        if a.nbytes > self.nbytes:
            raise InvalidArgument("host array larger than device buffer")
        self.ctx._call(self.ctx.lib.oq_copy_to_device, self.ctx.h, self.ptr, a.ctypes.data, a.nbytes)
        return self

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        self.ctx._call(self.ctx.lib.oq_copy_to_host, self.ctx.h, out.ctypes.data, self.ptr, out.nbytes)
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx._call(self.ctx.lib.oq_device_free, self.ctx.h, self.ptr)
            self.ptr = None


class Weight:
    """A GGML tensor uploaded once to HBM (oq_weight)."""

    def __init__(self, ctx: "Context", handle: int, type_id: int, ne0: int, ne1: int, owned_by_model: bool = False):
        self.ctx, self.h = ctx, handle
        self.type, self.ne0, self.ne1 = type_id, ne0, ne1
        self.owned_by_model = owned_by_model  # released with its Model, not by release()

    @property
    def device_bytes(self) -> int:
        db = C.c_uint64()
        _check(self.ctx.lib.oq_weight_info(self.h, None, None, None, C.byref(db)))
        return db.value

    def release(self) -> None:
        if self.h and not self.owned_by_model:
            self.ctx.lib.oq_weight_release(self.h)
        self.h = None


class Graph:
    def __init__(self, ctx: "Context", handle: int):
        self.ctx, self.h = ctx, handle

    def launch(self) -> None:
        self.ctx._call(self.ctx.lib.oq_graph_launch, self.ctx.h, self.h)

    def destroy(self) -> None:
        if self.h:
            self.ctx.lib.oq_graph_destroy(self.h)
            self.h = None


class Context:
    """One device + one HIP stream (oq_context)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        _check(self.lib.oq_context_create(device, C.byref(h)))
        self.h = h.value

    def _call(self, fn, *args) -> None:
        _check(fn(*args), self.h)

    def close(self) -> None:
        if self.h:
            self.lib.oq_context_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # memory
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    def sync(self) -> None:
        self._call(self.lib.oq_synchronize, self.h)

    # weights
    def upload(self, type_id: int, ne0: int, ne1: int, data) -> Weight:
        buf = np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        buf = np.ascontiguousarray(buf)
        h = C.c_void_p()
        self._call(self.lib.oq_weight_upload, self.h, type_id, ne0, ne1,
                   buf.ctypes.data if buf.size else None, buf.nbytes, C.byref(h))
        return Weight(self, h.value, type_id, ne0, ne1)

    def upload_from_device(self, type_id: int, ne0: int, ne1: int, buf: DeviceBuffer, nbytes: int) -> Weight:
        h = C.c_void_p()
        self._call(self.lib.oq_weight_upload_device, self.h, type_id, ne0, ne1, buf.ptr, nbytes, C.byref(h))
        return Weight(self, h.value, type_id, ne0, ne1)

    # compute (device buffers in, device buffers out; asynchronous on the context stream)
    def dequantize_rows(self, w: Weight, row0: int, nrows: int, out: DeviceBuffer) -> None:
        self._call(self.lib.oq_dequantize_rows, self.h, w.h, row0, nrows, out.ptr if out else None)

    def quantize_q8k(self, x: DeviceBuffer, m: int, k: int, out: DeviceBuffer) -> None:
        self._call(self.lib.oq_quantize_q8k, self.h, x.ptr, m, k, out.ptr)

    def argmax(self, logits: DeviceBuffer, n: int, token: DeviceBuffer, value: DeviceBuffer) -> None:
        self._call(self.lib.oq_argmax, self.h, logits.ptr, n, token.ptr, value.ptr)

    def matvec(self, w: Weight, x: DeviceBuffer, y: DeviceBuffer) -> None:
        self._call(self.lib.oq_matvec, self.h, w.h, x.ptr, y.ptr)

    def matvec_argmax(self, w: Weight, x: DeviceBuffer, y: DeviceBuffer, token: DeviceBuffer, value: DeviceBuffer) -> None:
        """Head matvec and its greedy token in one call (oq_matvec_argmax)."""
        self._call(self.lib.oq_matvec_argmax, self.h, w.h, x.ptr, y.ptr, token.ptr, value.ptr)

    def matvec_q8k(self, w: Weight, q8k: DeviceBuffer, y: DeviceBuffer) -> None:
        self._call(self.lib.oq_matvec_q8k, self.h, w.h, q8k.ptr, y.ptr)

    def matmul(self, w: Weight, m: int, x: DeviceBuffer, y: DeviceBuffer) -> None:
        self._call(self.lib.oq_matmul, self.h, w.h, m, x.ptr, y.ptr)

    def matmul_q8k(self, w: Weight, m: int, q8k: DeviceBuffer, y: DeviceBuffer) -> None:
        self._call(self.lib.oq_matmul_q8k, self.h, w.h, m, q8k.ptr, y.ptr)

    def deltanet_step(self, block: "DeltaNetBlockWeights", conv_history: DeviceBuffer, state: DeviceBuffer,
                      x: DeviceBuffer, y: DeviceBuffer, trace: DeviceBuffer | None = None) -> None:
        """One Gated DeltaNet decode block step (oq_deltanet_step); updates conv_history and state."""
        self._call(self.lib.oq_deltanet_step, self.h, C.byref(block.desc), conv_history.ptr, state.ptr, x.ptr, y.ptr,
                   trace.ptr if trace is not None else None)

    def deltanet_steps(self, block: "DeltaNetBlockWeights", m: int, conv_history: DeviceBuffer, state: DeviceBuffer,
                       x: DeviceBuffer, y: DeviceBuffer, trace: DeviceBuffer | None = None) -> None:
        """m consecutive tokens through the block (oq_deltanet_steps): x, y [m][E]; the same results
        as m deltanet_step calls in order; trace: m traces one after the other."""
        self._call(self.lib.oq_deltanet_steps, self.h, C.byref(block.desc), m, conv_history.ptr, state.ptr, x.ptr,
                   y.ptr, trace.ptr if trace is not None else None)

    def deltanet_step_noalloc(self, block: "DeltaNetBlockWeights", conv_history: DeviceBuffer, state: DeviceBuffer,
                              x: DeviceBuffer, y: DeviceBuffer, trace: DeviceBuffer | None = None) -> None:
        """oq_deltanet_step_noalloc: the same step on the library's fixed per-GPU workspace (no
        device allocation; calls overlapping on one GPU race)."""
        self._call(self.lib.oq_deltanet_step_noalloc, self.h, C.byref(block.desc), conv_history.ptr, state.ptr,
                   x.ptr, y.ptr, trace.ptr if trace is not None else None)

    # timing / graphs
    def kv_cache(self, capacity: int, kv_heads: int, key_dim: int, value_dim: int, dtype: str = "f32") -> "KvCache":
        """A device KV cache (oq_kv_cache_create); dtype "f16" stores binary16 elements
        (oq_kv_cache_create_typed)."""
        types = {"f32": 0, "f16": 1}
        if dtype not in types:
            raise InvalidArgument(f"KV cache dtype must be one of {sorted(types)}")
        h = C.c_void_p()
        self._call(self.lib.oq_kv_cache_create_typed, self.h, capacity, kv_heads, key_dim, value_dim, types[dtype],
                   C.byref(h))
        return KvCache(self, h.value)

    def rope(self, heads: DeviceBuffer, n_heads: int, head_dim: int, rotary_dim: int, sections, base: float,
             position) -> None:
        """apply_qwen35_rope on heads [n_heads][head_dim] in place (oq_rope)."""
        sec = (C.c_int32 * 4)(*[int(v) for v in sections])
        pos = (C.c_uint64 * 3)(*[int(v) for v in position])
        self._call(self.lib.oq_rope, self.h, heads.ptr, n_heads, head_dim, rotary_dim, sec, float(base), pos)

    def attention_step(self, q: DeviceBuffer, q_heads: int, k: DeviceBuffer, v: DeviceBuffer, cache: "KvCache",
                       out: DeviceBuffer) -> None:
        """causal_attention_step: appends (k, v) to the cache and attends (oq_attention_step)."""
        self._call(self.lib.oq_attention_step, self.h, q.ptr, q_heads, k.ptr, v.ptr, cache.h, out.ptr)

    def attention_block_step(self, block: "AttentionBlockWeights", cache: "KvCache", position, x: DeviceBuffer,
                             y: DeviceBuffer, trace: DeviceBuffer | None = None) -> None:
        """One full-attention decode block step (oq_attention_block_step); appends to the cache."""
        pos = (C.c_uint64 * 3)(*[int(v) for v in position])
        self._call(self.lib.oq_attention_block_step, self.h, C.byref(block.desc), cache.h, pos, x.ptr, y.ptr,
                   trace.ptr if trace is not None else None)

    def attention_block_steps(self, block: "AttentionBlockWeights", cache: "KvCache", positions, x: DeviceBuffer,
                              y: DeviceBuffer, trace: DeviceBuffer | None = None) -> None:
        """m consecutive tokens through the full-attention block (oq_attention_block_steps); positions:
        m (temporal, height, width) triples; appends m rows to the cache."""
        pos = [int(v) for p in positions for v in p]
        m = len(pos) // 3
        arr = (C.c_uint64 * len(pos))(*pos)
        self._call(self.lib.oq_attention_block_steps, self.h, C.byref(block.desc), cache.h, m, arr, x.ptr, y.ptr,
                   trace.ptr if trace is not None else None)

    def timer_start(self) -> None:
        self._call(self.lib.oq_timer_start, self.h)

    def timer_stop(self) -> float:
        ms = C.c_float()
        self._call(self.lib.oq_timer_stop, self.h, C.byref(ms))
        return ms.value

    def capture_begin(self) -> None:
        self._call(self.lib.oq_capture_begin, self.h)

    def capture_end(self) -> Graph:
        g = C.c_void_p()
        self._call(self.lib.oq_capture_end, self.h, C.byref(g))
        return Graph(self, g.value)


# ---------------------------------------------------------------- reference-shaped helpers

def greedy_token(ctx: Context, logits: DeviceBuffer, n: int) -> tuple[int, float]:
    """Greedy token over n logits in device memory, with the reference sampler's errors
    (src/runtime/sampler.cpp:22-44): InvalidArgument for NaN logits and for no finite candidate."""
    tok = ctx.alloc(4)
    val = ctx.alloc(4)
    try:
        ctx.argmax(logits, n, tok, val)
        t = int(tok.download(np.uint32, 1)[0])
        v = float(val.download(np.float32, 1)[0])
    finally:
        tok.free()
        val.free()
    if t == 0xFFFFFFFF:
        raise InvalidArgument("logits contain NaN")
    if not np.isfinite(v):
        raise InvalidArgument("logits contain no finite candidates")
    return t, v


def storage_matvec(ctx: Context, type_id: int, rows: int, cols: int, matrix: np.ndarray,
                   vector: np.ndarray) -> np.ndarray:
    """reference_storage_matvec (src/backend/cpu/quantized_reference.cpp:128-162) on the GPU:
    host bytes and host F32 vector in, host F32 output back (upload included)."""
    vec = np.ascontiguousarray(vector, dtype=np.float32)
    if rows == 0 or cols == 0:
        raise InvalidArgument("reference matvec dimensions must be non-zero")
    if vec.size != cols:
        raise InvalidArgument("reference matvec vector length mismatch")
    w = ctx.upload(type_id, cols, rows, matrix)
    try:
        xb = ctx.to_device(vec)
        yb = ctx.alloc(rows * 4)
        ctx.matvec(w, xb, yb)
        y = yb.download(np.float32, rows)
        xb.free()
        yb.free()
        return y
    finally:
        w.release()


def decode_rows(ctx: Context, type_id: int, cols: int, rows: int, data: np.ndarray) -> np.ndarray:
    """reference_decode_mapped_tensor (src/backend/cpu/quantized_reference.cpp:85-105) on the GPU."""
    w = ctx.upload(type_id, cols, rows, data)
    try:
        out = ctx.alloc(rows * cols * 4)
        ctx.dequantize_rows(w, 0, rows, out)
        r = out.download(np.float32, rows * cols)
        out.free()
        return r.reshape(rows, cols)
    finally:
        w.release()


DELTANET_WEIGHTS = ("qkv", "z", "beta", "alpha", "out", "gate", "up", "down")
DELTANET_VECTORS = ("input_norm", "conv_weight", "dt_bias", "decay", "out_norm", "post_norm")


class DeltaNetBlockWeights:
    """Device-resident weights of one Gated DeltaNet block: the eight projections uploaded once
    (weights[name] = (ggml type, host bytes)) and the F32 vectors copied to HBM."""

    def __init__(self, ctx: Context, dims: dict, weights: dict, vectors: dict):
        from ._lib import DeltaNetBlock
        E, F = int(dims["embedding"]), int(dims["ffn"])
        Hk, Hv, dk, dv = (int(dims[k]) for k in ("key_heads", "value_heads", "key_dim", "value_dim"))
        C_, V = 2 * Hk * dk + Hv * dv, Hv * dv
        shapes = {"qkv": (E, C_), "z": (E, V), "beta": (E, Hv), "alpha": (E, Hv), "out": (V, E),
                  "gate": (E, F), "up": (E, F), "down": (F, E)}
        self.weights = {n: ctx.upload(weights[n][0], shapes[n][0], shapes[n][1], weights[n][1])
                        for n in DELTANET_WEIGHTS}
        self.vectors = {n: ctx.to_device(np.ascontiguousarray(vectors[n], dtype=np.float32))
                        for n in DELTANET_VECTORS}
        d = DeltaNetBlock()
        for k in ("embedding", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel", "ffn"):
            setattr(d, k, int(dims[k]))
        d.eps = float(dims["eps"])
        for n in DELTANET_WEIGHTS:
            setattr(d, n, self.weights[n].h)
        for n in DELTANET_VECTORS:
            setattr(d, n, self.vectors[n].ptr)
        self.desc = d
        self.dims = dict(dims)

    def weight_bytes(self) -> int:
        """GGML bytes of the eight projections (what one block step streams)."""
        return sum(ggml_row_byte_size(w.ne0, w.type) * w.ne1 for w in self.weights.values())

    def release(self) -> None:
        for w in self.weights.values():
            w.release()
        for v in self.vectors.values():
            v.free()


class KvCache:
    """A device KV cache in the reference's layout (oq_kv_cache): keys [capacity][kv_heads][key_dim],
    values [capacity][kv_heads][value_dim], F32 (or binary16 for an F16 cache) in HBM."""

    def __init__(self, ctx: Context, handle: int):
        self.ctx = ctx
        self.h = handle
        self.capacity = int(ctx.lib.oq_kv_cache_capacity(handle))
        self.dtype = np.float16 if int(ctx.lib.oq_kv_cache_type(handle)) == 1 else np.float32
        k, v = C.c_void_p(), C.c_void_p()
        ctx._call(ctx.lib.oq_kv_cache_arrays, handle, C.byref(k), C.byref(v))
        self.keys_ptr, self.values_ptr = k.value, v.value

    def __len__(self) -> int:
        return int(self.ctx.lib.oq_kv_cache_size(self.h))

    def reset(self) -> None:
        self.ctx._call(self.ctx.lib.oq_kv_cache_reset, self.h)

    def truncate(self, new_length: int) -> None:
        self.ctx._call(self.ctx.lib.oq_kv_cache_truncate, self.h, new_length)

    def _view(self, ptr: int, width: int) -> DeviceBuffer:
        b = DeviceBuffer.__new__(DeviceBuffer)  # a view: never freed through this object
        b.ctx, b.ptr, b.nbytes = self.ctx, ptr, self.capacity * width * np.dtype(self.dtype).itemsize
        return b

    def download(self, kv_heads: int, key_dim: int, value_dim: int) -> tuple[np.ndarray, np.ndarray]:
        """(keys, values) as F32 [capacity][kv_heads][dim] arrays (an F16 cache's elements widened)."""
        kb = self._view(self.keys_ptr, kv_heads * key_dim).download(self.dtype).astype(np.float32)
        vb = self._view(self.values_ptr, kv_heads * value_dim).download(self.dtype).astype(np.float32)
        return kb.reshape(self.capacity, kv_heads, key_dim), vb.reshape(self.capacity, kv_heads, value_dim)

    def load(self, keys: np.ndarray, values: np.ndarray, length: int) -> None:
        """Stores the first `length` token rows of keys / values and sets the length (oq_kv_cache_load)."""
        k = np.ascontiguousarray(keys, dtype=np.float32)
        v = np.ascontiguousarray(values, dtype=np.float32)
        self.ctx._call(self.ctx.lib.oq_kv_cache_load, self.h, k.ctypes.data, v.ctypes.data, length)

    def release(self) -> None:
        if self.h:
            self.ctx.lib.oq_kv_cache_release(self.h)
            self.h = None


ATTENTION_WEIGHTS = ("q", "k", "v", "out", "gate", "up", "down")
ATTENTION_VECTORS = ("input_norm", "q_norm", "k_norm", "post_norm")


class AttentionBlockWeights:
    """Device-resident weights of one full-attention block: the seven projections uploaded once
    (weights[name] = (ggml type, host bytes)) and the F32 vectors copied to HBM."""

    def __init__(self, ctx: Context, dims: dict, weights: dict, vectors: dict):
        from ._lib import AttentionBlock
        E, F, Hq, Hkv, D = (int(dims[k]) for k in ("embedding", "ffn", "q_heads", "kv_heads", "head_dim"))
        Q, KV = Hq * D, Hkv * D
        shapes = {"q": (E, 2 * Q), "k": (E, KV), "v": (E, KV), "out": (Q, E), "gate": (E, F), "up": (E, F),
                  "down": (F, E)}
        self.weights = {n: ctx.upload(weights[n][0], shapes[n][0], shapes[n][1], weights[n][1])
                        for n in ATTENTION_WEIGHTS}
        self.vectors = {n: ctx.to_device(np.ascontiguousarray(vectors[n], dtype=np.float32))
                        for n in ATTENTION_VECTORS}
        d = AttentionBlock()
        for k in ("embedding", "q_heads", "kv_heads", "head_dim", "ffn", "rope_dim"):
            setattr(d, k, int(dims[k]))
        for i, v in enumerate(dims["rope_sections"]):
            d.rope_sections[i] = int(v)
        d.rope_base = float(dims["rope_base"])
        d.eps = float(dims["eps"])
        for n in ATTENTION_WEIGHTS:
            setattr(d, n, self.weights[n].h)
        for n in ATTENTION_VECTORS:
            setattr(d, n, self.vectors[n].ptr)
        self.desc = d
        self.dims = dict(dims)

    def weight_bytes(self) -> int:
        return sum(ggml_row_byte_size(w.ne0, w.type) * w.ne1 for w in self.weights.values())

    def release(self) -> None:
        for w in self.weights.values():
            w.release()
        for v in self.vectors.values():
            v.free()


# ---------------------------------------------------------------- whole-model upload

@dataclass(frozen=True)
class ModelTensor:
    name: str
    type: int
    dims: tuple
    nbytes: int
    weight: "Weight | None"
    data_dev: int | None


def model_tensor_descs(tensors) -> tuple:
    """oq_tensor_desc array for (name, dims, GGML type, payload offset) entries; returns the array
    and the encoded names (which must outlive the call)."""
    from ._lib import TensorDesc
    arr = (TensorDesc * len(tensors))()
    names = []
    for d, (name, dims, t, off) in zip(arr, tensors):
        nb = name.encode()
        names.append(nb)
        d.name = nb
        d.type = t
        d.n_dims = len(dims)
        for i, v in enumerate(dims):
            d.dims[i] = v
        d.offset = off
    return arr, names


def model_validate(payload_bytes: int, tensors) -> None:
    """oq_model_validate: the reference's MappedGgufModel checks on a tensor table (no device)."""
    lib = _lib.load()
    arr, _names = model_tensor_descs(tensors)
    _check(lib.oq_model_validate(payload_bytes, arr, len(tensors)))


class Model:
    """A whole GGUF payload uploaded once (oq_model_upload), tensors looked up by name."""

    def __init__(self, ctx: "Context", payload: np.ndarray, tensors):
        lib = _lib.load()
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        arr, _names = model_tensor_descs(tensors)
        h = C.c_void_p()
        _check(lib.oq_model_upload(ctx.h, payload.ctypes.data, payload.nbytes, arr, len(tensors), C.byref(h)), ctx.h)
        self.ctx, self.lib, self.h = ctx, lib, h

    @classmethod
    def from_gguf(cls, ctx: "Context", gguf_file) -> "Model":
        """Upload every tensor of a GGUF file read by oracle_amd.gguf.read (payload = the mmap'd file)."""
        tensors = [(t.name, t.dims, t.type, t.absolute_offset) for t in gguf_file.tensors]
        return cls(ctx, gguf_file.payload(), tensors)

    def __len__(self) -> int:
        return int(self.lib.oq_model_tensor_count(self.h))

    def device_bytes(self) -> int:
        return int(self.lib.oq_model_device_bytes(self.h))

    def tensor(self, name: str) -> ModelTensor:
        from ._lib import ModelTensorInfo
        idx = C.c_uint64()
        _check(self.lib.oq_model_find(self.h, name.encode(), C.byref(idx)))
        info = ModelTensorInfo()
        _check(self.lib.oq_model_tensor(self.h, idx.value, C.byref(info)))
        w = None
        if info.weight:
            w = Weight(self.ctx, info.weight, info.type, info.dims[0], info.dims[1], owned_by_model=True)
        return ModelTensor(info.name.decode(), info.type, tuple(info.dims[:info.n_dims]), info.nbytes, w,
                           info.data_dev)

    def release(self) -> None:
        if self.h:
            self.lib.oq_model_release(self.h)
            self.h = None
