"""Whole-model upload on the GPU (oq_model_upload): a GGUF file written like the reference's test
fixtures, uploaded once, every tensor looked up by name; rank-2 tensors of the multiplied types
decode bit for bit and multiply within the product bar against the oracle, every other tensor's
GGML bytes are in HBM unchanged."""
import ctypes as C

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import gguf, synth

from test_gguf_model import model_tensors

pytestmark = pytest.mark.gpu

TOL = 1e-4
KQ = (12, 13, 14)


def raw_bytes(ctx, ptr, n):
    out = np.empty(n, np.uint8)
    rc = ctx.lib.oq_copy_to_host(ctx.h, out.ctypes.data, C.c_void_p(ptr), n)
    assert rc == 0
    return out


def test_model_upload_and_lookup(ctx, tmp_path):
    rng = np.random.default_rng(11)
    tensors = model_tensors(rng)
    path = tmp_path / "m.gguf"
    gguf.write(path, tensors)
    f = gguf.read(path)
    model = oracle_amd.Model.from_gguf(ctx, f)
    try:
        assert len(model) == len(tensors)
        assert model.device_bytes() >= sum(d.nbytes for *_, d in tensors)
        for name, dims, t, data in tensors:
            mt = model.tensor(name)
            assert (mt.type, list(mt.dims), mt.nbytes) == (t, dims, data.nbytes)
            if len(dims) == 2 and oracle_amd.type_supported(t):
                cols, rows = dims
                assert mt.weight is not None and mt.data_dev is None
                dec = ctx.alloc(rows * cols * 4)
                ctx.dequantize_rows(mt.weight, 0, rows, dec)
                got = dec.download(np.float32, rows * cols).reshape(rows, cols)
                assert np.array_equal(got.view(np.uint32), oracle.decode_matrix(t, cols, rows, data).view(np.uint32))
                dec.free()
                x = rng.standard_normal(cols).astype(np.float32)
                xb, yb = ctx.to_device(x), ctx.alloc(rows * 4)
                ctx.matvec(mt.weight, xb, yb)
                y = yb.download(np.float32, rows)
                xhat = oracle.dequantize_q8k(oracle.quantize_q8k(x), cols) if t in KQ else x
                y_ref = oracle.storage_matvec(t, rows, cols, data, xhat, threads=4)
                norm = oracle.matvec_stats(t, rows, cols, data, xhat, threads=4)[1]
                assert np.all(np.abs(y.astype(np.float64) - y_ref) <= TOL * np.maximum(norm, 1e-30)), name
                xb.free()
                yb.free()
            else:
                assert mt.weight is None and mt.data_dev
                assert np.array_equal(raw_bytes(ctx, mt.data_dev, data.nbytes), data), name
        with pytest.raises(oracle_amd.OutOfRange):
            model.tensor("no.such.tensor")
    finally:
        model.release()


def test_model_upload_streams_through_staging(ctx, tmp_path):
    """A payload larger than the 256 MiB staging buffer: several staging batches."""
    rng = np.random.default_rng(12)
    rows, cols = 2048, 49152  # 56.6 MB of q4_K per tensor
    tensors = [(f"blk.{i}.ffn_down.weight", [cols, rows], 12, synth.q4_k(rng, rows, cols)) for i in range(6)]
    path = tmp_path / "big.gguf"
    gguf.write(path, tensors)
    model = oracle_amd.Model.from_gguf(ctx, gguf.read(path))
    try:
        for name, dims, t, data in tensors[::5]:
            w = model.tensor(name).weight
            dec = ctx.alloc(3 * cols * 4)
            ctx.dequantize_rows(w, rows - 3, 3, dec)
            got = dec.download(np.float32, 3 * cols).reshape(3, cols)
            rb = synth.row_bytes(t, cols)
            want = oracle.decode_matrix(t, cols, 3, data[(rows - 3) * rb:])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            dec.free()
    finally:
        model.release()
