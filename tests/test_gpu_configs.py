"""GPU parity at the benchmark's own full sizes, seeds and launches (every output row).

- Q4_K FFN gate/up decode GEMV, 12288 x 4096, batch 1, F32 activation quantized to Q8_K inside
  the kernel -- the launch the benchmark times (seed of its q4k_gemv workload);
- Q6_K output head, 151936 x 4096, batch 1 (seed of its q6k_head workload), followed by the greedy
  token on the device (oq_argmax), the head's consumer in the reference
  (src/runtime/qwen35_forward.cpp:450-465, src/runtime/sampler.cpp:22-44).
Bar: |y_gpu - y_ref| <= 1e-4 * sum_k |w_k * xhat_k| for every row, y_ref the oracle's sequential
F32 dot of the decoded row with the dequantized Q8_K activation.
"""
import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = min(16, oracle.default_threads())
SEED = 20261201  # the benchmark's base seed; workload i uses SEED + i


def full_rows_check(ctx, t, rows, cols, seed):
    rng = np.random.default_rng(seed)
    data = synth.weights(t, rng, rows, cols)
    x = synth.activations(rng, 1, cols)[0]
    w = ctx.upload(t, cols, rows, data)
    xb, yb = ctx.to_device(x), ctx.alloc(rows * 4)
    ctx.matvec(w, xb, yb)
    y = yb.download(np.float32, rows)
    xhat = oracle.dequantize_q8k(oracle.quantize_q8k(x), cols)
    y_ref = oracle.storage_matvec(t, rows, cols, data, xhat, threads=THREADS)
    norm = oracle.matvec_stats(t, rows, cols, data, xhat, threads=THREADS)[1]
    err = np.abs(y.astype(np.float64) - y_ref) / np.maximum(norm, 1e-30)
    print(f"type {t} {rows}x{cols}: max normalised error {err.max():.3e}")
    assert np.all(err <= TOL), f"worst row {int(err.argmax())}: {err.max():.3e}"
    xb.free()
    return w, yb, y, y_ref, norm


def test_q4k_gemv_12288x4096_bench_launch(ctx):
    w, yb, *_ = full_rows_check(ctx, 12, 12288, 4096, SEED + 0)
    yb.free()
    w.release()


def test_q6k_head_151936x4096_and_greedy_token(ctx):
    rows = 151936
    w, yb, y, y_ref, norm = full_rows_check(ctx, 14, rows, 4096, SEED + 2)
    tok, val = oracle_amd.greedy_token(ctx, yb, rows)
    # the device's choice over its own logits is exact: first index of the maximum
    assert (tok, val) == oracle.greedy_token(y)
    # the head with the greedy token in its epilogue: the same logits and token
    xb, y2b, tb, vb = ctx.to_device(synth.activations(np.random.default_rng(SEED + 2), 1, 4096)[0]), \
        ctx.alloc(rows * 4), ctx.alloc(4), ctx.alloc(4)
    ctx.matvec_argmax(w, xb, y2b, tb, vb)
    assert int(tb.download(np.uint32, 1)[0]) == oracle.greedy_token(y2b.download(np.float32, rows))[0]
    for b in (xb, y2b, tb, vb):
        b.free()
    # against the oracle's logits: the same token unless the two leading logits are closer than
    # the products' tolerance allows them to be ordered
    tok_ref, _ = oracle.greedy_token(y_ref)
    if tok != tok_ref:
        gap = abs(float(y_ref[tok_ref]) - float(y_ref[tok]))
        assert gap <= TOL * (norm[tok] + norm[tok_ref]), f"token {tok} vs oracle {tok_ref}, gap {gap:.3e}"
    yb.free()
    w.release()
