"""GPU parity through the C ABI against the CPU oracle on identical seeded inputs.

Bars: dequantized rows and Q8_K blocks bit-exact; products within
    |y_gpu - y_ref| <= 1e-4 * sum_k |w_k * xhat_k|   per output,
where y_ref is the reference's sequential F32 dot (oracle) of the decoded row with xhat, the F32
activation (q8_0 and plain rows) or the dequantized Q8_K activation (K-quant rows).
"""

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = min(16, oracle.default_threads())
KQ = (12, 13, 14)


def weights(t, rng, rows, cols):
    if t in (12, 13, 14, 8):
        return synth.weights(t, rng, rows, cols)
    if t == 0:
        return rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    if t == 1:
        return (rng.standard_normal(rows * cols) * 0.1).astype(np.float16).view(np.uint8)
    bits = (rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return bits.view(np.uint8)


def reference_products(t, rows, cols, data, x):
    """Oracle y (F32 sequential dots), normaliser sum|w xhat| per output, for x of shape [m, cols]."""
    x = np.atleast_2d(x)
    ys, norms = [], []
    for xm in x:
        xhat = oracle.dequantize_q8k(oracle.quantize_q8k(xm), cols) if t in KQ else xm
        ys.append(oracle.storage_matvec(t, rows, cols, data, xhat, threads=THREADS))
        norms.append(oracle.matvec_stats(t, rows, cols, data, xhat, threads=THREADS)[1])
    return np.stack(ys), np.stack(norms)


def check_close(y_gpu, y_ref, norm, tol=TOL):
    err = np.abs(y_gpu.astype(np.float64) - y_ref.astype(np.float64))
    bound = tol * np.maximum(norm, 1e-30)
    worst = float(np.max(err / np.maximum(norm, 1e-30)))
    assert np.all(err <= bound), f"max normalised error {worst:.3e} > {tol}"
    return worst


def gpu_matmul(ctx, w, x, rows):
    x = np.atleast_2d(np.ascontiguousarray(x, np.float32))
    xb = ctx.to_device(x)
    yb = ctx.alloc(x.shape[0] * rows * 4)
    if x.shape[0] == 1:
        ctx.matvec(w, xb, yb)
    else:
        ctx.matmul(w, x.shape[0], xb, yb)
    y = yb.download(np.float32, x.shape[0] * rows).reshape(x.shape[0], rows)
    xb.free()
    yb.free()
    return y


# ---------------------------------------------------------------- dequantization (bit-exact)

@pytest.mark.parametrize("t,rows,cols", [
    (12, 37, 4096), (12, 5, 256), (13, 19, 1024), (14, 23, 4096), (14, 3, 768),
    (8, 29, 4096), (8, 4, 96), (0, 7, 33), (1, 9, 1000), (30, 6, 130)])
def test_dequantize_bit_exact(ctx, t, rows, cols):
    rng = np.random.default_rng(1000 + t * 7 + cols)
    data = weights(t, rng, rows, cols)
    w = ctx.upload(t, cols, rows, data)
    out = ctx.alloc(rows * cols * 4)
    ctx.dequantize_rows(w, 0, rows, out)
    got = out.download(np.float32, rows * cols).reshape(rows, cols)
    want = oracle.decode_matrix(t, cols, rows, data)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a row window
    r0, nr = rows // 3, max(1, rows // 2)
    ctx.dequantize_rows(w, r0, nr, out)
    part = out.download(np.float32, nr * cols).reshape(nr, cols)
    assert np.array_equal(part.view(np.uint32), want[r0:r0 + nr].view(np.uint32))
    out.free()
    w.release()


def test_dequantize_golden_vectors(ctx, golden):
    for name in ("q5_k", "q6_k", "q8_0", "q5_k_raw", "q6_k_raw", "q8_0_raw", "q4_k"):
        t = int(golden[f"{name}_type"][0]) if f"{name}_type" in golden else 12
        rows, cols = golden[f"{name}_decoded_bits"].shape
        got = oracle_amd.decode_rows(ctx, t, cols, rows, golden[f"{name}_bytes"])
        assert np.array_equal(got.view(np.uint32), golden[f"{name}_decoded_bits"]), name
    # every binary16 pattern, NaN payloads included
    got = oracle_amd.decode_rows(ctx, 1, 65536, 1, golden["f16_all_bits"].view(np.uint8))
    assert np.array_equal(got.reshape(-1).view(np.uint32), golden["f16_all_decoded_bits"])


def test_dequantize_rejects_rows_out_of_range(ctx):
    rng = np.random.default_rng(5)
    w = ctx.upload(12, 256, 4, synth.q4_k(rng, 4, 256))
    out = ctx.alloc(4 * 256 * 4)
    with pytest.raises(oracle_amd.OutOfRange):
        ctx.dequantize_rows(w, 3, 2, out)
    ctx.dequantize_rows(w, 4, 0, out)  # empty window at the end is fine
    out.free()
    w.release()


# ---------------------------------------------------------------- Q8_K quantization (bit-exact)

def q8k_cases(rng):
    x = rng.standard_normal((5, 1024)).astype(np.float32)
    x[0, :256] = 0.0                                   # all-zero block
    x[1, :256] = 0.0
    x[1, 10], x[1, 200] = -3.0, 3.0                    # tie, first index negative
    x[1, 300], x[1, 301] = 7.0, -7.0                   # tie, first index positive
    x[2, :256] *= 1e-35                                # subnormal-range scale
    x[2, 256:512] *= 1e30
    x[3, :] = np.round(x[3, :] * 4) / 4                # many exact halves after scaling
    x[4, 0:256] = np.linspace(-127, 127, 256, dtype=np.float32)
    return x


def test_quantize_q8k_bit_exact(ctx):
    rng = np.random.default_rng(17)
    x = q8k_cases(rng)
    m, k = x.shape
    xb = ctx.to_device(x)
    qb = ctx.alloc(m * k // 256 * 292)
    ctx.quantize_q8k(xb, m, k, qb)
    got = qb.download(np.uint8)
    want = np.concatenate([oracle.quantize_q8k(row) for row in x])
    assert np.array_equal(got, want)
    xb.free()
    qb.free()


def test_quantize_q8k_rejects_ragged(ctx):
    xb = ctx.alloc(300 * 4)
    qb = ctx.alloc(292 * 2)
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.quantize_q8k(xb, 1, 300, qb)
    xb.free()
    qb.free()


# ---------------------------------------------------------------- products (tolerance)

@pytest.mark.parametrize("t,rows,cols", [
    (12, 301, 4096), (12, 64, 256), (12, 17, 768), (12, 40, 12288),
    (13, 77, 4096), (14, 129, 4096), (14, 33, 512), (14, 16, 12288),
    (8, 203, 4096), (8, 20, 96), (0, 33, 100), (1, 31, 1000), (30, 10, 512)])
def test_matvec_tolerance(ctx, t, rows, cols):
    rng = np.random.default_rng(2000 + t + rows)
    data = weights(t, rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(y, y_ref, norm)
    w.release()


@pytest.mark.parametrize("t", KQ)
def test_matvec_q8k_matches_integer_oracle(ctx, t):
    rng = np.random.default_rng(31 + t)
    rows, cols = 96, 2048
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    q8 = oracle.quantize_q8k(x)
    w = ctx.upload(t, cols, rows, data)
    qb = ctx.to_device(q8)
    yb = ctx.alloc(rows * 4)
    ctx.matvec_q8k(w, qb, yb)
    y = yb.download(np.float32, rows)
    ints = np.array([oracle.vec_dot_q8k(t, cols, r, q8) for r in data.reshape(rows, -1)], np.float32)
    _, norm = oracle.matvec_stats(t, rows, cols, data, oracle.dequantize_q8k(q8, cols), threads=THREADS)
    check_close(y, ints, norm, tol=2e-6)
    for b in (qb, yb):
        b.free()
    w.release()


@pytest.mark.parametrize("t", KQ)
@pytest.mark.parametrize("cols", [256, 4096, 8192, 12288, 16384])
def test_fused_quantization_is_bit_identical(ctx, t, cols):
    """F32 activations quantized inside the GEMV give exactly the result of the same GEMV fed with
    the standalone quantizer's Q8_K blocks (same integer sums, same float operations)."""
    rng = np.random.default_rng(500 + t + cols)
    rows = 97
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    x[:256] = np.where(np.arange(256) % 3 == 0, 0.0, x[:256])
    x[17], x[200] = 5.5, -5.5  # |x| tie inside the first super-block
    w = ctx.upload(t, cols, rows, data)
    xb = ctx.to_device(x)
    qb = ctx.alloc(cols // 256 * 292)
    y1 = ctx.alloc(rows * 4)
    y2 = ctx.alloc(rows * 4)
    ctx.matvec(w, xb, y1)
    ctx.quantize_q8k(xb, 1, cols, qb)
    ctx.matvec_q8k(w, qb, y2)
    a = y1.download(np.float32, rows)
    b = y2.download(np.float32, rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(a, y_ref[0], norm[0])
    for buf in (xb, qb, y1, y2):
        buf.free()
    w.release()


@pytest.mark.parametrize("t", [12, 14, 8])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8, 11])
def test_matmul_small_batch(ctx, t, m):
    rng = np.random.default_rng(400 + 10 * t + m)
    rows, cols = 130, 2048
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(y, y_ref, norm)
    w.release()


@pytest.mark.parametrize("m,rows,cols", [(16, 256, 4096), (37, 300, 4096), (64, 130, 12288), (200, 128, 8192)])
def test_matmul_matrix_cores(ctx, m, rows, cols):
    """m >= 16 q4_K products run on the F16 MFMA path; same tolerance as every other product."""
    rng = np.random.default_rng(900 + m + rows)
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(12, rows, cols, data, x)
    worst = check_close(y, y_ref, norm)
    assert worst < 0.5 * TOL, f"MFMA path margin too thin: {worst:.2e}"
    w.release()


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("splits", [None, "1", "3", "8"])
def test_matrix_cores_q8k_input_and_split_counts(ctx, t, splits):
    """The MFMA path (every K-quant type: weights converted in the MFMA waves) from caller-supplied
    Q8_K blocks equals the path from F32 activations bit for bit (same planar image), and every
    K-split count stays within the tolerance."""
    rng = np.random.default_rng(31337 + t)
    m, rows, cols = 70, 520, 8192
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    with oracle_amd.launch_options({} if splits is None else {"OQ_GEMM_SPLITS": splits}):
        y = gpu_matmul(ctx, w, x, rows)
        xb = ctx.to_device(x)
        qb = ctx.alloc(m * (cols // 256) * 292)
        yb = ctx.alloc(m * rows * 4)
        ctx.quantize_q8k(xb, m, cols, qb)
        ctx.matmul_q8k(w, m, qb, yb)
        y_q8k = yb.download(np.float32, m * rows).reshape(m, rows)
        for b in (xb, qb, yb):
            b.free()
    assert np.array_equal(y.view(np.uint32), y_q8k.view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    worst = check_close(y, y_ref, norm)
    assert worst < 0.5 * TOL, f"MFMA path margin too thin: {worst:.2e}"
    w.release()


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("env", [{}, {"OQ_GEMM_WS": "2"}])
def test_matrix_cores_extreme_activation_scales(ctx, t, env):
    """The matrix-core path's f16 activation image carries one power-of-two exponent per row, so
    rows far outside binary16's range (1e5 and 3e6 scales: |d q| > 65504) and far below it (1e-6,
    1e-30: subnormal or zero in binary16) stay finite, from F32 and from Q8_K inputs, in every
    kernel.  Rows whose sum spreads over many products meet the 1e-4 bar.  A row dominated by a
    few products (one element at 3e6, one block at 1e5 times the rest) is held to the path's
    rigorous bound instead: each operand rounded once to binary16 (relative 2^-11), so each
    product is off by at most about 2^-10 of itself, plus F32 summation: 2e-3 of sum |w xhat|
    (a missing or doubled row exponent would be off by a power of two)."""
    rng = np.random.default_rng(5150 + t)
    m, rows, cols = 24, 300, 4096
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    x[0] *= 1e5
    x[1] *= 1e-6
    x[2] *= 1e-30
    x[3, 17] = 3e6           # one huge element; the rest of the row quantizes to small integers
    x[4] = 0.0               # an all-zero row
    x[5, :256] *= 1e5        # one block far above the others
    w = ctx.upload(t, cols, rows, data)
    with oracle_amd.launch_options(env):
        y = gpu_matmul(ctx, w, x, rows)
        xb = ctx.to_device(x)
        qb = ctx.alloc(m * (cols // 256) * 292)
        yb = ctx.alloc(m * rows * 4)
        ctx.quantize_q8k(xb, m, cols, qb)
        ctx.matmul_q8k(w, m, qb, yb)
        y_q8k = yb.download(np.float32, m * rows).reshape(m, rows)
        for b in (xb, qb, yb):
            b.free()
    assert np.all(np.isfinite(y))
    assert np.array_equal(y.view(np.uint32), y_q8k.view(np.uint32))
    assert np.all(y[4] == 0.0)
    y_ref, norm = reference_products(t, rows, cols, data, x)
    for r in range(m):
        if r == 4:
            continue
        check_close(y[r:r + 1], y_ref[r:r + 1], norm[r:r + 1], tol=2e-3 if r in (3, 5) else TOL)
    w.release()


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("cols", [8192, 12288])
@pytest.mark.parametrize("env", [{}, {"OQ_GEMM_WS": "2"}])
def test_matrix_cores_bound_on_dominated_rows(ctx, t, cols, env):
    """Rows that a few products dominate, at the long K of down projections: a saturated SwiGLU
    output silu(g) * u with gate values N(-200, 80) (at least -85), rows of log-normal magnitudes
    (log-scale deviations 10 and 20) and a row with one non-zero element per block, so that one
    element leads each Q8_K block by a wide factor and a few blocks lead the row.  Every output
    stays within the path's bound, about 2^-10 of sum |w xhat| (1.5e-3 here: 2^-10 plus
    binary16-subnormal weights and F32 summation; an ideal one-rounding product reaches 2e-4 to
    7e-4 on these rows).  Each weight is the reference's F32 value rounded once to f16: rounding
    the q4_K / q5_K scale and min to f16 first puts the error of a weight that is the small
    difference of its two terms relative to those terms, which such rows expose."""
    rng = np.random.default_rng(7100 + t + cols)
    m, rows = 16, 256
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    g = np.maximum(rng.normal(-200.0, 80.0, cols), -85.0)
    x[0] = (g / (1.0 + np.exp(-g)) * rng.standard_normal(cols) * 100.0).astype(np.float32)
    for r, s in ((1, 10.0), (2, 20.0)):
        x[r] = (np.exp(np.clip(s * rng.standard_normal(cols), -80.0, 60.0)) * rng.standard_normal(cols)).astype(np.float32)
    x[3] = 0.0
    x[3, np.arange(0, cols, 256) + rng.integers(0, 256, cols // 256)] = rng.standard_normal(cols // 256)
    w = ctx.upload(t, cols, rows, data)
    with oracle_amd.launch_options(env):
        y = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(t, rows, cols, data, x)
    for r in range(4):
        check_close(y[r:r + 1], y_ref[r:r + 1], norm[r:r + 1], tol=1.5e-3)
    check_close(y[4:], y_ref[4:], norm[4:])
    w.release()


@pytest.mark.parametrize("m,rows,cols,splits", [(70, 520, 8192, None), (16, 33, 4096, None), (130, 300, 4096, "3"),
                                                (40, 257, 12288, "1"), (33, 64, 8192, "8")])
def test_q8_0_matrix_cores(ctx, m, rows, cols, splits):
    """q8_0 weights at m >= 16 run on matrix cores: the F32 activations rounded once to f16 (with
    the row exponent), weights f16(d q), F32 accumulation; within the product bar of the
    reference's F32 dot (src/backend/cpu/quantized_reference.cpp:50-64), tails in m and n, every
    split count, and against the integer-free GEMV path (OQ_GEMM_MFMA=0) within the same bar."""
    rng = np.random.default_rng(8800 + m + rows + cols)
    data = synth.q8_0(rng, rows, cols)
    blocks = data.reshape(-1, 34)
    blocks[rng.integers(0, blocks.shape[0], 50), 2 + rng.integers(0, 32, 50)] = 0x80  # q = -128 too
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(8, cols, rows, data)
    with oracle_amd.launch_options({} if splits is None else {"OQ_GEMM_SPLITS": splits}):
        y = gpu_matmul(ctx, w, x, rows)
    with oracle_amd.launch_options({"OQ_GEMM_MFMA": "0"}):
        y_gemv = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(8, rows, cols, data, x)
    worst = check_close(y, y_ref, norm)
    assert worst < 0.5 * TOL, f"MFMA path margin too thin: {worst:.2e}"
    check_close(y_gemv, y_ref, norm)
    assert not np.array_equal(y, y_gemv)  # the two paths really differ (f16 operands)
    w.release()


def test_q8_0_prefill_full_size_sampled_rows(ctx):
    """The MTP hidden projection's shape (nextn.eh_proj, q8_0, 2 x 4096 -> 4096,
    src/model/qwen35_weights.cpp:53-58) at M = 512: every output of 24 sampled activation rows."""
    rng = np.random.default_rng(8812)
    rows, cols, m = 4096, 8192, 512
    data = synth.q8_0(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(8, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    pick = np.array(sorted(set([0, 1, 255, 256, 511] + list(rng.integers(0, m, 19)))))
    y_ref, norm = reference_products(8, rows, cols, data, x[pick])
    check_close(y[pick], y_ref, norm)
    assert np.all(np.isfinite(y))
    w.release()


def test_q8_0_matrix_cores_extreme_activation_scales(ctx):
    """The q8_0 image scales each F32 row by a power of two into binary16's range: rows at 1e5
    and 1e-30 times N(0, 1) stay finite and within the bar; a row dominated by one element is
    held to the rigorous 2e-3 bound (see test_matrix_cores_extreme_activation_scales)."""
    rng = np.random.default_rng(8813)
    m, rows, cols = 20, 200, 4096
    data = synth.q8_0(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    x[0] *= 1e5
    x[1] *= 1e-30
    x[2, 5] = 7e6
    x[3] = 0.0
    w = ctx.upload(8, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    assert np.all(np.isfinite(y)) and np.all(y[3] == 0.0)
    y_ref, norm = reference_products(8, rows, cols, data, x)
    for r in range(m):
        if r != 3:
            check_close(y[r:r + 1], y_ref[r:r + 1], norm[r:r + 1], tol=2e-3 if r == 2 else TOL)
    w.release()


@pytest.mark.parametrize("cols", [4096, 8192])
def test_matrix_core_kernels_agree(ctx, cols):
    """The producer/consumer GEMM kernel (default) and the four-wave kernel (OQ_GEMM_WS=0)
    accumulate the same f16 operands in the same order: identical outputs, bit for bit."""
    rng = np.random.default_rng(2718 + cols)
    m, rows = 70, 520
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    ys = {}
    for v in ("1", "0", "2"):
        with oracle_amd.launch_options({"OQ_GEMM_WS": v}):
            ys[v] = gpu_matmul(ctx, w, x, rows)
    assert np.array_equal(ys["1"].view(np.uint32), ys["0"].view(np.uint32))
    # the kernel whose load waves convert the weights into LDS B tiles (the q5_K / q6_K path)
    assert np.array_equal(ys["1"].view(np.uint32), ys["2"].view(np.uint32))
    y_ref, norm = reference_products(12, rows, cols, data, x)
    check_close(ys["1"], y_ref, norm)
    w.release()


@pytest.mark.parametrize("t", [13, 14])
@pytest.mark.parametrize("cols", [4096, 8192])
def test_q5_q6_matrix_core_kernels_agree(ctx, t, cols):
    """q5_K and q6_K: the kernel whose MFMA waves convert the weights in registers (default) and
    the one whose load waves convert them into LDS B tiles (OQ_GEMM_WS=2) form the same f16
    operands and add them in the same order: identical outputs, bit for bit, on both
    dequantization paths (F32 scales below K = 8192, packed f16 from 8192)."""
    rng = np.random.default_rng(5150 + 7 * t + cols)
    m, rows = 70, 520
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    ys = {}
    for v in ("1", "2"):
        with oracle_amd.launch_options({"OQ_GEMM_WS": v}):
            ys[v] = gpu_matmul(ctx, w, x, rows)
    assert np.array_equal(ys["1"].view(np.uint32), ys["2"].view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(ys["1"], y_ref, norm)
    w.release()


@pytest.mark.parametrize("t", [13, 14])
@pytest.mark.parametrize("m,rows,cols", [(16, 256, 4096), (37, 300, 4096), (64, 130, 12288), (200, 128, 8192),
                                         (19, 70, 17408), (130, 513, 4352)])
def test_matmul_matrix_cores_q5_q6(ctx, t, m, rows, cols):
    """m >= 16 q5_K / q6_K products on the f16 MFMA path (weights converted in the MFMA waves'
    registers); Q8_K and F32 activations give the same bits."""
    rng = np.random.default_rng(9500 + 7 * t + m + rows + cols)
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    xb, qb, yb = ctx.to_device(x), ctx.alloc(m * (cols // 256) * 292), ctx.alloc(m * rows * 4)
    ctx.quantize_q8k(xb, m, cols, qb)
    ctx.matmul_q8k(w, m, qb, yb)
    y_q8k = yb.download(np.float32, m * rows).reshape(m, rows)
    for b in (xb, qb, yb):
        b.free()
    assert np.array_equal(y.view(np.uint32), y_q8k.view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    worst = check_close(y, y_ref, norm)
    assert worst < 0.5 * TOL, f"MFMA path margin too thin: {worst:.2e}"
    w.release()


@pytest.mark.parametrize("t", [13, 14])
def test_prefill_gemm_q5_q6_full_size_sampled_rows(ctx, t):
    """4096 x 12288 q5_K / q6_K down projections at M = 512, 24 sampled activation rows."""
    rng = np.random.default_rng(4244 + t)
    rows, cols, m = 4096, 12288, 512
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    pick = np.array(sorted(set([0, 1, 255, 256, 511] + list(rng.integers(0, m, 19)))))
    y_ref, norm = reference_products(t, rows, cols, data, x[pick])
    check_close(y[pick], y_ref, norm)
    assert np.all(np.isfinite(y))
    w.release()


def test_prefill_gemm_full_size_sampled_rows(ctx):
    """The 4096 x 12288 q4_K down projection at M = 512: every output of 24 sampled activation
    rows against the oracle (the rows are computed inside the full 512-row product)."""
    rng = np.random.default_rng(4242)
    rows, cols, m = 4096, 12288, 512
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    pick = np.array(sorted(set([0, 1, 255, 256, 511] + list(rng.integers(0, m, 19)))))
    y_ref, norm = reference_products(12, rows, cols, data, x[pick])
    check_close(y[pick], y_ref, norm)
    assert np.all(np.isfinite(y))
    w.release()


@pytest.mark.parametrize("env", [{"OQ_GEMV_ROWS": "2"}, {"OQ_FUSED_QUANT": "0"}, {"OQ_GEMV_MAX_WG": "7"},
                                 {"OQ_GEMV_STREAM": "1"}, {"OQ_GEMV_STREAM": "1", "OQ_STREAM_WAVES": "8"},
                                 {"OQ_GEMV_STREAM": "0"}])
def test_launch_variants_agree(ctx, env):
    rng = np.random.default_rng(77)
    rows, cols = 211, 4096
    results = {}
    for t in KQ:
        data = synth.weights(t, rng, rows, cols)
        x = rng.standard_normal((3, cols)).astype(np.float32)
        w = ctx.upload(t, cols, rows, data)
        base = gpu_matmul(ctx, w, x, rows)
        with oracle_amd.launch_options(env):
            var = gpu_matmul(ctx, w, x, rows)
        y_ref, norm = reference_products(t, rows, cols, data, x)
        check_close(var, y_ref, norm)
        results[t] = np.max(np.abs(var - base))
        w.release()


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (17, 4096), (5000, 1024), (9000, 2048), (8300, 4096)])
def test_q8_0_decode_gemv(ctx, rows, cols):
    """The q8_0 decode kernel (16-wave workgroups, x staged once per workgroup, several rows per
    wave when the rows outnumber the waves) against the oracle and against the general q8_0
    kernel (OQ_Q8_0_ROWS=0); outputs are poisoned with NaN before each launch."""
    rng = np.random.default_rng(880 + rows + cols)
    data = synth.q8_0(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ctx.upload(8, cols, rows, data)
    xb = ctx.to_device(x)
    yb = ctx.alloc(rows * 4)
    runs = []
    for flag in ("1", "0"):
        with oracle_amd.launch_options({"OQ_Q8_0_ROWS": flag}):
            yb.upload(np.full(rows, np.nan, np.float32))
            ctx.matvec(w, xb, yb)
            ctx.sync()
        runs.append(yb.download(np.float32, rows))
    y_ref, norm = reference_products(8, rows, cols, data, x)
    for r in runs:
        check_close(r, y_ref[0], norm[0])
    xb.free()
    yb.free()
    w.release()


@pytest.mark.parametrize("t,rows,cols,m", [(12, 4096, 12288, 4), (12, 5000, 1280, 3), (13, 700, 4096, 2),
                                           (14, 8269, 512, 8), (14, 300, 8192, 5), (12, 9000, 4096, 7),
                                           (12, 4096, 12288, 8), (14, 2000, 12288, 6), (13, 900, 12288, 7)])
def test_small_batch_streamed_kernel(ctx, t, rows, cols, m):
    """Small batches run the streamed kernel (one weight pass in flight per wave, m activation
    rows in LDS); it gives the batched kernel's bits (OQ_GEMV_STREAM_MT=0), also when it
    quantizes the F32 rows itself (OQ_FUSED_QUANT=1), including several rows per wave, K not a
    multiple of 4096 and m below the tier size."""
    rng = np.random.default_rng(6060 + t + rows + m)
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    xb = ctx.to_device(x)
    yb = ctx.alloc(m * rows * 4)
    runs = []
    # streamed, batched, and streamed with the quantization inside the kernel's staging
    for env in ({"OQ_GEMV_STREAM_MT": "1"}, {"OQ_GEMV_STREAM_MT": "0"},
                {"OQ_GEMV_STREAM_MT": "1", "OQ_FUSED_QUANT": "1"}):
        with oracle_amd.launch_options(env):
            yb.upload(np.full(m * rows, np.nan, np.float32))
            ctx.matmul(w, m, xb, yb)
            ctx.sync()
        runs.append(yb.download(np.float32, m * rows).reshape(m, rows))
    for r in runs[1:]:
        assert np.array_equal(runs[0].view(np.uint32), r.view(np.uint32))
    pick = np.array(sorted(set([0, m - 1])))
    y_ref, norm = reference_products(t, rows, cols, data, x[pick])
    check_close(runs[0][pick], y_ref, norm)
    xb.free()
    yb.free()
    w.release()


def test_matvec_deterministic(ctx):
    rng = np.random.default_rng(8)
    rows, cols = 1000, 4096
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    a = gpu_matmul(ctx, w, x, rows)
    b = gpu_matmul(ctx, w, x, rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    w.release()


@pytest.mark.parametrize("t,rows,cols", [(12, 8269, 512), (12, 8269, 4096), (12, 12293, 4096), (13, 8269, 512),
                                         (14, 12293, 512), (12, 8269, 12288)])
def test_decode_gemv_many_rows_per_wave(ctx, t, rows, cols):
    # Several rows per wave (and a ragged last round), through the streamed and the batched
    # decode kernels: each row is computed on every launch (outputs are poisoned with NaN before
    # each), with the same bits.
    rng = np.random.default_rng(4242 + t + rows + cols)
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    xb = ctx.to_device(x)
    yb = ctx.alloc(rows * 4)
    runs = []
    for env in ({}, {"OQ_GEMV_STREAM": "1"}, {"OQ_GEMV_STREAM": "0"}, {"OQ_GEMV_STREAM": "1"},
                {"OQ_GEMV_STREAM": "0", "OQ_GEMV_ROWS": "1"}):
        with oracle_amd.launch_options(env):
            yb.upload(np.full(rows, np.nan, np.float32))
            ctx.matvec(w, xb, yb)
            ctx.sync()
        runs.append(yb.download(np.float32, rows))
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(runs[0], y_ref, norm)
    xb.free()
    yb.free()
    w.release()


def test_decode_gemv_many_rows_in_graph(ctx):
    rng = np.random.default_rng(4343)
    rows, cols = 12293, 512
    ws = [ctx.upload(t, cols, rows, synth.weights(t, rng, rows, cols)) for t in KQ]
    xb = ctx.to_device(rng.standard_normal(cols).astype(np.float32))
    ybs = [ctx.alloc(rows * 4) for _ in ws]
    for w, yb in zip(ws, ybs):
        ctx.matvec(w, xb, yb)
    ctx.sync()
    eager = [yb.download(np.float32, rows) for yb in ybs]
    ctx.capture_begin()
    for w, yb in zip(ws, ybs):
        ctx.matvec(w, xb, yb)
    g = ctx.capture_end()
    for rep in range(3):
        for yb in ybs:
            ctx.matvec(ws[1], xb, ybs[1])
            yb.upload(np.full(rows, np.nan, np.float32))
        g.launch()
        ctx.sync()
        for e, yb in zip(eager, ybs):
            assert np.array_equal(yb.download(np.float32, rows).view(np.uint32), e.view(np.uint32)), rep
    g.destroy()
    for b in ybs + [xb]:
        b.free()
    for w in ws:
        w.release()


# ---------------------------------------------------------------- argument errors through the ABI

def test_abi_argument_errors(ctx):
    rng = np.random.default_rng(9)
    data = synth.q4_k(rng, 4, 512)
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.upload(12, 512, 4, data[:-1])                # byte size mismatch
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.upload(12, 512, 0, data)                     # zero rows
    with pytest.raises(oracle_amd.UnsupportedType):
        ctx.upload(12, 500, 4, data)                     # ragged row
    with pytest.raises(oracle_amd.UnsupportedType):
        ctx.upload(99, 512, 4, data)                     # unregistered type
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.upload(2, 512, 4, np.zeros(4 * 16 * 18, np.uint8))  # q4_0: registered, not decodable
    w8 = ctx.upload(8, 512, 4, synth.q8_0(rng, 4, 512))
    qb = ctx.alloc(2 * 292)
    yb = ctx.alloc(16)
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.matvec_q8k(w8, qb, yb)                       # Q8_K activations need a K-quant weight
    w4 = ctx.upload(12, 512, 4, data)
    xb = ctx.alloc(512 * 4 + 16)

    class Shifted:
        ptr = xb.ptr + 4
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.matvec(w4, Shifted, yb)                      # misaligned activations
    with pytest.raises(oracle_amd.InvalidArgument):
        ctx.matmul(w4, 0, xb, yb)
    for b in (qb, yb, xb):
        b.free()
    w8.release()
    w4.release()


# ---------------------------------------------------------------- graph replay

def test_graph_replay_matches_eager(ctx):
    rng = np.random.default_rng(21)
    rows, cols = 512, 4096
    ws = [ctx.upload(t, cols, rows, synth.weights(t, rng, rows, cols)) for t in (12, 14, 8)]
    x = rng.standard_normal(cols).astype(np.float32)
    xb = ctx.to_device(x)
    ybs = [ctx.alloc(rows * 4) for _ in ws]
    for w, yb in zip(ws, ybs):
        ctx.matvec(w, xb, yb)
    ctx.sync()
    eager = [yb.download(np.float32, rows) for yb in ybs]
    ctx.capture_begin()
    for w, yb in zip(ws, ybs):
        ctx.matvec(w, xb, yb)
    g = ctx.capture_end()
    for rep in range(3):
        for yb in ybs:  # clobber outputs with eager work between replays
            ctx.matvec(ws[0], xb, ybs[0])
            yb.upload(np.full(rows, np.nan, np.float32))
        g.launch()
        ctx.sync()
        for e, yb in zip(eager, ybs):
            assert np.array_equal(yb.download(np.float32, rows).view(np.uint32), e.view(np.uint32)), rep
    g.destroy()
    for b in ybs + [xb]:
        b.free()
    for w in ws:
        w.release()


def test_graph_replay_after_workspace_growth(ctx):
    """A graph keeps replaying the staging buffer it captured after an eager call grew the
    context's buffer (the old allocation is retired, not freed, while the graph lives)."""
    rng = np.random.default_rng(6060)
    rows, cols, m = 640, 4096, 4
    data = synth.q4_k(rng, rows, cols)
    w = ctx.upload(12, cols, rows, data)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    xb, yb = ctx.to_device(x), ctx.alloc(m * rows * 4)
    ctx.matmul(w, m, xb, yb)  # sizes the small staging buffer
    ctx.sync()
    eager = yb.download(np.float32, m * rows)
    ctx.capture_begin()
    ctx.matmul(w, m, xb, yb)
    g = ctx.capture_end()
    big = 256  # the matrix-core path needs a much larger buffer: the context grows it
    xbig = ctx.to_device(rng.standard_normal((big, cols)).astype(np.float32))
    ybig = ctx.alloc(big * rows * 4)
    ctx.matmul(w, big, xbig, ybig)
    ctx.sync()
    for _ in range(3):
        yb.upload(np.full(m * rows, np.nan, np.float32))
        g.launch()
        ctx.sync()
        assert np.array_equal(yb.download(np.float32, m * rows).view(np.uint32), eager.view(np.uint32))
        ctx.matmul(w, big, xbig, ybig)  # eager work on the grown buffer between replays
        ctx.sync()
    g.destroy()
    ctx.matmul(w, m, xb, yb)
    ctx.sync()
    assert np.array_equal(yb.download(np.float32, m * rows).view(np.uint32), eager.view(np.uint32))
    for b in (xb, yb, xbig, ybig):
        b.free()
    w.release()


@pytest.mark.parametrize("t,rows,cols,m", [
    (12, 700, 17408, 1), (12, 300, 17408, 3), (13, 257, 24576, 1), (14, 333, 24576, 2), (12, 130, 65536, 1),
    (14, 90, 65536, 5), (13, 64, 17408, 8), (12, 4096, 17408, 1)])
def test_long_rows(ctx, t, rows, cols, m):
    """K-quant rows longer than 16384 elements (the reference's dot has no length limit,
    src/backend/cpu/quantized_reference.cpp:128-162): windows of passes multiplied by consecutive
    launches, each adding its partial sums; F32 and Q8_K activations give the same bits."""
    rng = np.random.default_rng(7000 + t + cols + m)
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(t, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    xb, qb, yb = ctx.to_device(x), ctx.alloc(m * (cols // 256) * 292), ctx.alloc(m * rows * 4)
    ctx.quantize_q8k(xb, m, cols, qb)
    yb.upload(np.full(m * rows, np.nan, np.float32))
    ctx.matmul_q8k(w, m, qb, yb)
    y_q8k = yb.download(np.float32, m * rows).reshape(m, rows)
    for b in (xb, qb, yb):
        b.free()
    assert np.array_equal(y.view(np.uint32), y_q8k.view(np.uint32))
    y_ref, norm = reference_products(t, rows, cols, data, x)
    check_close(y, y_ref, norm)
    w.release()


def test_long_rows_matrix_cores(ctx):
    """The M >= 16 q4_K product on matrix cores with K = 17408 (not a multiple of 4096)."""
    rng = np.random.default_rng(7171)
    rows, cols, m = 256, 17408, 32
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    y = gpu_matmul(ctx, w, x, rows)
    y_ref, norm = reference_products(12, rows, cols, data, x)
    check_close(y, y_ref, norm)
    w.release()


@pytest.mark.parametrize("m,rows,cols", [(16, 256, 4096), (37, 300, 4096), (64, 130, 12288), (200, 128, 8192),
                                         (19, 70, 17408)])
def test_matmul_int8_matrix_cores(ctx, m, rows, cols):
    """The int8 MFMA alternative (OQ_GEMM_INT8=1): Q8_K x nibble sub-block products rescaled in
    int32, min correction on f16 matrix cores; F32 and Q8_K activations give the same bits."""
    rng = np.random.default_rng(8100 + m + rows + cols)
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    with oracle_amd.launch_options({"OQ_GEMM_INT8": "1"}):
        y = gpu_matmul(ctx, w, x, rows)
        xb, qb, yb = ctx.to_device(x), ctx.alloc(m * (cols // 256) * 292), ctx.alloc(m * rows * 4)
        ctx.quantize_q8k(xb, m, cols, qb)
        ctx.matmul_q8k(w, m, qb, yb)
        y_q8k = yb.download(np.float32, m * rows).reshape(m, rows)
        for b in (xb, qb, yb):
            b.free()
    assert np.array_equal(y.view(np.uint32), y_q8k.view(np.uint32))
    y_ref, norm = reference_products(12, rows, cols, data, x)
    worst = check_close(y, y_ref, norm)
    # the products are exact integers scaled in F32: far inside the bar
    assert worst < 1e-5, worst
    w.release()


def test_matmul_int8_full_size_sampled_rows(ctx):
    rng = np.random.default_rng(4243)
    rows, cols, m = 4096, 12288, 512
    data = synth.q4_k(rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    w = ctx.upload(12, cols, rows, data)
    with oracle_amd.launch_options({"OQ_GEMM_INT8": "1"}):
        y = gpu_matmul(ctx, w, x, rows)
    pick = np.array(sorted(set([0, 1, 127, 128, 511] + list(rng.integers(0, m, 11)))))
    y_ref, norm = reference_products(12, rows, cols, data, x[pick])
    check_close(y[pick], y_ref, norm)
    w.release()
