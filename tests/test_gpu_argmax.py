"""Greedy token over logits in device memory (oq_argmax) against the oracle's greedy token
(src/runtime/sampler.cpp:22-44, src/runtime/qwen35_mtp.cpp:300-308): the same index and value,
bit for bit, including ties, extreme positions, infinities and the sampler's errors."""
import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu


def device_token(ctx, v):
    buf = ctx.to_device(np.ascontiguousarray(v, np.float32))
    try:
        return oracle_amd.greedy_token(ctx, buf, len(v))
    finally:
        buf.free()


@pytest.mark.parametrize("n", [1, 2, 1023, 1024, 1025, 4097, 151936])
def test_random_logits(ctx, n):
    rng = np.random.default_rng(300 + n)
    for _ in range(3):
        v = rng.standard_normal(n).astype(np.float32) * 4
        assert device_token(ctx, v) == oracle.greedy_token(v)


def test_ties_and_positions(ctx):
    rng = np.random.default_rng(301)
    n = 151936
    for pos in (0, 1, 1023, 1024, 65535, n - 2, n - 1):
        v = rng.integers(-50, 50, n).astype(np.float32)
        v[pos] = 100.0
        assert device_token(ctx, v) == (pos, 100.0)
        # a tie later than pos (and one earlier when there is room): the first index wins
        w = v.copy()
        w[(pos + 777) % n] = 100.0
        assert device_token(ctx, w) == oracle.greedy_token(w)
    many = rng.integers(0, 3, n).astype(np.float32)  # the maximum 2.0 at thousands of indices
    assert device_token(ctx, many) == oracle.greedy_token(many)
    assert device_token(ctx, np.full(5000, -7.0, np.float32)) == (0, -7.0)


def test_infinities_and_nan(ctx):
    v = np.full(3000, -np.inf, np.float32)
    v[2500] = -1e30
    assert device_token(ctx, v) == (2500, float(np.float32(-1e30)))
    with pytest.raises(oracle_amd.InvalidArgument, match="no finite"):
        device_token(ctx, np.full(3000, -np.inf, np.float32))
    w = np.zeros(3000, np.float32)
    w[1234] = np.inf
    with pytest.raises(oracle_amd.InvalidArgument, match="no finite"):
        device_token(ctx, w)
    for pos in (0, 1500, 2999):
        x = np.ones(3000, np.float32)
        x[pos] = np.nan
        with pytest.raises(oracle_amd.InvalidArgument, match="NaN"):
            device_token(ctx, x)


def test_argument_errors(ctx):
    buf = ctx.alloc(64)
    tok = ctx.alloc(4)
    with pytest.raises(oracle_amd.InvalidArgument, match="empty"):
        ctx.argmax(buf, 0, tok, tok)
    with pytest.raises(oracle_amd.InvalidArgument, match="token-id range"):
        ctx.argmax(buf, 1 << 32, tok, tok)
    buf.free()
    tok.free()


def test_head_logits_to_token(ctx):
    """Q6_K output head then greedy token on the device: the token is the oracle's greedy token of
    the device's own logits (the logits themselves are checked by the GEMV parity tests)."""
    rng = np.random.default_rng(302)
    rows, cols = 20000, 1024
    data = synth.q6_k(rng, rows, cols)
    w = ctx.upload(14, cols, rows, data)
    xb = ctx.to_device(rng.standard_normal(cols).astype(np.float32))
    yb = ctx.alloc(rows * 4)
    ctx.matvec(w, xb, yb)
    tok = oracle_amd.greedy_token(ctx, yb, rows)
    logits = yb.download(np.float32, rows)
    assert tok == oracle.greedy_token(logits)
    for b in (xb, yb):
        b.free()
    w.release()


def test_argmax_in_graph(ctx):
    rng = np.random.default_rng(303)
    n = 50000
    v = rng.standard_normal(n).astype(np.float32)
    lb, tb, vb = ctx.to_device(v), ctx.alloc(4), ctx.alloc(4)
    ctx.capture_begin()
    ctx.argmax(lb, n, tb, vb)
    g = ctx.capture_end()
    want = oracle.greedy_token(v)
    for rep in range(3):
        tb.upload(np.array([7], np.uint32))
        g.launch()
        ctx.sync()
        assert int(tb.download(np.uint32, 1)[0]) == want[0], rep
        assert float(vb.download(np.float32, 1)[0]) == want[1], rep
    g.destroy()
    for b in (lb, tb, vb):
        b.free()


def fused_head(ctx, w, x, rows):
    """oq_matvec_argmax: (logits, token, value) downloaded."""
    xb, yb, tb, vb = ctx.to_device(np.ascontiguousarray(x, np.float32)), ctx.alloc(rows * 4), ctx.alloc(4), ctx.alloc(4)
    try:
        ctx.matvec_argmax(w, xb, yb, tb, vb)
        return (yb.download(np.float32, rows), int(tb.download(np.uint32, 1)[0]),
                float(vb.download(np.float32, 1)[0]))
    finally:
        for b in (xb, yb, tb, vb):
            b.free()


@pytest.mark.parametrize("t,rows,cols", [(14, 20000, 1024), (12, 4099, 4096), (13, 777, 2048), (14, 151936, 4096),
                                         (12, 33, 12288), (8, 3000, 1024), (14, 5, 256)])
def test_matvec_argmax_equals_two_calls(ctx, t, rows, cols):
    """The head with the greedy token in its epilogue (K-quant weights; other types run the two
    calls): logits bit-identical to oq_matvec, token the first index of their maximum."""
    rng = np.random.default_rng(310 + t + rows)
    data = synth.weights(t, rng, rows, cols)
    w = ctx.upload(t, cols, rows, data)
    x = rng.standard_normal(cols).astype(np.float32)
    y, tok, val = fused_head(ctx, w, x, rows)
    xb, yb = ctx.to_device(x), ctx.alloc(rows * 4)
    ctx.matvec(w, xb, yb)
    y2 = yb.download(np.float32, rows)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    assert (tok, val) == oracle.greedy_token(y2)
    assert oracle_amd.greedy_token(ctx, yb, rows) == (tok, val)
    for b in (xb, yb):
        b.free()
    w.release()


def test_matvec_argmax_ties_and_nan(ctx):
    """Duplicated maximal rows far apart (different workgroups): the first index wins; a NaN
    logit (a weight row with a NaN scale) gives the NaN token."""
    rng = np.random.default_rng(320)
    rows, cols = 40000, 1024
    rb = synth.row_bytes(14, cols)
    data = synth.weights(14, rng, rows, cols).reshape(rows, rb)
    x = rng.standard_normal(cols).astype(np.float32)
    w = ctx.upload(14, cols, rows, data.ravel())
    y, tok, _ = fused_head(ctx, w, x, rows)
    w.release()
    for dup in (tok + 1, rows - 1, 17):
        d2 = data.copy()
        d2[dup] = d2[tok]
        w = ctx.upload(14, cols, rows, d2.ravel())
        y2, tok2, val2 = fused_head(ctx, w, x, rows)
        assert (tok2, val2) == oracle.greedy_token(y2)
        assert tok2 == min(tok, dup)
        w.release()
    d3 = data.copy()
    # q6_K block: ... f16 d at byte 208 of each 210-byte block: NaN scale in row 12345
    d3[12345, 208:210] = np.array([0x00, 0x7E], np.uint8)
    w = ctx.upload(14, cols, rows, d3.ravel())
    y3, tok3, _ = fused_head(ctx, w, x, rows)
    assert np.isnan(y3[12345]) and tok3 == 0xFFFFFFFF
    w.release()
