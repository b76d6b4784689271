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
