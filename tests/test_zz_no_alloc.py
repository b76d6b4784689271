"""oq_deltanet_step_noalloc (the allocation-free entry point) against oq_deltanet_step, through
the C ABI: the same kernels on a fixed per-GPU workspace, so every output must be identical bit
for bit -- y, the traced intermediates, the updated state and convolution history -- on two calls
in a row, the second with a smaller block; a block too large for the fixed workspace is refused;
the entry point can be captured into a graph with no eager call before it."""
import ctypes as C

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu

SMALL = dict(synth.DELTANET_DIMS, embedding=1024, key_heads=2, value_heads=4, ffn=1536)


def step_both(ctx, dims, seed):
    d, w, vec, hist, st, x = synth.deltanet_block(np.random.default_rng(seed), dims)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    n_trace = sum(oracle.deltanet_trace_sizes(d).values())
    E = d["embedding"]
    out = {}
    try:
        xb = ctx.to_device(x)
        for which in ("step", "noalloc"):
            hb, sb = ctx.to_device(hist), ctx.to_device(st)
            yb, tb = ctx.alloc(E * 4), ctx.alloc(n_trace * 4)
            yb.upload(np.full(E, np.nan, np.float32))
            tb.upload(np.full(n_trace, np.nan, np.float32))
            if which == "step":
                ctx.deltanet_step(blk, hb, sb, xb, yb, tb)
            else:
                rc = ctx.lib.oq_deltanet_step_noalloc(ctx.h, C.byref(blk.desc), hb.ptr, sb.ptr, xb.ptr, yb.ptr, tb.ptr)
                assert rc == 0, ctx.lib.oq_last_error(ctx.h).decode()
            ctx.sync()
            out[which] = [b.download(np.float32, n).view(np.uint32) for b, n in
                          ((yb, E), (tb, n_trace), (sb, st.size), (hb, hist.size))]
            for b in (hb, sb, yb, tb):
                b.free()
        xb.free()
    finally:
        blk.release()
    for name, a, b in zip(("y", "trace", "state", "history"), out["step"], out["noalloc"]):
        assert np.array_equal(a, b), name
    assert not np.any(np.isnan(out["noalloc"][0].view(np.float32)))


def test_noalloc_matches_step_two_calls(ctx):
    # full-size block (hidden 4096, FFN 12288), then a smaller one on the same GPU array
    step_both(ctx, synth.DELTANET_DIMS, 71)
    step_both(ctx, SMALL, 72)


def test_noalloc_matches_step_any_shape(ctx):
    # key heads of 16 and value heads of 32: the per-stage launches with the any-shape delta rule
    step_both(ctx, dict(SMALL, key_dim=16, value_dim=32, value_heads=8, conv_kernel=3), 74)


def test_noalloc_rejects_block_beyond_capacity(ctx):
    cap = int(ctx.lib.oq_deltanet_noalloc_capacity())
    assert cap == 4 << 20
    d, w, vec, hist, st, x = synth.deltanet_block(np.random.default_rng(73), SMALL)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        hb, sb, xb, yb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(x), ctx.alloc(d["embedding"] * 4)
        blk.desc.ffn = cap // 4  # the FFN fields alone would need 3 * cap bytes
        rc = ctx.lib.oq_deltanet_step_noalloc(ctx.h, C.byref(blk.desc), hb.ptr, sb.ptr, xb.ptr, yb.ptr, None)
        assert rc == oracle_amd._lib.OQ_INVALID_ARGUMENT
        assert "exceeds" in ctx.lib.oq_last_error(ctx.h).decode()
        for b in (hb, sb, xb, yb):
            b.free()
    finally:
        blk.release()


def test_noalloc_captured_without_eager_call(ctx):
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(74), SMALL)
    rng = np.random.default_rng(75)
    xs = [rng.standard_normal(d["embedding"]).astype(np.float32) for _ in range(3)]
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        he, se, hg, sg = (ctx.to_device(a) for a in (hist, st, hist, st))
        xb, yg, ye = ctx.alloc(d["embedding"] * 4), ctx.alloc(d["embedding"] * 4), ctx.alloc(d["embedding"] * 4)
        ctx.capture_begin()
        ctx.deltanet_step_noalloc(blk, hg, sg, xb, yg)
        g = ctx.capture_end()
        for x in xs:
            xb.upload(x)
            ctx.deltanet_step(blk, he, se, xb, ye)
            ctx.sync()
            g.launch()
            ctx.sync()
            assert np.array_equal(ye.download(np.float32, d["embedding"]), yg.download(np.float32, d["embedding"]))
        assert np.array_equal(se.download(np.float32, st.size), sg.download(np.float32, st.size))
        g.destroy()
        for b in (he, se, hg, sg, xb, yg, ye):
            b.free()
    finally:
        blk.release()
