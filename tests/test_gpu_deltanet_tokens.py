"""GPU parity of the multi-token Gated DeltaNet step (oq_deltanet_steps): m consecutive tokens
through one block, against the oracle's restatement of the reference block
(qwen35_block.cpp:406-605) applied token by token, as the reference's multi-token evaluation does
(src/runtime/qwen35_target_multi.cpp:14-25).

Stage by stage per token, as tests/test_gpu_deltanet.py checks the single step: each traced stage
against the oracle's computation of it from the device's own inputs to it.  The convolution
history before token t follows exactly from the history before the call and the device's traced
q/k/v rows of the earlier tokens; the recurrent state before token t is the oracle's delta rule
carried from the state before the call over the device's traced inputs of the earlier tokens.
The state after the call is compared with that carried state (its differences add up over the
tokens: 2e-5 of max |state| for m <= 16).  The device runs the delta rule's tokens inside one launch
with each token's arithmetic that of the single step, so its output also equals m single steps
of the per-token kernels bit for bit when the inputs are the same: test_steps_equal_single_steps.
"""

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth
from test_gpu_deltanet import CHAIN_TOL, KQ, SMALL, STAGE_TOL, THREADS, TOL, close, project

pytestmark = pytest.mark.gpu

STATE_TOL = 2e-5  # the state carried over several tokens, relative to max |state|


def run_tokens(ctx, d, w, vec, hist, st, xs, trace=True):
    """One oq_deltanet_steps call over the rows of xs: y [m][E], per-token traces, history, state."""
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    m, E = xs.shape
    sizes = oracle.deltanet_trace_sizes(d)
    per = sum(sizes.values())
    bufs = []
    try:
        hb, sb, xb, yb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(xs), ctx.alloc(m * E * 4)
        bufs += [hb, sb, xb, yb]
        tb = ctx.alloc(m * per * 4) if trace else None
        if tb is not None:
            bufs.append(tb)
        ctx.deltanet_steps(blk, m, hb, sb, xb, yb, tb)
        ctx.sync()
        traces = []
        if trace:
            flat = tb.download(np.float32, m * per).reshape(m, per)
            for t in range(m):
                tr, off = {}, 0
                for n, sz in sizes.items():
                    tr[n] = flat[t, off:off + sz]
                    off += sz
                traces.append(tr)
        return (yb.download(np.float32, m * E).reshape(m, E), traces,
                hb.download(np.float32, hist.size).reshape(hist.shape), sb.download(np.float32, st.size).reshape(st.shape))
    finally:
        for b in bufs:
            b.free()
        blk.release()


def check_token(d, w, vec, x, y, g, hist0, state0, check_projections=True):
    """Token t's stages from the device's inputs to them; returns the oracle's state after it."""
    E = d["embedding"]
    Hk, Hv, dk, dv, eps = (d[k] for k in ("key_heads", "value_heads", "key_dim", "value_dim", "eps"))
    C_, V, F = 2 * Hk * dk + Hv * dv, Hv * dv, d["ffn"]
    worst = {}
    if check_projections:
        normed = oracle.rms_norm_rows(x, vec["input_norm"], E, eps)
        projections = {"qkv": ("qkv", normed, C_, E), "z": ("z", normed, V, E), "beta": ("beta", normed, Hv, E),
                       "alpha": ("alpha", normed, Hv, E), "branch": ("out", g["gated"], E, V),
                       "gate": ("gate", g["post"], F, E), "up": ("up", g["post"], F, E),
                       "ffn": ("down", g["act"], E, F)}
        for n, (wn, inp, rows, cols) in projections.items():
            yo, norm = project(w, wn, inp, rows, cols)
            worst[n] = float(np.max(np.abs(g[n].astype(np.float64) - yo) / np.maximum(norm, 1e-30)))
            assert worst[n] <= TOL, f"{n}: normalised error {worst[n]:.3e}"
    close("conv", g["conv"], oracle.conv_step(hist0.copy(), vec["conv_weight"], g["qkv"], apply_silu=True), worst)
    q = np.stack([g["conv"][(h % Hk) * dk:(h % Hk + 1) * dk] for h in range(Hv)])
    k = np.stack([g["conv"][Hk * dk + (h % Hk) * dk:Hk * dk + (h % Hk + 1) * dk] for h in range(Hv)])
    beta = np.array([oracle.sigmoid(b) for b in g["beta"]], np.float32)
    ld = np.array([np.float32(oracle.softplus(float(np.float32(a + b)))) * c
                   for a, b, c in zip(g["alpha"], vec["dt_bias"], vec["decay"])], np.float32)
    close("beta_s", g["beta_s"], beta, worst)
    close("log_decay", g["log_decay"], ld, worst)
    state = state0.copy()
    rec = oracle.gated_delta_step(q, k, g["conv"][2 * Hk * dk:].reshape(Hv, dv), beta, ld, state, eps).reshape(-1)
    close("rec", g["rec"], rec, worst)
    zs = np.array([oracle.silu(v) for v in g["z"]], np.float32)
    close("gated", g["gated"], oracle.rms_norm_rows(g["rec"], vec["out_norm"], dv, eps) * zs, worst)
    close("resid", g["resid"], x + g["branch"], worst)
    close("post", g["post"], oracle.rms_norm_rows(g["resid"], vec["post_norm"], E, eps), worst)
    close("act", g["act"], np.array([oracle.silu(a) for a in g["gate"]], np.float32) * g["up"], worst)
    close("y", y, g["resid"] + g["ffn"], worst)
    return state


def shifted(hist, qkv):
    out = np.empty_like(hist)
    out[:, :-1] = hist[:, 1:]
    out[:, -1] = qkv
    return out


@pytest.mark.parametrize("dims,m", [
    (SMALL, 4),
    (dict(SMALL, key_heads=4, key_dim=64, value_dim=64, value_heads=8, conv_kernel=3), 3),
    (dict(SMALL, key_dim=32, value_dim=192, value_heads=4, key_heads=4, conv_kernel=2), 5),
    (dict(SMALL, value_dim=256, value_heads=2, key_heads=1), 2),
    (SMALL, 1),
    (SMALL, 9),
    (SMALL, 11),
    (dict(SMALL, conv_kernel=6), 3),
    (dict(SMALL, embedding=8192), 2),
    (dict(SMALL, embedding=4096), 2),
    (synth.DELTANET_DIMS, 6),
], ids=["hk2_hv4_m4", "dk64_dv64_k3_m3", "dk32_dv192_k2_m5", "dv256_m2", "m1", "m9", "m11", "k6_m3", "e8192_m2",
        "e4096_m2", "full_m6"])
def test_tokens_match_oracle(ctx, dims, m):
    """Every token's stages, the history (exact) and the carried state after the call.  Up to 8
    tokens one in-projection launch also runs the convolution and gates (taps <= 4); 9 tokens add
    a one-token launch and the separate convolution launch for it, 11 a second three-token launch,
    six taps the separate launch for all."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(61), dims)
    xs = np.random.default_rng(62).standard_normal((m, d["embedding"])).astype(np.float32)
    y, traces, hist_g, st_g = run_tokens(ctx, d, w, vec, hist, st, xs)
    h, s = hist.copy(), st.copy()
    h_o, s_o = hist.copy(), st.copy()
    for t in range(m):
        s = check_token(d, w, vec, xs[t], y[t], traces[t], h, s)
        h = shifted(h, traces[t]["qkv"])
        y_o = oracle.deltanet_step(d, w, vec, h_o, s_o, xs[t], threads=THREADS)
        assert np.max(np.abs(y[t] - y_o)) <= CHAIN_TOL * np.max(np.abs(y_o)), t
    assert np.array_equal(hist_g, h)
    assert np.max(np.abs(st_g - s)) <= STATE_TOL * np.max(np.abs(s))


def test_tokens_full_block_matrix_cores(ctx):
    """The hidden-4096 block (32 heads of 128, FFN 12288) over 16 tokens: every projection takes
    the matrix-core path (m >= 16, K >= 4096).  Tokens 0, 7 and 15 are checked stage by stage with
    their projections; every token's other stages are checked and the state carried."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(71))
    m = 16
    xs = np.random.default_rng(72).standard_normal((m, d["embedding"])).astype(np.float32)
    y, traces, hist_g, st_g = run_tokens(ctx, d, w, vec, hist, st, xs)
    h, s = hist.copy(), st.copy()
    for t in range(m):
        s = check_token(d, w, vec, xs[t], y[t], traces[t], h, s, check_projections=t in (0, 7, 15))
        h = shifted(h, traces[t]["qkv"])
    assert np.array_equal(hist_g, h)
    assert np.max(np.abs(st_g - s)) <= STATE_TOL * np.max(np.abs(s))
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("m", [2, 4, 9])
def test_tokens_trace_does_not_change_results(ctx, m):
    """Untraced, the down projection adds the residual in its own stores and the gated norm writes
    the out projection's Q8_K blocks; traced, both stay separate launches; at two tokens the post
    norm's rows are stored only when traced: the same bits."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(85), SMALL)
    xs = np.random.default_rng(86).standard_normal((m, d["embedding"])).astype(np.float32)
    y0, _, h0, s0 = run_tokens(ctx, d, w, vec, hist, st, xs, trace=False)
    y1, _, h1, s1 = run_tokens(ctx, d, w, vec, hist, st, xs, trace=True)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    assert np.array_equal(h0, h1) and np.array_equal(s0.view(np.uint32), s1.view(np.uint32))


def test_steps_equal_single_steps(ctx):
    """Below 16 tokens the call's kernels per token are those of the single step's per-stage
    schedule (OQ_BLOCK_FUSED=0: RMSNorm, the same small-batch products from one Q8_K image,
    convolution, delta rule, gated norm): m single steps give the same bits as one m-token call."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(81), SMALL)
    m = 4
    xs = np.random.default_rng(82).standard_normal((m, d["embedding"])).astype(np.float32)
    y, _, hist_g, st_g = run_tokens(ctx, d, w, vec, hist, st, xs, trace=False)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        hb, sb, yb = ctx.to_device(hist), ctx.to_device(st), ctx.alloc(d["embedding"] * 4)
        ys = []
        with oracle_amd.launch_options({"OQ_BLOCK_FUSED": "0", "OQ_FUSED_QUANT": "0"}):
            for t in range(m):
                xb = ctx.to_device(xs[t])
                ctx.deltanet_step(blk, hb, sb, xb, yb)
                ctx.sync()
                ys.append(yb.download(np.float32, d["embedding"]))
                xb.free()
        single = np.stack(ys)
        # the projections of one token at m = 1 and inside an m-row product add the same integer
        # dot products in the same order (the small-batch kernels give the batch-1 kernel's bits)
        assert np.array_equal(single.view(np.uint32), y.view(np.uint32))
        assert np.array_equal(hb.download(np.float32, hist.size).reshape(hist.shape), hist_g)
        assert np.array_equal(sb.download(np.float32, st.size).reshape(st.shape), st_g)
        for b in (hb, sb, yb):
            b.free()
    finally:
        blk.release()


def test_tokens_errors(ctx):
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(91), SMALL)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        hb, sb = ctx.to_device(hist), ctx.to_device(st)
        xb, yb = ctx.alloc(2 * d["embedding"] * 4), ctx.alloc(2 * d["embedding"] * 4)
        with pytest.raises(oracle_amd.InvalidArgument, match="token count must be non-zero"):
            ctx.deltanet_steps(blk, 0, hb, sb, xb, yb)
        blk.desc.value_dim = 96
        with pytest.raises(oracle_amd.InvalidArgument):
            ctx.deltanet_steps(blk, 2, hb, sb, xb, yb)
        blk.desc.value_dim = d["value_dim"]
        for b in (hb, sb, xb, yb):
            b.free()
    finally:
        blk.release()
