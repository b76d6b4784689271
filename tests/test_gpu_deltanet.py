"""GPU parity of the Gated DeltaNet decode block (oq_deltanet_step) against the oracle's
restatement of the reference block (qwen35_block.cpp:406-605) on identical seeded inputs.

Stage by stage: every intermediate the device produced is compared with the oracle's
computation of that stage from the device's own inputs to it (the traced previous stages, the
state and convolution history before the step), so each stage is held to its own bar:
- projections (qkv, z, beta, alpha, out -> branch, gate, up, down -> ffn): the product bar of
  the matvec path, |y_gpu - y_orc| <= 1e-4 * sum_k |w_k * xhat_k| per output;
- elementwise and per-head stages (conv + SiLU, gates, delta rule output and state, gated
  RMSNorm, residuals, post-norm, SwiGLU, y): within 2e-6 of the stage's scale (max |value|):
  the same F32/double operation order as the reference, up to the last-ulp differences of
  expf / log1pf and of double-sum order.
End to end (device chain vs oracle chain from the same x) only a wiring check is possible: the
Q8_K re-quantization of each projection input is discontinuous, so the ~1e-6 relative stage
differences flip a rounding of some element with probability ~1e-3 per element; one flip in
the post-norm moves gate/up by ~1e-3 of their scale, and the SwiGLU and the down projection's
re-quantization amplify it (measured: up to ~1.5e-2 of max |y| on the small blocks, 4e-6 on
the full block).  The bound is 5e-2 of max |y| (a wrong residual, norm or head mapping is
O(1)); the state, upstream of the FFN, stays within 1e-4 of max |state|.
"""

import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4          # projections (normalised by sum |w xhat|)
STAGE_TOL = 2e-6    # elementwise stages, relative to the stage's max |value|
CHAIN_TOL = 5e-2    # end-to-end y, relative to max |y| (wiring check, see above)
THREADS = min(16, oracle.default_threads())
KQ = (12, 13, 14)


def run_gpu(ctx, d, w, vec, hist, st, xs):
    """Device steps over xs; per step: y, trace, and the history / state before the step."""
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        hb, sb = ctx.to_device(hist), ctx.to_device(st)
        sizes = oracle.deltanet_trace_sizes(d)
        tb = ctx.alloc(sum(sizes.values()) * 4)
        yb = ctx.alloc(d["embedding"] * 4)
        steps = []
        for x in xs:
            h0 = hb.download(np.float32, hist.size).reshape(hist.shape)
            s0 = sb.download(np.float32, st.size).reshape(st.shape)
            xb = ctx.to_device(x)
            ctx.deltanet_step(blk, hb, sb, xb, yb, tb)
            ctx.sync()
            flat = tb.download(np.float32, sum(sizes.values()))
            tr, off = {}, 0
            for n, sz in sizes.items():
                tr[n] = flat[off:off + sz]
                off += sz
            steps.append({"x": x, "y": yb.download(np.float32, d["embedding"]), "trace": tr, "hist0": h0,
                          "state0": s0})
            xb.free()
        return steps, hb.download(np.float32, hist.size).reshape(hist.shape), \
            sb.download(np.float32, st.size).reshape(st.shape)
    finally:
        blk.release()


def project(w, name, inp, rows, cols):
    """Oracle projection of the device's input: y and the per-output normaliser sum |w xhat|."""
    t, data = w[name]
    xhat = oracle.dequantize_q8k(oracle.quantize_q8k(inp), cols) if t in KQ else inp
    y = oracle.storage_matvec(t, rows, cols, data, xhat, threads=THREADS)
    return y, oracle.matvec_stats(t, rows, cols, data, xhat, threads=THREADS)[1]


def close(name, got, want, worst):
    scale = float(np.max(np.abs(want))) or 1.0
    worst[name] = float(np.max(np.abs(got.astype(np.float64) - want))) / scale
    assert worst[name] <= STAGE_TOL, f"{name}: error {worst[name]:.3e} of scale"


def check_stages(d, w, vec, step, state_after):
    """Each device stage against the oracle's computation of it from the device's inputs."""
    E, F = d["embedding"], d["ffn"]
    Hk, Hv, dk, dv, eps = (d[k] for k in ("key_heads", "value_heads", "key_dim", "value_dim", "eps"))
    C_, V = 2 * Hk * dk + Hv * dv, Hv * dv
    g, x = step["trace"], step["x"]
    worst = {}
    normed = oracle.rms_norm_rows(x, vec["input_norm"], E, eps)
    projections = {"qkv": ("qkv", normed, C_, E), "z": ("z", normed, V, E), "beta": ("beta", normed, Hv, E),
                   "alpha": ("alpha", normed, Hv, E), "branch": ("out", g["gated"], E, V),
                   "gate": ("gate", g["post"], F, E), "up": ("up", g["post"], F, E), "ffn": ("down", g["act"], E, F)}
    for n, (wn, inp, rows, cols) in projections.items():
        y, norm = project(w, wn, inp, rows, cols)
        worst[n] = float(np.max(np.abs(g[n].astype(np.float64) - y) / np.maximum(norm, 1e-30)))
        assert worst[n] <= TOL, f"{n}: normalised error {worst[n]:.3e}"
    hist = step["hist0"].copy()
    close("conv", g["conv"], oracle.conv_step(hist, vec["conv_weight"], g["qkv"], apply_silu=True), worst)
    q = np.stack([g["conv"][(t % Hk) * dk:(t % Hk + 1) * dk] for t in range(Hv)])
    k = np.stack([g["conv"][Hk * dk + (t % Hk) * dk:Hk * dk + (t % Hk + 1) * dk] for t in range(Hv)])
    beta = np.array([oracle.sigmoid(b) for b in g["beta"]], np.float32)
    ld = np.array([np.float32(oracle.softplus(float(np.float32(a + b)))) * c
                   for a, b, c in zip(g["alpha"], vec["dt_bias"], vec["decay"])], np.float32)
    close("beta_s", g["beta_s"], beta, worst)
    close("log_decay", g["log_decay"], ld, worst)
    state = step["state0"].copy()
    rec = oracle.gated_delta_step(q, k, g["conv"][2 * Hk * dk:].reshape(Hv, dv), beta, ld, state, eps).reshape(-1)
    close("rec", g["rec"], rec, worst)
    close("state", state_after, state, worst)
    zs = np.array([oracle.silu(v) for v in g["z"]], np.float32)
    close("gated", g["gated"], oracle.rms_norm_rows(g["rec"], vec["out_norm"], dv, eps) * zs, worst)
    close("resid", g["resid"], x + g["branch"], worst)
    close("post", g["post"], oracle.rms_norm_rows(g["resid"], vec["post_norm"], E, eps), worst)
    close("act", g["act"], np.array([oracle.silu(a) for a in g["gate"]], np.float32) * g["up"], worst)
    close("y", step["y"], g["resid"] + g["ffn"], worst)
    return worst


def check_history(step, hist_after):
    """The convolution history after a step: shifted left by one, the device's qkv appended."""
    assert np.array_equal(hist_after[:, :-1], step["hist0"][:, 1:])
    assert np.array_equal(hist_after[:, -1], step["trace"]["qkv"])


SMALL = dict(synth.DELTANET_DIMS, embedding=1024, key_heads=2, value_heads=4, ffn=1536)


@pytest.mark.parametrize("dims", [
    SMALL,
    dict(SMALL, key_heads=4, key_dim=64, value_dim=64, value_heads=8, conv_kernel=3),
    dict(SMALL, value_dim=256, value_heads=2, key_heads=1),
    dict(SMALL, key_dim=32, value_dim=192, value_heads=4, key_heads=4, conv_kernel=2),
    dict(SMALL, ffn=17408),
    dict(SMALL, conv_kernel=8),
], ids=["hk2_hv4", "dk64_dv64_k3", "dv256", "dk32_dv192_k2", "ffn17408", "k8"])
@pytest.mark.parametrize("env", [{"OQ_BLOCK_FUSED": "1"}, {"OQ_BLOCK_FUSED": "1", "OQ_BLOCK_STREAM": "0"},
                                 {"OQ_BLOCK_FUSED": "0"}], ids=["fused", "fused_batched", "separate"])
def test_deltanet_steps_match_oracle(ctx, dims, env):
    """Every device schedule: the fused one (five launches: normalised in-projections with the
    convolution and gates, delta rule, out projection + residual, normalised gate/up + SwiGLU,
    down + residual; the residual projections streamed, or with OQ_BLOCK_STREAM=0 in the batched
    structure) and the one launch per stage (OQ_BLOCK_FUSED=0)."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(21), dims)
    rng = np.random.default_rng(22)
    xs = [rng.standard_normal(d["embedding"]).astype(np.float32) for _ in range(3)]
    with oracle_amd.launch_options(env):
        steps, hist_g, st_g = run_gpu(ctx, d, w, vec, hist, st, xs)
    h_o, s_o = hist.copy(), st.copy()
    for i, stp in enumerate(steps):
        after = steps[i + 1]["state0"] if i + 1 < len(steps) else st_g
        hist_after = steps[i + 1]["hist0"] if i + 1 < len(steps) else hist_g
        check_stages(d, w, vec, stp, after)
        check_history(stp, hist_after)
        y_o = oracle.deltanet_step(d, w, vec, h_o, s_o, stp["x"], threads=THREADS)
        assert np.max(np.abs(stp["y"] - y_o)) <= CHAIN_TOL * np.max(np.abs(y_o))
        assert np.max(np.abs(after - s_o)) <= TOL * np.max(np.abs(s_o))


def test_deltanet_full_block_matches_oracle(ctx):
    # the Qwen3.5-style block at hidden 4096: 32 heads, dk = dv = 128, FFN 12288
    d, w, vec, hist, st, x = synth.deltanet_block(np.random.default_rng(31))
    steps, hist_g, st_g = run_gpu(ctx, d, w, vec, hist, st, [x])
    worst = check_stages(d, w, vec, steps[0], st_g)
    y_o = oracle.deltanet_step(d, w, vec, hist, st, x, threads=THREADS)
    chain = float(np.max(np.abs(steps[0]["y"] - y_o)) / np.max(np.abs(y_o)))
    print("worst stage errors", {k: f"{v:.2e}" for k, v in worst.items()}, f"chain {chain:.2e}")
    assert chain <= CHAIN_TOL
    assert np.max(np.abs(st_g - st)) <= TOL * np.max(np.abs(st))
    check_history(steps[0], hist_g)


@pytest.mark.parametrize("dims", [SMALL, dict(SMALL, conv_kernel=3)], ids=["k4", "k3"])
@pytest.mark.parametrize("env", [{}, {"OQ_BLOCK_STREAM": "0"}], ids=["streamed", "batched"])
def test_deltanet_trace_does_not_change_results(ctx, dims, env):
    """Without a trace the block skips the stores only the trace reads (raw projections, the
    normalised FFN input, the gated row): y, the state and the history must be the same bits."""
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(41), dims)
    rng = np.random.default_rng(42)
    xs = [rng.standard_normal(d["embedding"]).astype(np.float32) for _ in range(2)]
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    bufs = []
    try:
        tb = ctx.alloc(sum(oracle.deltanet_trace_sizes(d).values()) * 4)
        bufs.append(tb)
        runs = []
        for traced in (True, False):
            hb, sb, yb = ctx.to_device(hist), ctx.to_device(st), ctx.alloc(d["embedding"] * 4)
            bufs += [hb, sb, yb]
            ys = []
            for x in xs:
                xb = ctx.to_device(x)
                with oracle_amd.launch_options(env):
                    if traced:
                        ctx.deltanet_step(blk, hb, sb, xb, yb, tb)
                    else:
                        ctx.deltanet_step(blk, hb, sb, xb, yb)
                ctx.sync()
                ys.append(yb.download(np.float32, d["embedding"]))
                xb.free()
            runs.append((ys, hb.download(np.float32, hist.size), sb.download(np.float32, st.size)))
        (y_t, h_t, s_t), (y_n, h_n, s_n) = runs
        for a, b in zip(y_t, y_n):
            assert np.array_equal(a, b)
        assert np.array_equal(h_t, h_n) and np.array_equal(s_t, s_n)
    finally:
        for b in bufs:
            b.free()
        blk.release()


def test_deltanet_rejects_bad_shapes(ctx):
    d, w, vec, hist, st, x = synth.deltanet_block(np.random.default_rng(41), SMALL)
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        hb, sb, xb, yb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(x), ctx.alloc(d["embedding"] * 4)
        blk.desc.key_dim = 4097  # wider than the any-shape delta rule's LDS rows
        with pytest.raises(oracle_amd.InvalidArgument, match="key_dim <= 4096"):
            ctx.deltanet_step(blk, hb, sb, xb, yb)
        blk.desc.key_dim = d["key_dim"]
        blk.desc.value_dim = 96  # the projections no longer match
        with pytest.raises(oracle_amd.InvalidArgument, match="has shape"):
            ctx.deltanet_step(blk, hb, sb, xb, yb)
        blk.desc.value_dim = d["value_dim"]
        blk.desc.ffn = d["ffn"] + 256  # gate/up/down no longer match
        with pytest.raises(oracle_amd.InvalidArgument):
            ctx.deltanet_step(blk, hb, sb, xb, yb)
        blk.desc.ffn = d["ffn"]
        ctx.deltanet_step(blk, hb, sb, xb, yb)
        ctx.sync()
    finally:
        blk.release()


def test_deltanet_graph_replay_matches_eager(ctx):
    # the block captured into a HIP graph (no allocation, no memset inside) replays like eager calls
    d, w, vec, hist, st, _ = synth.deltanet_block(np.random.default_rng(51), SMALL)
    rng = np.random.default_rng(52)
    xs = [rng.standard_normal(d["embedding"]).astype(np.float32) for _ in range(3)]
    blk = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    try:
        he, se, hg, sg = (ctx.to_device(a) for a in (hist, st, hist, st))
        xb, yb = ctx.alloc(d["embedding"] * 4), ctx.alloc(d["embedding"] * 4)
        xb.upload(xs[0])
        ctx.deltanet_step(blk, hg, sg, xb, yb)  # sizes the workspace before capture
        ctx.sync()
        hg.upload(hist)
        sg.upload(st)
        ctx.capture_begin()
        ctx.deltanet_step(blk, hg, sg, xb, yb)
        g = ctx.capture_end()
        ye = ctx.alloc(d["embedding"] * 4)
        for x in xs:
            xb.upload(x)
            ctx.deltanet_step(blk, he, se, xb, ye)
            ctx.sync()
            e = ye.download(np.float32, d["embedding"])
            g.launch()
            ctx.sync()
            r = yb.download(np.float32, d["embedding"])
            assert np.array_equal(e, r)
        assert np.array_equal(se.download(np.float32, st.size), sg.download(np.float32, st.size))
        g.destroy()
    finally:
        blk.release()
