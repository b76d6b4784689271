"""Benchmark of the quantized-weight matrix path on one MI355X.

Default workload: Q4_K FFN gate/up decode GEMV, 12288 rows x 4096 columns, batch 1; F32
activation ~N(0,1) quantized to Q8_K on the device inside the same kernel.  One step = one
matvec (F32 x in HBM -> F32 y in HBM).  K steps are captured into one HIP graph and replayed
between two HIP events on the library's stream; steps cycle over >= 512 MiB of distinct weight
copies so the 256 MiB Infinity Cache cannot serve them.  `value` = weight bytes / step time.

Also reported: the M=512 Q4_K prefill GEMM (4096 x 12288) in TOPS when the matrix-core path is
available, the roofline of the dominant kernel, and the reference CPU algorithm (the oracle's
restatement, single thread) timed on a bounded sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import oracle_amd  # noqa: E402
from oracle_amd import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp16": 2500.0, "int8": 5000.0}
MALL_DEFEAT_BYTES = 512 << 20

# name -> (type, rows N, cols K, batch M, description)
WORKLOADS = {
    "q4k_gemv": (12, 12288, 4096, 1, "Q4_K FFN gate/up decode GEMV 12288x4096, batch 1, Q8_K activations"),
    "q8_0_gemv": (8, 4096, 4096, 1, "Q8_0 GEMV 4096x4096, batch 1, F32 activations"),
    "q6k_head": (14, 151936, 4096, 1, "Q6_K output-head GEMV 151936x4096, batch 1, Q8_K activations"),
    "q4k_down_m1": (12, 4096, 12288, 1, "Q4_K down-projection GEMV 4096x12288, batch 1, Q8_K activations"),
    "q4k_down_m4": (12, 4096, 12288, 4, "Q4_K down-projection GEMM 4096x12288, M=4, Q8_K activations"),
    "q4k_down_m512": (12, 4096, 12288, 512, "Q4_K down-projection GEMM 4096x12288, M=512, Q8_K activations"),
}
SEED = 20261201


def weight_bytes(t, n, k):
    return synth.row_bytes(t, k) * n


def run_gpu(ctx, name, steps, warmup, copies_min_bytes=MALL_DEFEAT_BYTES):
    t, n, k, m, desc = WORKLOADS[name]
    rng = np.random.default_rng(SEED + list(WORKLOADS).index(name))
    data = synth.weights(t, rng, n, k)
    wb = data.nbytes
    ncopies = max(1, math.ceil(copies_min_bytes / wb))
    dev = ctx.to_device(data)
    ws = [ctx.upload_from_device(t, k, n, dev, wb) for _ in range(ncopies)]
    dev.free()
    x = synth.activations(rng, m, k)
    xb = ctx.to_device(x)
    yb = ctx.alloc(m * n * 4)

    def step(i):
        if m == 1:
            ctx.matvec(ws[i % ncopies], xb, yb)
        else:
            ctx.matmul(ws[i % ncopies], m, xb, yb)

    step(0)  # sizes any staging buffer before capture
    ctx.sync()
    ctx.capture_begin()
    for i in range(warmup):
        step(i)
    g_warm = ctx.capture_end()
    ctx.capture_begin()
    for i in range(steps):
        step(i)
    g = ctx.capture_end()
    g_warm.launch()
    ctx.sync()
    ctx.timer_start()
    g.launch()
    ms = ctx.timer_stop()
    g.destroy()
    g_warm.destroy()
    ms_step = ms / steps
    xbytes = m * k * 4
    ybytes = m * n * 4
    res = {
        "workload": name, "desc": desc, "type": t, "rows": n, "cols": k, "m": m,
        "weight_bytes": wb, "copies": ncopies, "ms_per_step": ms_step,
        "us_per_step": ms_step * 1e3,
        "weight_gbs": wb / (ms_step * 1e-3) / 1e9,
        "algorithmic_bytes": wb + xbytes + ybytes,
        "tops": 2.0 * m * n * k / (ms_step * 1e-3) / 1e12,
    }
    if name == "q6k_head":
        # greedy token over the head's logits, on the device (oq_argmax), timed on its own
        tb, vb = ctx.alloc(4), ctx.alloc(4)
        ctx.argmax(yb, n, tb, vb)
        ctx.sync()
        ctx.capture_begin()
        for _ in range(steps):
            ctx.argmax(yb, n, tb, vb)
        ga = ctx.capture_end()
        ga.launch()
        ctx.sync()
        ctx.timer_start()
        ga.launch()
        res["greedy_token_us"] = ctx.timer_stop() * 1e3 / steps
        ga.destroy()
        tb.free()
        vb.free()
    for w in ws:
        w.release()
    xb.free()
    yb.free()
    return res


def run_deltanet(ctx, steps, warmup, copies_min_bytes=MALL_DEFEAT_BYTES):
    """One Gated DeltaNet decode block (hidden 4096, 32 heads of dk = dv = 128, FFN 12288) per
    step, chained on the device (oq_deltanet_step); steps cycle over block copies whose weights
    total >= 512 MiB, so every step streams its projections from HBM."""
    rng = np.random.default_rng(SEED + 100)
    d, w, vec, hist, st, x = synth.deltanet_block(rng)
    first = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    wb = first.weight_bytes()
    ncopies = max(1, math.ceil(copies_min_bytes / wb))
    blocks = [first] + [oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec) for _ in range(ncopies - 1)]
    hb, sb, xb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(x)
    yb = ctx.alloc(d["embedding"] * 4)

    def step(i):
        ctx.deltanet_step(blocks[i % ncopies], hb, sb, xb, yb)

    step(0)  # sizes the block workspace before capture
    ctx.sync()
    ctx.capture_begin()
    for i in range(warmup):
        step(i)
    g_warm = ctx.capture_end()
    ctx.capture_begin()
    for i in range(steps):
        step(i)
    g = ctx.capture_end()
    g_warm.launch()
    ctx.sync()
    ctx.timer_start()
    g.launch()
    ms = ctx.timer_stop()
    g.destroy()
    g_warm.destroy()
    for b in blocks:
        b.release()
    for buf in (hb, sb, xb, yb):
        buf.free()
    ms_step = ms / steps
    return {"workload": "deltanet_block", "weight_bytes": wb, "copies": ncopies, "ms_per_step": ms_step,
            "us_per_block": ms_step * 1e3, "weight_gbs": wb / (ms_step * 1e-3) / 1e9,
            "state_bytes": 2 * st.nbytes, "dims": d}


def run_copy_calibration(ctx, steps, nbytes=28311552):
    """Device-to-device copies of a known size: the FETCH_SIZE / WRITE_SIZE counters of this
    dispatch calibrate the same counters read on the GEMV kernels."""
    src = ctx.alloc(nbytes)
    dst = ctx.alloc(nbytes)
    ctx.lib.oq_copy_device(ctx.h, dst.ptr, src.ptr, nbytes)
    ctx.sync()
    ctx.timer_start()
    for _ in range(steps):
        ctx.lib.oq_copy_device(ctx.h, dst.ptr, src.ptr, nbytes)
    ms = ctx.timer_stop()
    src.free()
    dst.free()
    return {"workload": "copy_calibration", "bytes": nbytes, "us_per_copy": ms * 1e3 / steps}


def committed_traffic(name):
    """HBM bytes per launch of the workload's dominant kernel, from the committed rocprofv3
    counter summary (oracle_amd/profile.sh writes it); None when there is none."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if not p.exists():
        return None
    return json.loads(p.read_text())["traffic_bytes"]


def cpu_baseline(name, budget_s=12.0):
    """The reference's CPU algorithm (oracle restatement: decode block, sequential F32 dot) on
    the same workload, single thread, repeated until ~budget_s seconds; plus all host cores."""
    import oracle

    t, n, k, m, _ = WORKLOADS[name]
    rng = np.random.default_rng(SEED + list(WORKLOADS).index(name))
    data = synth.weights(t, rng, n, k)
    x = synth.activations(rng, 1, k)[0]
    xhat = oracle.dequantize_q8k(oracle.quantize_q8k(x), k) if t in (12, 13, 14) else x
    rows = n
    if t == 14:  # bound the 151936-row head: time a contiguous slice
        rows = 16384
    sample = data[: rows * synth.row_bytes(t, k)]
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.storage_matvec(t, rows, k, sample, xhat, threads=1)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    single = sample.nbytes * reps / el / 1e9
    threads = min(oracle.default_threads(), 16)
    reps2, t0 = 0, time.perf_counter()
    while True:
        oracle.storage_matvec(t, rows, k, sample, xhat, threads=threads)
        reps2 += 1
        el2 = time.perf_counter() - t0
        if el2 >= budget_s / 3 or reps2 >= 2000:
            break
    multi = sample.nbytes * reps2 / el2 / 1e9
    return {
        "value": single, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{reps} x {rows}x{k} type-{t} matvec (oracle restatement of reference_storage_matvec, "
                  f"-O2 -ffp-contract=off), {el:.1f} s",
        "us_per_matvec_1core": el / reps * 1e6 * (n / rows),
        "all_cores": {"value": multi, "cores": threads, "us_per_matvec": el2 / reps2 * 1e6 * (n / rows)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="q4k_gemv",
                    choices=sorted(WORKLOADS) + ["copy_calibration", "deltanet_block"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the quantized matrix path is "
              "row-sharded across GPUs by design but only the single-GPU kernel is built and timed.",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit(2)

    ctx = oracle_amd.Context(0)
    if args.workload == "copy_calibration":
        print(json.dumps(run_copy_calibration(ctx, args.steps)), flush=True)
        ctx.close()
        return
    if args.workload == "deltanet_block":
        r = run_deltanet(ctx, args.steps, args.warmup)
        ctx.close()
        print(json.dumps({
            "metric": "DeltaNet decode block weight GB/s", "value": round(r["weight_gbs"], 2), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xu4 dot (i32) + f32",
            "data": "synthetic (seeded block weights, state ~ N(0, 0.01), x ~ N(0,1))",
            "config": {"workload": "Gated DeltaNet decode block, batch 1", **r["dims"],
                       "weight_bytes": r["weight_bytes"], "block_copies_cycled": r["copies"]},
            "us_per_block": round(r["us_per_block"], 2),
            "hbm_frac_weight_bytes": round(r["weight_gbs"] / HBM_PEAK_GBS, 4)}), flush=True)
        return
    main_res = run_gpu(ctx, args.workload, args.steps, args.warmup)
    secondary = block = None
    if not args.no_secondary and args.workload == "q4k_gemv":
        secondary = run_gpu(ctx, "q4k_down_m512", max(5, args.steps // 20), max(2, args.warmup // 5))
        block = run_deltanet(ctx, max(5, args.steps // 10), max(2, args.warmup // 5))
    ctx.close()

    t, n, k, m, desc = WORKLOADS[args.workload]
    gbs = main_res["weight_gbs"]
    achieved = main_res["algorithmic_bytes"] / (main_res["ms_per_step"] * 1e-3) / 1e9
    out = {
        "metric": "Q4_K GEMV weight GB/s (% of HBM peak); M=512 Q4_K GEMM TOPS (% MFMA)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xu4 dot (i32) + f32 scales",
        "data": "synthetic (seeded: weights per workload distributions, x ~ N(0,1))",
        "config": {"workload": desc, "rows": n, "cols": k, "batch": m, "weight_type": "q4_K" if t == 12 else t,
                   "weight_copies_cycled": main_res["copies"], "seed": SEED},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(args.workload)},
        "us_per_gemv": round(main_res["us_per_step"], 3),
        **({"greedy_token_us": round(main_res["greedy_token_us"], 3)} if "greedy_token_us" in main_res else {}),
        "hbm_frac_weight_bytes": round(gbs / HBM_PEAK_GBS, 4),
    }
    if secondary is not None:
        out["gemm_m512"] = {"tops": round(secondary["tops"], 2), "us": round(secondary["us_per_step"], 2),
                            "frac_fp16_mfma_peak": round(secondary["tops"] / MFMA_PEAK_TFLOPS["fp16"], 4),
                            "frac_int8_mfma_peak": round(secondary["tops"] / MFMA_PEAK_TFLOPS["int8"], 4)}
    if block is not None:
        out["deltanet_block"] = {"us": round(block["us_per_block"], 2), "weight_gbs": round(block["weight_gbs"], 1),
                                 "hbm_frac": round(block["weight_gbs"] / HBM_PEAK_GBS, 4),
                                 "weight_bytes": block["weight_bytes"]}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.workload)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
