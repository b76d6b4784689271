"""Benchmark of the quantized-weight matrix path on one MI355X.

Default workload: Q4_K FFN gate/up decode GEMV, 12288 rows x 4096 columns, batch 1; F32
activation ~N(0,1) quantized to Q8_K on the device inside the same kernel.  One step = one
matvec (F32 x in HBM -> F32 y in HBM).  K steps are launched back to back between two HIP events
on the library's stream, right behind the W warmup steps (timed_steps); steps cycle over
>= 512 MiB of distinct weight copies so the 256 MiB Infinity Cache cannot serve them.  `value` =
weight bytes / step time.

Also reported: the M=512 Q4_K prefill GEMM (4096 x 12288) in TOPS when the matrix-core path is
available; the Q8_0 4096x4096 GEMV, the Q6_K 151936x4096 output head (with the greedy token) and
the M=4 Q4_K 4096x12288 product, each with its own roofline; the DeltaNet and attention blocks;
the roofline of the dominant kernel; and the reference CPU algorithm (the oracle's restatement,
single thread) timed on a bounded sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
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
TYPE_NAMES = {8: "q8_0", 12: "q4_K", 13: "q5_K", 14: "q6_K"}
MALL_DEFEAT_BYTES = 512 << 20

# name -> (type, rows N, cols K, batch M, description)
WORKLOADS = {
    "q4k_gemv": (12, 12288, 4096, 1, "Q4_K FFN gate/up decode GEMV 12288x4096, batch 1, Q8_K activations"),
    "q8_0_gemv": (8, 4096, 4096, 1, "Q8_0 GEMV 4096x4096, batch 1, F32 activations"),
    "q6k_head": (14, 151936, 4096, 1, "Q6_K output-head GEMV 151936x4096, batch 1, Q8_K activations"),
    "q4k_down_m1": (12, 4096, 12288, 1, "Q4_K down-projection GEMV 4096x12288, batch 1, Q8_K activations"),
    "q4k_down_m4": (12, 4096, 12288, 4, "Q4_K down-projection GEMM 4096x12288, M=4, Q8_K activations"),
    "q4k_down_m512": (12, 4096, 12288, 512, "Q4_K down-projection GEMM 4096x12288, M=512, Q8_K activations"),
    "q5k_down_m512": (13, 4096, 12288, 512, "Q5_K down-projection GEMM 4096x12288, M=512, Q8_K activations"),
    "q6k_down_m512": (14, 4096, 12288, 512, "Q6_K down-projection GEMM 4096x12288, M=512, Q8_K activations"),
    "q5k_gemv": (13, 12288, 4096, 1, "Q5_K FFN gate/up decode GEMV 12288x4096, batch 1, Q8_K activations"),
    "q8_0_eh_m512": (8, 4096, 8192, 512, "Q8_0 MTP hidden projection GEMM 4096x8192 (nextn.eh_proj), M=512, F32 activations"),
}
SEED = 20261201


def weight_bytes(t, n, k):
    return synth.row_bytes(t, k) * n


def timed_steps(ctx, step, steps, warmup, first=0):
    """W warmup steps, then exactly K timed steps; returns the K steps' milliseconds.

    Steps are launched eagerly through the C ABI (about 3 us of host time per launch, less than
    a step, so the GPU never waits for the host).  After a host synchronization the W warmup
    steps are launched and, right behind them on the same stream, the HIP event pair around the
    K timed steps: the events measure the K steps back to back (they are recorded without a
    system-scope fence, so no cache write-back of the event itself falls inside the interval).
    A host synchronization closes the timed region.  (HIP graphs were measured too: a graph's first launch adds ~15-20 us of
    host set-up that the GPU waits for, 0.7-1 us per step at K = 20.)

    Step indices run on from the warmup into the timed steps (first, first + 1, ...), so with
    steps cycling over >= 512 MiB of copies no timed step reads a copy that the previous 256 MiB
    of reads touched (the Infinity Cache cannot serve it)."""
    ctx.sync()
    for i in range(warmup):
        step(first + i)
    ctx.timer_start()
    for i in range(steps):
        step(first + warmup + i)
    ms = ctx.timer_stop()
    ctx.sync()
    return ms


def timed_graph(ctx, step, steps, warmup, first, step_bytes):
    """The K timed steps captured in order into one HIP graph, timed as one launch: the steps'
    kernels run back to back with no host launch between them (what a profiler's kernel trace
    then records is the timed configuration).  The graph's first launch (its set-up) is untimed;
    then eager steps over the copies after the timed range, at least 256 MiB of them (and at
    least W), so that no timed step reads a copy the Infinity Cache may still hold; then the
    timed launch."""
    ctx.sync()
    ctx.capture_begin()
    for i in range(steps):
        step(first + warmup + i)
    g = ctx.capture_end()
    try:
        g.launch()
        eager = max(warmup, math.ceil((MALL_DEFEAT_BYTES // 2) / max(step_bytes, 1)) + 1)
        for i in range(eager):
            step(first + warmup + steps + i)
        ctx.timer_start()
        g.launch()
        ms = ctx.timer_stop()
        ctx.sync()
    finally:
        g.destroy()
    return ms


def run_gpu(ctx, name, steps, warmup, copies_min_bytes=MALL_DEFEAT_BYTES, graph=False):
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

    lib, h, xp, yp, whs = ctx.lib, ctx.h, xb.ptr, yb.ptr, [w.h for w in ws]

    def step(i):
        # direct C-ABI calls: the least host time per launch
        rc = lib.oq_matvec(h, whs[i % ncopies], xp, yp) if m == 1 else lib.oq_matmul(h, whs[i % ncopies], m, xp, yp)
        if rc != 0:
            raise RuntimeError(f"step {i}: {lib.oq_last_error(h).decode()}")

    if m == 1:
        ctx.matvec(ws[0], xb, yb)  # checked call; sizes any staging buffer
    else:
        ctx.matmul(ws[0], m, xb, yb)
    ctx.sync()
    ms = timed_graph(ctx, step, steps, warmup, 1, wb) if graph else timed_steps(ctx, step, steps, warmup, first=1)
    ms_step = ms / steps
    xbytes = m * k * 4
    ybytes = m * n * 4
    res = {
        "workload": name, "desc": desc, "type": t, "rows": n, "cols": k, "m": m,
        # the exact input bytes (weights as the reference stores them, and x), for reproduction
        "weights_sha256": hashlib.sha256(data.tobytes()).hexdigest()[:16],
        "x_sha256": hashlib.sha256(x.tobytes()).hexdigest()[:16],
        "weight_bytes": wb, "copies": ncopies, "ms_per_step": ms_step,
        "us_per_step": ms_step * 1e3,
        "weight_gbs": wb / (ms_step * 1e-3) / 1e9,
        "algorithmic_bytes": wb + xbytes + ybytes,
        "tops": 2.0 * m * n * k / (ms_step * 1e-3) / 1e12,
        "steps": steps,
    }
    if name == "q6k_head":
        # greedy token over the head's logits, on the device (oq_argmax), timed on its own
        tb, vb = ctx.alloc(4), ctx.alloc(4)
        ctx.argmax(yb, n, tb, vb)
        ctx.sync()
        def argmax_step(i):
            if ctx.lib.oq_argmax(ctx.h, yb.ptr, n, tb.ptr, vb.ptr) != 0:
                raise RuntimeError("argmax failed")

        res["greedy_token_us"] = timed_steps(ctx, argmax_step, steps, warmup) * 1e3 / steps

        # the head with the greedy token in its epilogue (oq_matvec_argmax), per step
        def fused_step(i):
            if ctx.lib.oq_matvec_argmax(ctx.h, whs[i % ncopies], xp, yp, tb.ptr, vb.ptr) != 0:
                raise RuntimeError("matvec_argmax failed")

        res["head_and_token_us"] = timed_steps(ctx, fused_step, steps, warmup, first=1 + warmup + steps) * 1e3 / steps
        tb.free()
        vb.free()
    for w in ws:
        w.release()
    xb.free()
    yb.free()
    return res


def run_deltanet(ctx, steps, warmup, copies_min_bytes=MALL_DEFEAT_BYTES, tokens=1, graph=False):
    """One Gated DeltaNet decode block (hidden 4096, 32 heads of dk = dv = 128, FFN 12288) per
    step, chained on the device (oq_deltanet_step; with tokens > 1, oq_deltanet_steps over that
    many consecutive tokens); steps cycle over block copies whose weights total >= 512 MiB, so every
    step streams its projections from HBM.  graph: the K steps captured into one HIP graph and
    timed as one launch (timed_graph), as a decode loop replaying captured blocks runs them."""
    rng = np.random.default_rng(SEED + 100)
    d, w, vec, hist, st, x = synth.deltanet_block(rng)
    if tokens > 1:
        x = rng.standard_normal((tokens, d["embedding"])).astype(np.float32)
    first = oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec)
    wb = first.weight_bytes()
    ncopies = max(1, math.ceil(copies_min_bytes / wb))
    blocks = [first] + [oracle_amd.DeltaNetBlockWeights(ctx, d, w, vec) for _ in range(ncopies - 1)]
    hb, sb, xb = ctx.to_device(hist), ctx.to_device(st), ctx.to_device(x)
    yb = ctx.alloc(tokens * d["embedding"] * 4)

    lib, h = ctx.lib, ctx.h
    descs = [C.byref(b.desc) for b in blocks]
    hp, sp, xp, yp = hb.ptr, sb.ptr, xb.ptr, yb.ptr

    def step(i):
        rc = lib.oq_deltanet_step(h, descs[i % ncopies], hp, sp, xp, yp, None) if tokens == 1 else \
            lib.oq_deltanet_steps(h, descs[i % ncopies], tokens, hp, sp, xp, yp, None)
        if rc != 0:
            raise RuntimeError(f"step {i}: {lib.oq_last_error(h).decode()}")

    step(0)  # checked call; sizes the block workspace
    ctx.sync()
    ms = timed_graph(ctx, step, steps, warmup, 1, wb) if graph else timed_steps(ctx, step, steps, warmup, first=1)
    for b in blocks:
        b.release()
    for buf in (hb, sb, xb, yb):
        buf.free()
    ms_step = ms / steps
    return {"workload": "deltanet_block", "weight_bytes": wb, "copies": ncopies, "ms_per_step": ms_step,
            "us_per_block": ms_step * 1e3, "weight_gbs": wb / (ms_step * 1e-3) / 1e9,
            "state_bytes": 2 * st.nbytes, "dims": d, "tokens": tokens, "us_per_token": ms_step * 1e3 / tokens}


ATTN_GEOMETRY = dict(q_heads=16, kv_heads=4, head_dim=256, tokens=32768)


def run_attention(ctx, steps, warmup, copies_min_bytes=MALL_DEFEAT_BYTES, kv_dtype="f32", **geometry):
    """Single-token GQA attention (oq_attention_step): 16 query heads over 4 KV heads of 256 with
    32768 tokens cached (F32 keys and values, 256 MiB; an F16 cache, kv_dtype "f16", 128 MiB);
    steps cycle over caches totalling >= 512 MiB.  Each step appends one token; the cache is
    truncated back (host-side bookkeeping only) so every step attends over the same number of
    tokens."""
    g = dict(ATTN_GEOMETRY, **geometry)
    hq, hkv, d, T = g["q_heads"], g["kv_heads"], g["head_dim"], g["tokens"]
    rng = np.random.default_rng(SEED + 200)
    kv_bytes = 2 * T * hkv * d * (2 if kv_dtype == "f16" else 4)
    ncopies = max(1, math.ceil(copies_min_bytes / kv_bytes))
    keys = rng.standard_normal((T, hkv, d)).astype(np.float32)
    values = rng.standard_normal((T, hkv, d)).astype(np.float32)
    caches = []
    for _ in range(ncopies):
        c = ctx.kv_cache(T + 1, hkv, d, d, dtype=kv_dtype)
        c.load(keys, values, T - 1)
        caches.append(c)
    del keys, values
    qb = ctx.to_device((2.0 * rng.standard_normal((hq, d))).astype(np.float32))
    kb = ctx.to_device(rng.standard_normal((hkv, d)).astype(np.float32))
    vb = ctx.to_device(rng.standard_normal((hkv, d)).astype(np.float32))
    ob = ctx.alloc(hq * d * 4)
    lib, h = ctx.lib, ctx.h
    hs = [c.h for c in caches]

    def step(i):
        c = hs[i % ncopies]
        if lib.oq_attention_step(h, qb.ptr, hq, kb.ptr, vb.ptr, c, ob.ptr) != 0 or \
                lib.oq_kv_cache_truncate(c, T - 1) != 0:
            raise RuntimeError(f"step {i}: {lib.oq_last_error(h).decode()}")

    step(0)  # sizes the partial-sum buffer
    ctx.sync()
    ms = timed_steps(ctx, step, steps, warmup, first=1)
    for c in caches:
        c.release()
    for b in (qb, kb, vb, ob):
        b.free()
    ms_step = ms / steps
    alg = kv_bytes + 2 * hq * d * 4 + 2 * hkv * d * 4
    return {"workload": "attention_decode", "ms_per_step": ms_step, "us_per_step": ms_step * 1e3,
            "kv_bytes": kv_bytes, "algorithmic_bytes": alg, "gbs": alg / (ms_step * 1e-3) / 1e9,
            "copies": ncopies, "geometry": g}


def run_attention_block(ctx, steps, warmup, cached=4096, copies_min_bytes=MALL_DEFEAT_BYTES, tokens=1, kv_dtype="f32"):
    """One full-attention decode block (hidden 4096, 16 query heads over 4 KV heads of 256, FFN
    12288) over 4096 cached tokens per step (oq_attention_block_step; with tokens > 1, that many
    consecutive tokens per step through oq_attention_block_steps); steps cycle over block copies
    (weights + cache) totalling >= 512 MiB; the cache is truncated back after each step."""
    rng = np.random.default_rng(SEED + 300)
    d, w, vec, keys, values, x = synth.attention_block(rng, cached=cached)
    first = oracle_amd.AttentionBlockWeights(ctx, d, w, vec)
    wb = first.weight_bytes()
    kvb = (keys.nbytes + values.nbytes) // (2 if kv_dtype == "f16" else 1)
    ncopies = max(1, math.ceil(copies_min_bytes / (wb + kvb)))
    blocks = [first] + [oracle_amd.AttentionBlockWeights(ctx, d, w, vec) for _ in range(ncopies - 1)]
    caches = []
    for _ in range(ncopies):
        c = ctx.kv_cache(cached + tokens, d["kv_heads"], d["head_dim"], d["head_dim"], dtype=kv_dtype)
        c.load(keys, values, cached)
        caches.append(c)
    xs = np.stack([x] + [rng.standard_normal(x.shape).astype(np.float32) for _ in range(tokens - 1)])
    xb, yb = ctx.to_device(xs), ctx.alloc(tokens * d["embedding"] * 4)
    lib, h = ctx.lib, ctx.h
    descs = [C.byref(b.desc) for b in blocks]
    hs = [c.h for c in caches]
    pos = (C.c_uint64 * (3 * tokens))(*[cached + t for t in range(tokens) for _ in range(3)])

    def step(i):
        c = hs[i % ncopies]
        if tokens == 1:
            rc = lib.oq_attention_block_step(h, descs[i % ncopies], c, pos, xb.ptr, yb.ptr, None)
        else:
            rc = lib.oq_attention_block_steps(h, descs[i % ncopies], c, tokens, pos, xb.ptr, yb.ptr, None)
        if rc != 0 or lib.oq_kv_cache_truncate(c, cached) != 0:
            raise RuntimeError(f"step {i}: {lib.oq_last_error(h).decode()}")

    step(0)  # checked call; sizes the block workspace
    ctx.sync()
    ms = timed_steps(ctx, step, steps, warmup, first=1)
    for b in blocks:
        b.release()
    for c in caches:
        c.release()
    for buf in (xb, yb):
        buf.free()
    ms_step = ms / steps
    return {"workload": "attention_block", "weight_bytes": wb, "kv_bytes": kvb, "copies": ncopies, "tokens": tokens,
            "ms_per_step": ms_step, "us_per_block": ms_step * 1e3, "us_per_token": ms_step * 1e3 / tokens,
            "gbs": (wb + kvb) / (ms_step * 1e-3) / 1e9, "dims": {k: v for k, v in d.items()}, "cached": cached}


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


def _timed(fn, budget_s, max_reps):
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= max_reps:
            return reps, el


def cpu_baseline(name, budget_s=10.0):
    """The reference CPU algorithm on the workload, timed on this host (a baseline, not the target).

    value: the oracle's restatement of reference_storage_matvec (decode block, sequential F32 dot,
    -O2 -ffp-contract=off) on the workload itself, one thread ("port": the reference has no Q4_K
    decoder).  Beside it: the same on the process's CPU share, and the reference's own code compiled
    from its sources (oracle/_ref/libref.so: reference_storage_dot over row ranges) on the nearest
    path it runs, Q5_K at the same shape, on one thread and on the CPU share."""
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
    threads = oracle.default_threads()
    host_cpus = os.cpu_count() or 1
    reps, el = _timed(lambda: oracle.storage_matvec(t, rows, k, sample, xhat, threads=1), budget_s, 1000)
    single = sample.nbytes * reps / el / 1e9
    reps2, el2 = _timed(lambda: oracle.storage_matvec(t, rows, k, sample, xhat, threads=threads), budget_s / 4, 2000)
    multi = sample.nbytes * reps2 / el2 / 1e9
    out = {
        "value": single, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{reps} x {rows}x{k} type-{t} matvec (oracle restatement of reference_storage_matvec, "
                  f"-O2 -ffp-contract=off), {el:.1f} s, 1 thread",
        "host_cpus": host_cpus,
        "us_per_matvec_1core": el / reps * 1e6 * (n / rows),
        "all_cores": {"value": multi, "cores": threads, "us_per_matvec": el2 / reps2 * 1e6 * (n / rows)},
    }
    if oracle.ref_available():
        q5 = synth.weights(13, np.random.default_rng(SEED + 50), rows, k)
        r1, e1 = _timed(lambda: oracle.ref_storage_matvec_threads(13, rows, k, q5, x, 1), budget_s / 2, 1000)
        rN, eN = _timed(lambda: oracle.ref_storage_matvec_threads(13, rows, k, q5, x, threads), budget_s / 4, 2000)
        out["reference_q5_k"] = {
            "kind": "reference", "unit": "GB/s",
            "sample": f"{rows}x{k} Q5_K matvec, the reference's reference_storage_dot compiled from its sources",
            "value_1core": q5.nbytes * r1 / e1 / 1e9, "us_per_matvec_1core": e1 / r1 * 1e6 * (n / rows),
            "value_all_cores": q5.nbytes * rN / eN / 1e9, "cores": threads,
            "us_per_matvec_all_cores": eN / rN * 1e6 * (n / rows)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="q4k_gemv",
                    choices=sorted(WORKLOADS) + ["copy_calibration", "deltanet_block", "attention_decode",
                                                 "attention_block"])
    ap.add_argument("--tokens", type=int, default=1, help="deltanet_block: consecutive tokens per step")
    ap.add_argument("--kv", choices=["f32", "f16"], default="f32", help="attention_decode: KV cache element type")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time the workload's K steps as one captured HIP graph launch (for kernel traces)")
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
        r = run_deltanet(ctx, args.steps, args.warmup, tokens=args.tokens, graph=args.graph)
        ctx.close()
        print(json.dumps({
            "metric": "DeltaNet decode block weight GB/s", "value": round(r["weight_gbs"], 2), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xu4 dot (i32) + f32",
            "data": "synthetic (seeded block weights, state ~ N(0, 0.01), x ~ N(0,1))",
            "config": {"workload": "Gated DeltaNet decode block, batch 1" if r["tokens"] == 1 else
                       f"Gated DeltaNet block, {r['tokens']} consecutive tokens per step (oq_deltanet_steps)", **r["dims"],
                       "weight_bytes": r["weight_bytes"], "block_copies_cycled": r["copies"],
                       "launch": "one HIP graph of the timed steps" if args.graph else "eager C-ABI calls"},
            "us_per_block": round(r["us_per_block"], 2), "tokens": r["tokens"], "us_per_token": round(r["us_per_token"], 2),
            "hbm_frac_weight_bytes": round(r["weight_gbs"] / HBM_PEAK_GBS, 4)}), flush=True)
        return
    if args.workload == "attention_block":
        r = run_attention_block(ctx, args.steps, args.warmup, tokens=args.tokens, kv_dtype=args.kv)
        ctx.close()
        print(json.dumps({
            "metric": "attention decode block GB/s (weights + KV cache)", "value": round(r["gbs"], 2), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xu4 dot (i32) + f32",
            "data": "synthetic (seeded block weights, keys/values/x ~ N(0,1))",
            "config": {"workload": "Qwen3.5 full-attention decode block, batch 1" if r["tokens"] == 1 else
                       f"Qwen3.5 full-attention block, {r['tokens']} consecutive tokens per step (oq_attention_block_steps)",
                       **r["dims"],
                       "cached_tokens": r["cached"], "weight_bytes": r["weight_bytes"], "kv_bytes": r["kv_bytes"],
                       "block_copies_cycled": r["copies"]},
            "us_per_block": round(r["us_per_block"], 2), "tokens": r["tokens"], "us_per_token": round(r["us_per_token"], 2),
            "hbm_frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}), flush=True)
        return
    if args.workload == "attention_decode":
        r = run_attention(ctx, args.steps, args.warmup, kv_dtype=args.kv)
        ctx.close()
        print(json.dumps({
            "metric": "GQA decode attention GB/s of KV cache", "value": round(r["gbs"], 2), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32" if args.kv == "f32" else "f32 (f16 cache)",
            "data": "synthetic (keys, values, k, v ~ N(0,1), q ~ N(0,4))",
            "config": {"workload": f"single-token GQA attention over an {args.kv.upper()} KV cache", **r["geometry"],
                       "kv_bytes": r["kv_bytes"], "caches_cycled": r["copies"], "kv_element": args.kv},
            "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": committed_traffic("attention_decode" if args.kv == "f32" else "attention_decode_f16")},
            "us_per_step": round(r["us_per_step"], 2)}), flush=True)
        return
    main_res = run_gpu(ctx, args.workload, args.steps, args.warmup, graph=args.graph)
    secondary = block = block2 = block4 = attn = attn16 = attn_block = attn_block2 = attn_block4 = None
    configs = {}
    if not args.no_secondary and args.workload == "q4k_gemv":
        # the other single-GPU configurations, each with its own roofline; steps of a few to a few
        # hundred microseconds, so at least 10-50 of them (a millisecond or two of GPU time each)
        secondary = run_gpu(ctx, "q4k_down_m512", max(10, args.steps // 2), max(3, args.warmup))
        for name in ("q8_0_gemv", "q6k_head", "q4k_down_m4"):
            configs[name] = run_gpu(ctx, name, max(50, args.steps), max(5, args.warmup))
        block = run_deltanet(ctx, max(20, args.steps), max(5, args.warmup))
        block2 = run_deltanet(ctx, max(20, args.steps), max(5, args.warmup), tokens=2)
        block4 = run_deltanet(ctx, max(20, args.steps), max(5, args.warmup), tokens=4)
        attn = run_attention(ctx, max(20, args.steps), max(5, args.warmup))
        attn16 = run_attention(ctx, max(20, args.steps), max(5, args.warmup), kv_dtype="f16")
        attn_block = run_attention_block(ctx, max(20, args.steps), max(5, args.warmup))
        attn_block2 = run_attention_block(ctx, max(20, args.steps), max(5, args.warmup), tokens=2)
        attn_block4 = run_attention_block(ctx, max(20, args.steps), max(5, args.warmup), tokens=4)
    ctx.close()

    t, n, k, m, desc = WORKLOADS[args.workload]
    gbs = main_res["weight_gbs"]
    achieved = main_res["algorithmic_bytes"] / (main_res["ms_per_step"] * 1e-3) / 1e9
    metric = ("Q4_K GEMV weight GB/s (% of HBM peak); M=512 Q4_K GEMM TOPS (% MFMA)" if args.workload == "q4k_gemv"
              else f"{desc}: weight GB/s")
    # m >= 16 runs on the matrix cores (f16 MFMA): bound by their peak, not by HBM
    mfma = m >= 16
    if mfma:
        roofline = {"bound": "mfma", "achieved": round(main_res["tops"], 2), "peak": MFMA_PEAK_TFLOPS["fp16"],
                    "unit": "TFLOP/s", "frac": round(main_res["tops"] / MFMA_PEAK_TFLOPS["fp16"], 4),
                    "traffic": committed_traffic(args.workload)}
    else:
        roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic(args.workload)}
    out = {
        "metric": metric,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (f32 accumulate)" if mfma else "int8xu4 dot (i32) + f32 scales",
        "data": "synthetic (seeded: weights per workload distributions, x ~ N(0,1))",
        "config": {"workload": desc, "rows": n, "cols": k, "batch": m, "weight_type": TYPE_NAMES[t],
                   "weight_copies_cycled": main_res["copies"], "seed": SEED,
                   "launch": "one HIP graph of the timed steps" if args.graph else "eager C-ABI calls",
                   "weights_sha256": main_res["weights_sha256"], "x_sha256": main_res["x_sha256"]},
        "roofline": roofline,
        "us_per_gemv": round(main_res["us_per_step"], 3),
        **({"tflops": round(main_res["tops"], 2)} if m > 1 else {}),
        **({"greedy_token_us": round(main_res["greedy_token_us"], 3),
            "head_and_token_us": round(main_res["head_and_token_us"], 3)} if "greedy_token_us" in main_res else {}),
        "hbm_frac_weight_bytes": round(gbs / HBM_PEAK_GBS, 4),
    }
    if secondary is not None:
        out["gemm_m512"] = {"tops": round(secondary["tops"], 2), "us": round(secondary["us_per_step"], 2),
                            "steps": secondary["steps"], "copies": secondary["copies"],
                            "traffic": committed_traffic("q4k_down_m512"),
                            "frac_fp16_mfma_peak": round(secondary["tops"] / MFMA_PEAK_TFLOPS["fp16"], 4),
                            "frac_int8_mfma_peak": round(secondary["tops"] / MFMA_PEAK_TFLOPS["int8"], 4)}
    for name, r in configs.items():
        alg = r["algorithmic_bytes"] / (r["ms_per_step"] * 1e-3) / 1e9
        entry = {"desc": r["desc"], "us": round(r["us_per_step"], 3), "steps": r["steps"],
                 "weight_gbs": round(r["weight_gbs"], 1), "copies": r["copies"],
                 "roofline": {"bound": "hbm", "achieved": round(alg, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(alg / HBM_PEAK_GBS, 4), "traffic": committed_traffic(name),
                              "algorithmic_bytes": r["algorithmic_bytes"]}}
        if "head_and_token_us" in r:
            entry["head_and_token_us"] = round(r["head_and_token_us"], 3)
            entry["greedy_token_us"] = round(r["greedy_token_us"], 3)
        out[name] = entry
    if block is not None:
        out["deltanet_block"] = {"us": round(block["us_per_block"], 2), "weight_gbs": round(block["weight_gbs"], 1),
                                 "hbm_frac": round(block["weight_gbs"] / HBM_PEAK_GBS, 4),
                                 "weight_bytes": block["weight_bytes"]}
    if block2 is not None:
        out["deltanet_block_2_tokens"] = {"us": round(block2["us_per_block"], 2),
                                          "us_per_token": round(block2["us_per_token"], 2),
                                          "weight_gbs": round(block2["weight_gbs"], 1)}
    if block4 is not None:
        out["deltanet_block_4_tokens"] = {"us": round(block4["us_per_block"], 2),
                                          "us_per_token": round(block4["us_per_token"], 2),
                                          "weight_gbs": round(block4["weight_gbs"], 1)}
    if attn_block is not None:
        out["attention_block"] = {"us": round(attn_block["us_per_block"], 2), "gbs": round(attn_block["gbs"], 1),
                                  "hbm_frac": round(attn_block["gbs"] / HBM_PEAK_GBS, 4),
                                  "weight_bytes": attn_block["weight_bytes"], "kv_bytes": attn_block["kv_bytes"],
                                  "cached_tokens": attn_block["cached"]}
    if attn_block2 is not None:
        out["attention_block_2_tokens"] = {"us": round(attn_block2["us_per_block"], 2),
                                           "us_per_token": round(attn_block2["us_per_token"], 2),
                                           "cached_tokens": attn_block2["cached"]}
    if attn_block4 is not None:
        out["attention_block_4_tokens"] = {"us": round(attn_block4["us_per_block"], 2),
                                           "us_per_token": round(attn_block4["us_per_token"], 2),
                                           "cached_tokens": attn_block4["cached"]}
    if attn is not None:
        out["attention_decode"] = {"us": round(attn["us_per_step"], 2), "kv_gbs": round(attn["gbs"], 1),
                                   "hbm_frac": round(attn["gbs"] / HBM_PEAK_GBS, 4), **attn["geometry"]}
    if attn16 is not None:
        out["attention_decode_f16_cache"] = {"us": round(attn16["us_per_step"], 2), "kv_gbs": round(attn16["gbs"], 1),
                                             "hbm_frac": round(attn16["gbs"] / HBM_PEAK_GBS, 4), **attn16["geometry"]}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.workload)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
