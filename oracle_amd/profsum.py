"""Summaries of rocprofv3 output for the profiles/ directory (run by oracle_amd/profile.sh).

    python -m oracle_amd.profsum stats DIR [--match SUBSTR ...]
        per-kernel call count and durations from DIR/**/*kernel_stats.csv
    python -m oracle_amd.profsum traffic --kernel SUBSTR --fetch DIR --write DIR
                                         --copy-fetch DIR --copy-write DIR --copy-bytes N
        HBM bytes per dispatch of the matching kernel: FETCH_SIZE and WRITE_SIZE (KiB per
        dispatch, median over dispatches) each scaled by bytes / counter of a device-to-device
        copy of N bytes profiled the same way.  With --per-kernel, one entry per launch of the
        step instead: dispatches grouped by kernel name and grid size (a kernel launched twice per
        step with different grids, e.g. a block's in-projection and gate/up GEMVs, is two
        entries), in order of first dispatch.
    python -m oracle_amd.profsum dispatches --kernel SUBSTR [--last N] DIR
        durations of the matching kernel's dispatches in start order from DIR/**/*kernel_trace.csv
        (the last N), their mean and median, and the GPU's idle gaps between them
    python -m oracle_amd.profsum counters --kernel SUBSTR --cus N --simds-per-cu 4 DIR [DIR ...]
        median per dispatch of every counter collected under the DIRs for the matching kernel,
        plus derived figures: MFMA-busy fraction of each SIMD's active cycles
        (SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE / XCDs)), MFMA rate of the dispatch
        (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 flop / GRBM_GUI_ACTIVE cycles).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import statistics
import sys


def _rows(directory: str, pattern: str) -> list[dict]:
    rows: list[dict] = []
    for f in sorted(glob.glob(f"{directory}/**/{pattern}", recursive=True)):
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def kernel_stats(directory: str, match: list[str] | None = None) -> list[dict]:
    out = []
    for r in _rows(directory, "*kernel_stats.csv"):
        name = r["Name"]
        if match and not any(m in name for m in match):
            continue
        out.append({
            "kernel": name,
            "calls": int(r["Calls"]),
            "avg_us": float(r["AverageNs"]) / 1e3,
            "min_us": float(r["MinNs"]) / 1e3,
            "max_us": float(r["MaxNs"]) / 1e3,
            "percent": float(r["Percentage"]),
        })
    return out


def counter_median(directory: str, kernel: str, counter: str) -> tuple[float, int]:
    vals = [float(r["Counter_Value"]) for r in _rows(directory, "*counter_collection.csv")
            if kernel in r["Kernel_Name"] and r["Counter_Name"] == counter]
    if not vals:
        raise SystemExit(f"no {counter} samples for kernel matching {kernel!r} under {directory}")
    return statistics.median(vals), len(vals)


def _launch_key(r: dict) -> tuple[str, str]:
    return r["Kernel_Name"], r.get("Grid_Size", "")


def traffic_per_launch(kernel: str, fetch: str, write: str, copy_fetch: str, copy_write: str, copy_bytes: int,
                       copy_kernel: str = "copyBuffer") -> dict:
    cf, _ = counter_median(copy_fetch, copy_kernel, "FETCH_SIZE")
    cw, _ = counter_median(copy_write, copy_kernel, "WRITE_SIZE")
    f_scale = copy_bytes / (cf * 1024.0)
    w_scale = copy_bytes / (cw * 1024.0)
    groups: dict[tuple[str, str], dict[str, list[float]]] = {}
    for directory, counter in ((fetch, "FETCH_SIZE"), (write, "WRITE_SIZE")):
        rows = [r for r in _rows(directory, "*counter_collection.csv")
                if kernel in r["Kernel_Name"] and r["Counter_Name"] == counter]
        rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0) or 0))
        for r in rows:
            groups.setdefault(_launch_key(r), {"FETCH_SIZE": [], "WRITE_SIZE": []})[counter].append(
                float(r["Counter_Value"]))
    launches = []
    for (name, grid), v in groups.items():
        if not v["FETCH_SIZE"] or not v["WRITE_SIZE"]:
            continue
        kf, kw = statistics.median(v["FETCH_SIZE"]), statistics.median(v["WRITE_SIZE"])
        launches.append({
            "kernel": name, "grid_size": grid, "dispatches": [len(v["FETCH_SIZE"]), len(v["WRITE_SIZE"])],
            "fetch_kib_per_dispatch": kf, "write_kib_per_dispatch": kw,
            "fetch_bytes": kf * 1024.0 * f_scale, "write_bytes": kw * 1024.0 * w_scale,
            "traffic_bytes": kf * 1024.0 * f_scale + kw * 1024.0 * w_scale,
        })
    if not launches:
        raise SystemExit(f"no FETCH_SIZE / WRITE_SIZE samples for kernels matching {kernel!r}")
    return {"kernel_match": kernel, "copy_bytes": copy_bytes, "copy_fetch_kib": cf, "copy_write_kib": cw,
            "fetch_scale": f_scale, "write_scale": w_scale, "launches": launches}


def traffic(kernel: str, fetch: str, write: str, copy_fetch: str, copy_write: str, copy_bytes: int,
            copy_kernel: str = "copyBuffer") -> dict:
    kf, nf = counter_median(fetch, kernel, "FETCH_SIZE")
    kw, nw = counter_median(write, kernel, "WRITE_SIZE")
    cf, _ = counter_median(copy_fetch, copy_kernel, "FETCH_SIZE")
    cw, _ = counter_median(copy_write, copy_kernel, "WRITE_SIZE")
    f_scale = copy_bytes / (cf * 1024.0)
    w_scale = copy_bytes / (cw * 1024.0)
    return {
        "kernel": kernel,
        "fetch_kib_per_dispatch": kf, "write_kib_per_dispatch": kw, "dispatches": [nf, nw],
        "copy_bytes": copy_bytes, "copy_fetch_kib": cf, "copy_write_kib": cw,
        "fetch_scale": f_scale, "write_scale": w_scale,
        "fetch_bytes": kf * 1024.0 * f_scale, "write_bytes": kw * 1024.0 * w_scale,
        "traffic_bytes": kf * 1024.0 * f_scale + kw * 1024.0 * w_scale,
    }


def dispatches(directory: str, kernel: str, last: int | None = None) -> dict:
    rows = [r for r in _rows(directory, "*kernel_trace.csv") if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if last:
        rows = rows[-last:]
    if not rows:
        raise SystemExit(f"no dispatches of a kernel matching {kernel!r} under {directory}")
    us = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]
    gaps = [(int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1e3 for a, b in zip(rows, rows[1:])]
    return {"kernel": rows[0]["Kernel_Name"], "dispatches": len(us), "mean_us": statistics.mean(us),
            "median_us": statistics.median(us), "us": [round(u, 3) for u in us],
            "gap_us": [round(g, 3) for g in gaps]}


def counters(kernel: str, dirs: list[str], cus: int, simds_per_cu: int, xcds: int) -> dict:
    vals: dict[str, list[float]] = {}
    for d in dirs:
        for r in _rows(d, "*counter_collection.csv"):
            if kernel in r["Kernel_Name"]:
                vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    med = {k: statistics.median(v) for k, v in sorted(vals.items())}
    out: dict = {"kernel": kernel, "dispatches": {k: len(v) for k, v in sorted(vals.items())}, "median": med}
    gui = med.get("GRBM_GUI_ACTIVE")
    if gui:
        cycles = gui / xcds  # GRBM_GUI_ACTIVE is summed over the XCDs
        out["active_cycles_per_xcd"] = cycles
        if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
            out["mfma_busy_frac"] = med["SQ_VALU_MFMA_BUSY_CYCLES"] / (cus * simds_per_cu * cycles)
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in med:
            # one MOPS unit = 512 flop; rate at the cycles of the dispatch (clock not assumed)
            out["mfma_f16_flop_per_cycle_per_cu"] = med["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512.0 / (cycles * cus)
        if "SQ_INSTS_VALU_MFMA_MOPS_I8" in med:
            out["mfma_i8_op_per_cycle_per_cu"] = med["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512.0 / (cycles * cus)
    if med.get("SQ_INSTS_MFMA"):
        # vector (non-MFMA) instructions issued per MFMA instruction
        out["valu_per_mfma"] = (med.get("SQ_INSTS_VALU", 0.0) - med["SQ_INSTS_MFMA"]) / med["SQ_INSTS_MFMA"]
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--match", nargs="*")
    t = sub.add_parser("traffic")
    for k in ("kernel", "fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--per-kernel", action="store_true")
    d = sub.add_parser("dispatches")
    d.add_argument("--kernel", required=True)
    d.add_argument("--last", type=int)
    d.add_argument("dir")
    c = sub.add_parser("counters")
    c.add_argument("--kernel", required=True)
    c.add_argument("--cus", type=int, default=256)
    c.add_argument("--simds-per-cu", type=int, default=4)
    c.add_argument("--xcds", type=int, default=8)
    c.add_argument("dirs", nargs="+")
    a = ap.parse_args(argv)
    if a.cmd == "counters":
        print(json.dumps(counters(a.kernel, a.dirs, a.cus, a.simds_per_cu, a.xcds), indent=1))
        return 0
    if a.cmd == "dispatches":
        r = dispatches(a.dir, a.kernel, a.last)
        print(f"# {r['dispatches']} dispatches: mean {r['mean_us']:.3f} us, median {r['median_us']:.3f} us")
        print("# durations (us): " + " ".join(f"{u:.2f}" for u in r["us"]))
        print("# gaps before the next (us): " + " ".join(f"{g:.2f}" for g in r["gap_us"]))
        return 0
    if a.cmd == "stats":
        rows = kernel_stats(a.dir, a.match)
        print(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'pct':>7}  kernel")
        for r in rows:
            print(f"{r['calls']:>6} {r['avg_us']:>10.3f} {r['min_us']:>10.3f} {r['max_us']:>10.3f} "
                  f"{r['percent']:>7.2f}  {r['kernel'][:160]}")
        return 0
    fn = traffic_per_launch if a.per_kernel else traffic
    print(json.dumps(fn(a.kernel, a.fetch, a.write, a.copy_fetch, a.copy_write, a.copy_bytes), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
