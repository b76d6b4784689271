"""The profile summariser's traffic figures (oracle_amd/profsum.py) on synthetic rocprofv3 counter
tables: per-dispatch medians scaled by the copy calibration, and, per launch, dispatches of one
kernel name kept apart by grid size."""

import csv
import json

from oracle_amd import profsum

FIELDS = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_table(directory, rows):
    directory.mkdir(parents=True)
    with open(directory / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(FIELDS, r)))


def tables(tmp_path):
    # a step of three launches: gemv_block (grid 1000), delta, gemv_block again (grid 3000);
    # copy calibration: 1000 KiB counted for 1024000 bytes (scale 1), writes counted at half
    step = [("gemv_block<1>", 1000, 40.0, 4.0), ("delta", 64, 8.0, 8.0), ("gemv_block<1>", 3000, 120.0, 12.0)]
    fetch, write = [], []
    for s in range(3):
        for i, (name, grid, f, w) in enumerate(step):
            d = 3 * s + i
            fetch.append((d, grid, name, "FETCH_SIZE", f + s))  # medians: the middle step's value
            write.append((d, grid, name, "WRITE_SIZE", w + s))
    write_table(tmp_path / "f", fetch)
    write_table(tmp_path / "w", write)
    write_table(tmp_path / "cf", [(0, 256, "copyBuffer", "FETCH_SIZE", 1000.0)])
    write_table(tmp_path / "cw", [(0, 256, "copyBuffer", "WRITE_SIZE", 500.0)])
    return [str(tmp_path / n) for n in ("f", "w", "cf", "cw")]


def test_traffic_per_launch_keeps_same_named_kernels_apart(tmp_path):
    f, w, cf, cw = tables(tmp_path)
    out = profsum.traffic_per_launch("", f, w, cf, cw, 1024000)
    assert [(x["kernel"], x["grid_size"]) for x in out["launches"]] == [
        ("gemv_block<1>", "1000"), ("delta", "64"), ("gemv_block<1>", "3000")]
    first = out["launches"][0]
    assert first["dispatches"] == [3, 3]
    assert first["fetch_bytes"] == 41.0 * 1024.0
    assert first["write_bytes"] == 5.0 * 1024.0 * 2.0
    assert out["launches"][2]["traffic_bytes"] == (121.0 + 2.0 * 13.0) * 1024.0
    json.dumps(out)


def test_traffic_by_name_matches_every_launch_of_it(tmp_path):
    f, w, cf, cw = tables(tmp_path)
    one = profsum.traffic("delta", f, w, cf, cw, 1024000)
    assert one["fetch_bytes"] == 9.0 * 1024.0 and one["write_bytes"] == 9.0 * 1024.0 * 2.0
    both = profsum.traffic("gemv_block", f, w, cf, cw, 1024000)  # the two launches' median mixed
    assert both["dispatches"] == [6, 6]


def test_dispatches_in_start_order_with_gaps(tmp_path):
    d = tmp_path / "trace"
    d.mkdir()
    fields = ["Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    rows = [("k<12>", 3000, 10000), ("other", 100, 900), ("k<12>", 1000, 2000), ("k<12>", 12000, 19500)]
    with open(d / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(fields, r)))
    r = profsum.dispatches(str(d), "k<12>")
    assert r["us"] == [1.0, 7.0, 7.5] and r["gap_us"] == [1.0, 2.0]
    assert r["median_us"] == 7.0 and abs(r["mean_us"] - 15.5 / 3) < 1e-12
    assert profsum.dispatches(str(d), "k<12>", last=2)["us"] == [7.0, 7.5]
