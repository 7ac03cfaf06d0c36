"""bench.py's reduction of a rocprofv3 kernel trace (CPU only): the headline kernel's average duration and its
interval from the previous kernel's end on the same queue, from a synthetic trace with two queues, kernels of
other grids and names, and torch kernels in between."""
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

FIELDS = ["Kernel_Name", "Queue_Id", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y",
          "Workgroup_Size_X"]
HEAD = "void mimo::decode_gateup_kernel<8, true, false, true>(mimo::ExpertsArgs, int)"


def _row(name, q, t0, t1, gx, gy=1, wx=256):
    return {"Kernel_Name": name, "Queue_Id": q, "Start_Timestamp": t0, "End_Timestamp": t1, "Grid_Size_X": gx,
            "Grid_Size_Y": gy, "Workgroup_Size_X": wx}


def test_trace_parse_headline(tmp_path, capsys):
    rows = []
    t = 1_000_000
    for step in range(3):               # router (2 us) -> gap 1 us -> headline (16 + step us) -> down (9 us)
        rows.append(_row("void mimo::router_logits_small_kernel<2>(mimo::RouterSmallArgs)", 1, t, t + 2000, 69632))
        t += 3000
        rows.append(_row(HEAD, 1, t, t + 16000 + 1000 * step, 32768, 8))
        t += 16000 + 1000 * step
        rows.append(_row("void mimo::decode_down_combine_kernel<8, true>(mimo::ExpertsArgs, int)", 1, t, t + 9000,
                         262144, 1, 1024))
        t += 9000
    # the same kernel on another grid (a 2-row step) and on another queue must not count as the headline
    rows.append(_row(HEAD, 1, t + 500, t + 30500, 32768, 16))
    rows.append(_row("void at::native::elementwise_kernel<128, 4>(int, float)", 2, 0, 5000, 1024))
    rows.append(_row(HEAD, 2, 6000, 26000, 32768, 16))
    d = tmp_path / "trace"
    d.mkdir()
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow(r)
    out = tmp_path / "trace.json"
    bench.trace_parse(str(d), str(out))
    got = json.loads(out.read_text())["decode_gateup_kernel:decode_m1"]
    assert got["launches"] == 3
    assert abs(got["avg_us"] - 17.0) < 1e-9                      # (16 + 17 + 18) / 3
    assert abs(got["after_previous_end_us"] - 18.0) < 1e-9       # duration + the 1 us gap after the router
    table = capsys.readouterr().out
    assert "| `decode_gateup_kernel<8, true, false, true>` | 32768×8 | 256 | 3 | 17.00 |" in table
    assert "elementwise" not in table                            # torch's kernels are left out
