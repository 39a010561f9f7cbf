"""CPU checks of the rocprofv3 trace summariser used for the committed kernel-trace profiles."""
import csv

from kernelbench_harbor_amd import rocprof_summary as rs

FIELDS = ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Workgroup_Size_X",
          "Start_Timestamp", "End_Timestamp"]


def _trace(path, launches):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        t = 0
        for i, (name, grid, dur_ns) in enumerate(launches):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Grid_Size_X": grid,
                        "Grid_Size_Y": 1, "Workgroup_Size_X": 256, "Start_Timestamp": t,
                        "End_Timestamp": t + dur_ns})
            t += dur_ns + 1000


def test_by_next_splits_coinciding_grids(tmp_path):
    # two calls per step: M=1024 (GEMM 100 us, reduce grid 1048576), M=2048 (GEMM 200 us)
    launches = []
    for _ in range(3):
        launches += [("kbh::gemm", 65536, 100_000), ("kbh::wide_reduce", 1048576, 10_000),
                     ("kbh::gemm", 65536, 200_000), ("kbh::wide_reduce", 2097152, 12_000),
                     ("other", 64, 1_000)]
    p = tmp_path / "t_kernel_trace.csv"
    _trace(p, launches)
    merged = rs.summarize(str(p), "kbh::")
    gemm = [r for r in merged if r["kernel"] == "kbh::gemm"]
    assert len(gemm) == 1 and gemm[0]["calls"] == 6 and abs(gemm[0]["avg_us"] - 150.0) < 1e-9
    split = rs.summarize(str(p), "kbh::", by_next="wide_reduce")
    by = {r["next_grid"]: r for r in split if r["kernel"] == "kbh::gemm"}
    assert sorted(by) == [1048576, 2097152]
    assert by[1048576]["calls"] == 3 and abs(by[1048576]["avg_us"] - 100.0) < 1e-9
    assert abs(by[2097152]["avg_us"] - 200.0) < 1e-9
    reduces = [r for r in split if r["kernel"] == "kbh::wide_reduce"]
    assert all(r["next_grid"] == 0 for r in reduces) and len(reduces) == 2
