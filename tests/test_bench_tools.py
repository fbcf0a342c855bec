"""bench.py's host-side tools, on the CPU: the rocprofv3 CSV summary the
committed profiles are made with, and the argument checks that refuse a run
before any GPU work."""
import csv
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def _bench(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def test_summarize_groups_traces_by_kernel_and_shape(tmp_path):
    name = "void wpcg::(anonymous namespace)::k_gemv_fast<4, 0, 1>(wpcg::(anonymous namespace)::FastBatch)"
    rows = []
    for dur, gx, gy in ((5000, 64 * 512, 3), (7000, 64 * 512, 3), (9000, 64 * 512, 3), (4000, 128 * 512, 1)):
        rows.append({"Kernel_Name": name, "Grid_Size_X": gx, "Workgroup_Size_X": 512, "Grid_Size_Y": gy,
                     "Workgroup_Size_Y": 1, "Start_Timestamp": 1000, "End_Timestamp": 1000 + dur})
    rows.append({"Kernel_Name": "__amd_rocclr_copyBuffer", "Grid_Size_X": 256 * 256, "Workgroup_Size_X": 256,
                 "Grid_Size_Y": 1, "Workgroup_Size_Y": 1, "Start_Timestamp": 0, "End_Timestamp": 2000})
    _write(tmp_path / "run_kernel_trace.csv", rows)
    r = _bench("--summarize", str(tmp_path))
    assert r.returncode == 0, r.stderr
    lines = [ln.split() for ln in r.stdout.splitlines() if ln.startswith("k_gemv_fast")]
    # (kernel, 64 x 3): 3 launches, mean 7.00 us, median 7.00; (128 x 1): 1 launch, 4.00
    assert ["64", "x", "3", "3", "7.00", "7.00"] == lines[0][-6:]
    assert ["128", "x", "1", "1", "4.00", "4.00"] == lines[1][-6:]
    r = _bench("--summarize", str(tmp_path), "--match", "copyBuffer")
    assert "k_gemv_fast" not in r.stdout and "__amd_rocclr_copyBuffer" in r.stdout


def test_summarize_counters_mean_and_last_dispatch(tmp_path):
    rows = []
    for did, v in ((1, 100.0), (2, 300.0), (3, 800.0)):
        for part in (0.25, 0.75):  # a counter may come in several rows per dispatch
            rows.append({"Dispatch_Id": did, "Kernel_Name": "__amd_rocclr_copyBuffer", "Grid_Size": 65536,
                         "Workgroup_Size": 256, "Counter_Name": "FETCH_SIZE", "Counter_Value": v * part})
    _write(tmp_path / "run_counter_collection.csv", rows)
    r = _bench("--summarize", str(tmp_path))
    assert r.returncode == 0, r.stderr
    f = [ln.split() for ln in r.stdout.splitlines() if "FETCH_SIZE" in ln][0]
    assert f[-4:] == ["FETCH_SIZE", "3", "400.0", "800.0"]


def test_summarize_without_csv_fails(tmp_path):
    assert _bench("--summarize", str(tmp_path)).returncode == 1


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_unknown_section_is_refused():
    r = _bench("--only", "cfg9")
    assert r.returncode == 2 and "cfg9" in r.stderr
