"""Host-side parts of the measurement contract, on the CPU: bench.py refuses more than one
GPU with a message, the traffic figure is read only from a summary measured on the current
sources (and the committed summaries are), the CPU baseline's thread rule, and the
calibration arithmetic of the traffic summary on a synthetic counter file."""
import csv
import json
import os
import subprocess
import sys

import pytest

import bench
from filtervectorcode_refactor_amd import profile_summaries as PS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_gpus_above_one_exit_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_traffic_read_only_from_current_summary(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    (tmp_path / "profiles").mkdir()
    assert bench.read_traffic("cfgX") == (None, "not measured")
    p = tmp_path / "profiles" / "traffic_select_cross_cfgX.txt"
    p.write_text("traffic_bytes_per_launch: 123\nkernel_source_sha256: " + "0" * 64 + "\n")
    value, status = bench.read_traffic("cfgX")
    assert value is None and status.startswith("stale")
    p.write_text("traffic_bytes_per_launch: 123\nkernel_source_sha256: " + bench.kernel_source_digest() + "\n")
    assert bench.read_traffic("cfgX") == (123.0, "measured (traffic_select_cross_cfgX.txt)")


@pytest.mark.parametrize("cfg", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_committed_summaries_match_the_sources(cfg):
    """The committed traffic summaries were measured on the sources in the tree (a change
    of the kernels, the launch code or the HIP flags needs a new measurement)."""
    value, status = bench.read_traffic(cfg)
    assert value is not None and value > 0, status


def test_cpu_baseline_thread_rule(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "7")
    assert bench.baseline_threads() == 7
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.baseline_threads() == len(os.sched_getaffinity(0))
    inv = bench.cpu_inventory()
    assert inv["logical_cpus"] == os.cpu_count() and inv["nproc"] == len(os.sched_getaffinity(0))


def _counter_csv(path, rows):
    path.mkdir(parents=True)
    cols = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path / "p_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(cols, r)))


def test_traffic_summary_calibration(tmp_path, monkeypatch):
    """The copy kernel moves 1 GiB: FETCH_SIZE reading 524,288 KiB scales the select's
    reading by 2, WRITE_SIZE reading 1,048,576 KiB by 1; the first select dispatch counts."""
    sel = "ung_select_kernel<8, 1, false, 2, true>(SelectParams)"
    copy = "__amd_rocclr_copyBuffer"
    d = tmp_path / "meas"
    _counter_csv(d / "FETCH_SIZE", [(3, sel, 2925568, 1000.0, 0, 15_000_000), (4, sel, 2925568, 999.0, 0, 1),
                                    (9, copy, 262144, 524288.0, 0, 1), (10, copy, 64, 4.0, 0, 1)])
    _counter_csv(d / "WRITE_SIZE", [(3, sel, 2925568, 10.0, 0, 16_000_000), (9, copy, 262144, 1048576.0, 0, 1)])
    monkeypatch.setattr(PS, "ROOT", str(tmp_path))
    (tmp_path / "profiles").mkdir()
    PS.traffic("cfg2", str(d))
    text = (tmp_path / "profiles" / "traffic_select_cross_cfg2.txt").read_text()
    want = int(round(1000.0 * 1024 * 2 + 10.0 * 1024 * 1))
    assert f"traffic_bytes_per_launch: {want}\n" in text
    assert "kernel_source_sha256: " + bench.kernel_source_digest() in text
    assert "duration 15.00 ms (FETCH pass) / 16.00 ms (WRITE pass)" in text
