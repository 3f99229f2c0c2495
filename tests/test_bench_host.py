"""CPU checks of bench.py's host logic: the in-run traffic measurement stands
down (returns None, starts no child process) where it cannot or must not run,
the --gpus guard, and the committed traffic records the fallback reads."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _no_child(*a, **k):
    raise AssertionError("measure_traffic started a child process")


def test_measure_traffic_without_rocprofv3(monkeypatch):
    import shutil
    monkeypatch.setattr(shutil, "which", lambda name: None)
    monkeypatch.setattr(subprocess, "Popen", _no_child)
    assert bench.measure_traffic("dsv3_fp8_M4096") is None


def test_measure_traffic_under_an_outer_profiler(monkeypatch):
    import shutil
    monkeypatch.setattr(shutil, "which", lambda name: "/opt/rocm/bin/rocprofv3")
    monkeypatch.setattr(subprocess, "Popen", _no_child)
    monkeypatch.setenv("ROCPROF_KERNEL_TRACE", "1")
    assert bench.measure_traffic("dsv3_fp8_M4096") is None
    monkeypatch.delenv("ROCPROF_KERNEL_TRACE")
    monkeypatch.setenv("LD_PRELOAD", "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so")
    assert bench.measure_traffic("dsv3_fp8_M4096") is None


def test_measure_traffic_needs_a_committed_kernel_name(monkeypatch):
    import shutil
    monkeypatch.setattr(shutil, "which", lambda name: "/opt/rocm/bin/rocprofv3")
    monkeypatch.setattr(subprocess, "Popen", _no_child)
    assert bench.measure_traffic("no_such_workload") is None


def test_committed_traffic_records_name_their_kernel():
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as fh:
        recs = json.load(fh)
    assert bench.DEFAULT_WORKLOAD in recs
    for key, rec in recs.items():
        assert rec.get("kernel"), key
        assert rec["bytes_per_launch"] == rec["fetch_bytes"] + rec["write_bytes"], key
        assert bench.traffic_of(key) == rec["bytes_per_launch"]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "--gpus 2 is not supported" in r.stderr
