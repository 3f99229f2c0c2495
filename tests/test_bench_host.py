"""CPU checks of bench.py's host logic: the in-run traffic measurement stands
down (returns None, starts no child process) where it cannot or must not run,
the --gpus guard, the committed traffic records the fallback reads, and the
correctness gate's handling of non-finite outputs."""
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


def test_published_figures_name_existing_workloads_and_convert_to_their_unit():
    from ferret_amd import workloads as W

    class R:  # the Runner fields published_of reads
        pass

    for key, p in bench.PUBLISHED.items():
        wl = W.WORKLOADS[key]
        assert p["unit"] == "TFLOP/s" and p["value"] > 0 and p["source"]
        r = R()
        r.flops = W.flops(wl)
        # a kernel time at which this run matches the published figure exactly
        us = r.flops / (p["value"] * 1e12) * 1e6
        got = bench.published_of(wl, r, us)
        assert got["ratio"] == pytest.approx(1.0, abs=1e-3) and got["this_run"] == pytest.approx(p["value"], rel=1e-3)
        assert bench.published_of(wl, r, 0.0) is None
    # GateUp M=16: 2 * 16 * 24576 * 4096 flops; the reference's kernel runs them at 62.91 TFLOP/s
    assert W.flops(W.WORKLOADS["qwen3_gateup_M16"]) == 2 * 16 * 24576 * 4096
    assert bench.published_of(W.WORKLOADS["dsv3_fp8_M4096"], R(), 100.0) is None


def test_gate_rejects_non_finite_outputs():
    """An all-NaN or partly-Inf output has no finite error to report (the
    metric skips those elements), so the gate must fail it on the count."""
    import numpy as np
    from oracle import metrics as MT
    ref = np.random.default_rng(0).standard_normal((8, 64)).astype(np.float32)
    assert bench.passes_gate(*MT.fp8_rel_err(ref.copy(), ref))
    for bad in (np.full_like(ref, np.nan), np.where(np.arange(ref.size).reshape(ref.shape) == 5, np.inf, ref)):
        err, nbad = MT.fp8_rel_err(bad, ref)
        assert nbad > 0 and err < 1e-2            # the error alone would pass
        assert not bench.passes_gate(err, nbad)
    assert not bench.passes_gate(*MT.fp8_rel_err(ref * 1.02, ref))
