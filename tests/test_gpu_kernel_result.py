"""End to end on the GPU: `bench.py --kernel-result` for one family prints the
reference's KERNEL_RESULT / KERNEL_RESULT_REFERENCE lines, the task file's
configs parse out of them with the reference's regexes, every config passed
its oracle gate (a failing one would read 0.0), and the task scores above 0.

The reference's own protocol (task_spec.py:277-430): the kernel binary prints
these lines, task_spec parses and scores them.  Short timing here (20
iterations, 0.2 s warmup): the test checks the surface, not the figures.
"""
import json
import os
import subprocess
import sys

import pytest

from ferret_amd import scoring as S

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_kernel_result_lines_score_through_the_task_file(hip):
    task = S.load_task_spec(os.path.join(ROOT, "ferret_amd", "tasks", "mi355x-kimi-w13-tp8.yaml"))
    print("[case] bench.py --kernel-result kimi_tp8", flush=True)
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--kernel-result", "kimi_tp8",
                          "--iters", "20", "--warmup-s", "0.2", "--cpu-budget", "1"],
                         capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert res.returncode == 0, res.stderr[-2000:]
    got = S.parse_kernel_output(res.stdout)
    ref = S.parse_reference_output(res.stdout)
    names = [c.name for c in task.configs]
    assert sorted(got) == sorted(names) and sorted(ref) == sorted(names)
    assert all(got[n] > 0.0 for n in names), got          # 0.0 marks a config that failed its gate
    assert all(ref[n] > 0.0 for n in names), ref
    roof = json.loads(next(line for line in res.stdout.splitlines() if line.startswith("ROOFLINE "))[9:])
    assert all(roof[n]["valid"] for n in names), roof
    score, ratios = S.compute_score(got, ref, task)
    assert score > 0.0 and set(ratios) == set(names)
