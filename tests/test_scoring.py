"""The KERNEL_RESULT scoring surface, pinned by the reference's own known answers."""
import os
import textwrap

import pytest

from ferret_amd import scoring as S

TASKS = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ferret_amd", "tasks")


def _spec(tmp_path, body):
    p = tmp_path / "t.yaml"
    p.write_text(textwrap.dedent(body))
    return S.load_task_spec(p)


BASE = """
name: t
gpu: MI355X
arch: gfx950
precision: FP8
problem: {description: d, shapes: {M: 1}}
baseline: {source: cpu}
"""


def test_parser_known_answers_from_reference_selftest():
    # Literal cases of task_spec.py:498-505.
    sample = 'noise\nKERNEL_RESULT {"Q1": 31.0, "Q2": 54.7}\nmore noise'
    sample_ref = 'KERNEL_RESULT_REFERENCE {"Q1": 25.0, "Q2": 50.0}'
    assert S.parse_kernel_output(sample) == {"Q1": 31.0, "Q2": 54.7}
    assert S.parse_reference_output(sample_ref) == {"Q1": 25.0, "Q2": 50.0}
    both = sample + "\n" + sample_ref
    assert S.parse_kernel_output(both) == {"Q1": 31.0, "Q2": 54.7}
    assert S.parse_reference_output(both) == {"Q1": 25.0, "Q2": 50.0}


def test_parser_edge_cases():
    assert S.parse_kernel_output("") == {}
    assert S.parse_reference_output("KERNEL_RESULT {\"a\": 1}") == {}
    # non-numeric values (the reference's INVALID convention) are dropped
    assert S.parse_kernel_output('KERNEL_RESULT {"a": "INVALID", "b": 2}') == {"b": 2.0}
    # reference line alone never counts as a kernel result
    assert S.parse_kernel_output('KERNEL_RESULT_REFERENCE {"a": 1.0}') == {}
    # legacy formats
    assert S.parse_kernel_output("Q_LEN=1: 31.5 TFLOPS\nQ_LEN=4: 50 TFLOPS") == {"Q1": 31.5, "Q4": 50.0}
    assert S.parse_kernel_output("Latency_ms: Q1=18.4\nTFLOPS: Q1=31.1 Q2=40") == {"Q1": 31.1, "Q2": 40.0}
    # malformed JSON falls through to the legacy parsers
    assert S.parse_kernel_output("KERNEL_RESULT {bad json}\nTFLOPS: Q3=1.5") == {"Q3": 1.5}


def test_scoring_dry_run_cases(tmp_path):
    # The reference self-test's cases A/B/C (task_spec.py:478-492).
    spec = _spec(tmp_path, BASE + """
configs:
  - {name: a, args: {}}
  - {name: b, args: {}}
  - {name: c, args: {}}
""")
    ref = {"a": 100.0, "b": 100.0, "c": 100.0}
    assert S.compute_score({"a": 100.0, "b": 100.0, "c": 100.0}, ref, spec)[0] == pytest.approx(1.0)
    assert S.compute_score({"a": 90.0, "b": 90.0, "c": 90.0}, ref, spec)[0] == pytest.approx(0.9)
    score, ratios = S.compute_score({"a": 70.0, "b": 110.0, "c": 110.0}, ref, spec)
    assert score == pytest.approx(0.7) and ratios["b"] == pytest.approx(1.1)
    assert S.should_advance_stage(0.95, ratios, spec) and not S.should_advance_stage(0.85, ratios, spec)
    # missing reference -> ratio 0
    assert S.compute_score({"a": 1.0}, {}, spec)[0] == 0.0


def test_weighted_and_focus_and_strict(tmp_path):
    spec = _spec(tmp_path, BASE + """
configs:
  - {name: a, args: {}, weight: 3}
  - {name: b, args: {}, weight: 1, target_ratio: 1.2}
scoring: weighted_avg
stage_gate: {ratio: 0.5, strict: true}
""")
    score, ratios = S.compute_score({"a": 1.0, "b": 2.0}, {"a": 1.0, "b": 1.0}, spec)
    assert score == pytest.approx((3 * 1.0 + 1 * 2.0) / 4)
    assert S.should_advance_stage(score, ratios, spec)               # a 1.0 >= 0.95, b 2.0 >= 1.2
    score, ratios = S.compute_score({"a": 1.0, "b": 1.1}, {"a": 1.0, "b": 1.0}, spec)
    assert score > 0.5 and not S.should_advance_stage(score, ratios, spec)   # strict: b 1.1 < 1.2
    spec2 = _spec(tmp_path, BASE + """
configs:
  - {name: a, args: {}}
  - {name: b, args: {}}
scoring: focus
focus_config: b
""")
    assert S.compute_score({"a": 1.0, "b": 0.5}, {"a": 1.0, "b": 1.0}, spec2)[0] == pytest.approx(0.5)


def test_validation_errors(tmp_path):
    with pytest.raises(ValueError, match="'configs' is absent"):
        _spec(tmp_path, BASE)
    with pytest.raises(ValueError, match="appears twice"):
        _spec(tmp_path, BASE + "configs:\n  - {name: a, args: {}}\n  - {name: a, args: {}}\n")
    with pytest.raises(ValueError, match="scoring 'best' is not one of"):
        _spec(tmp_path, BASE + "configs:\n  - {name: a, args: {}}\nscoring: best\n")
    with pytest.raises(ValueError, match="focus_config"):
        _spec(tmp_path, BASE + "configs:\n  - {name: a, args: {}}\nscoring: focus\nfocus_config: z\n")
    # every problem of one file is reported together
    with pytest.raises(ValueError, match="target_ratio has to be positive.*weight cannot be negative"):
        _spec(tmp_path, BASE + "configs:\n  - {name: a, args: {}, target_ratio: 0, weight: -1}\n")


def test_mi355x_task_files_load_and_match_bench_families():
    import bench
    by_name = {}
    for f in sorted(os.listdir(TASKS)):
        spec = S.load_task_spec(os.path.join(TASKS, f))
        assert spec.gpu == "MI355X" and spec.arch == "gfx950"
        by_name.update({c.name: spec for c in spec.configs})
    assert set(by_name) == set(bench.FAMILIES["all"])


def test_task_config_args_match_the_workloads_they_name():
    """Every task config names a workload whose shape is the config's args, and
    every family member is a workload."""
    import bench
    from ferret_amd import workloads as W
    for fam, keys in bench.FAMILIES.items():
        assert all(k in W.WORKLOADS for k in keys), fam
    for f in sorted(os.listdir(TASKS)):
        for c in S.load_task_spec(os.path.join(TASKS, f)).configs:
            wl = W.WORKLOADS[c.name]
            for arg, val in c.args.items():
                if arg == "zipf_s":
                    assert wl.zipf_s == val, (c.name, arg)
                else:
                    assert getattr(wl, arg) == val, (c.name, arg, getattr(wl, arg), val)


def test_bench_lines_score_through_the_parser():
    out = ('[log] noise\nKERNEL_RESULT {"x": 10.0, "y": 0.0}\n'
           'KERNEL_RESULT_REFERENCE {"x": 0.5, "y": 0.25}\nROOFLINE {"x": {"frac": 0.8}}\n')
    assert S.parse_kernel_output(out) == {"x": 10.0, "y": 0.0}
    assert S.parse_reference_output(out) == {"x": 0.5, "y": 0.25}
