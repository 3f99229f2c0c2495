"""task.yaml loading and KERNEL_RESULT scoring, behaviour-compatible with ferret.

Mirrors the reference's scoring surface so that bench output from this build is
parsed and scored unchanged:

* ``load_task_spec``      — task_spec.py:104-269 (required keys, validation errors)
* ``parse_kernel_output`` — task_spec.py:283-328 (KERNEL_RESULT JSON line, then
  the legacy "Q_LEN=N: x TFLOPS" and "TFLOPS: Q1=..." forms)
* ``parse_reference_output`` — task_spec.py:331-356 (KERNEL_RESULT_REFERENCE)
* ``compute_score`` / ``should_advance_stage`` — task_spec.py:364-430
  (ratio = kernel / reference per config; min_ratio | weighted_avg | focus)

The two result-line regular expressions are the reference's exactly (an
interface: a line must match both parsers the same way).
"""
from __future__ import annotations

import json
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import yaml

SCORING_POLICIES = ("min_ratio", "weighted_avg", "focus")

RESULT_RE = re.compile(r"KERNEL_RESULT(?!_REFERENCE)\s+(\{[^\n]*\})")
REFERENCE_RE = re.compile(r"KERNEL_RESULT_REFERENCE\s+(\{[^\n]*\})")
_QLEN_RE = re.compile(r"Q_LEN=(\d+):\s*([\d.]+)\s*TFLOPS")
_QSHORT_RE = re.compile(r"Q(\d+)=([\d.]+)")


@dataclass
class ConfigEntry:
    name: str
    args: dict[str, Any]
    target_ratio: float = 0.95
    weight: float = 1.0


@dataclass
class StageGate:
    ratio: float = 0.9
    strict: bool = False


@dataclass
class TaskSpec:
    name: str
    gpu: str
    arch: str
    precision: str
    description: str
    shapes: dict[str, Any]
    baseline_source: str
    configs: list[ConfigEntry]
    scoring: str = "min_ratio"
    focus_config: str = ""
    stage_gate: StageGate = field(default_factory=StageGate)
    constraints: list[str] = field(default_factory=list)
    hints: list[str] = field(default_factory=list)
    references: list[str] = field(default_factory=list)
    result_keys: list[str] = field(default_factory=list)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _number(value, what: str) -> float:
    try:
        return float(value)
    except (TypeError, ValueError) as exc:
        raise ValueError(f"{what} must be a number") from exc


def load_task_spec(path: str | Path) -> TaskSpec:
    """Load and validate a task.yaml; raise ValueError with a clear message on bad input."""
    path = Path(path)
    _require(path.exists(), f"task spec not found: {path}")
    try:
        data = yaml.safe_load(path.read_text())
    except yaml.YAMLError as exc:
        raise ValueError(f"task spec is not valid YAML: {exc}") from exc
    _require(isinstance(data, dict), f"task spec must be a YAML mapping, got {type(data).__name__}")
    for key in ("name", "gpu", "arch", "precision", "problem", "baseline", "configs"):
        _require(key in data, f"task spec missing required field: {key}")

    problem = data["problem"]
    _require(isinstance(problem, dict), "task spec.problem must be a mapping")
    _require("description" in problem, "task spec.problem missing required field: description")
    _require("shapes" in problem, "task spec.problem missing required field: shapes")
    _require(isinstance(problem["shapes"], dict), "task spec.problem.shapes must be a mapping")
    baseline = data["baseline"]
    _require(isinstance(baseline, dict), "task spec.baseline must be a mapping")
    _require("source" in baseline, "task spec.baseline missing required field: source")

    raw_configs = data["configs"]
    _require(isinstance(raw_configs, list) and raw_configs, "task spec.configs must be a non-empty list")
    configs: list[ConfigEntry] = []
    names: set[str] = set()
    for i, c in enumerate(raw_configs):
        _require(isinstance(c, dict), f"config[{i}] must be a mapping")
        for req in ("name", "args"):
            _require(req in c, f"config[{i}] missing required field: {req}")
        name = str(c["name"])
        _require(name not in names, f"duplicate config name: {name}")
        names.add(name)
        _require(isinstance(c["args"], dict), f"config[{i}] ({name}).args must be a mapping")
        target = _number(c.get("target_ratio", 0.95), f"config[{i}] ({name}).target_ratio")
        weight = _number(c.get("weight", 1.0), f"config[{i}] ({name}).weight")
        _require(target > 0, f"config[{i}] ({name}).target_ratio must be > 0")
        _require(weight >= 0, f"config[{i}] ({name}).weight must be >= 0")
        configs.append(ConfigEntry(name, c["args"], target, weight))

    scoring = str(data.get("scoring", "min_ratio"))
    _require(scoring in SCORING_POLICIES,
             f"invalid scoring policy: {scoring!r}. Must be one of {SCORING_POLICIES}")
    focus = str(data.get("focus_config", ""))
    if scoring == "focus":
        _require(bool(focus), "scoring=focus requires focus_config to be set")
        _require(focus in names, f"focus_config {focus!r} not in configs list (available: {[c.name for c in configs]})")
    if scoring == "weighted_avg":
        _require(sum(c.weight for c in configs) > 0,
                 "scoring=weighted_avg requires at least one config with weight > 0")

    gate = data.get("stage_gate", {}) or {}
    _require(isinstance(gate, dict), "task spec.stage_gate must be a mapping")
    gate_ratio = _number(gate.get("ratio", 0.9), "task spec.stage_gate.ratio")
    _require(gate_ratio > 0, "task spec.stage_gate.ratio must be > 0")

    output = data.get("output", {}) or {}
    _require(isinstance(output, dict), "task spec.output must be a mapping")
    lists = {}
    for key in ("constraints", "hints", "references"):
        vals = list(data.get(key, []) or [])
        _require(all(isinstance(v, str) for v in vals), f"task spec.{key} must be a list of strings")
        lists[key] = vals

    return TaskSpec(
        name=str(data["name"]), gpu=str(data["gpu"]), arch=str(data["arch"]),
        precision=str(data["precision"]), description=str(problem["description"]),
        shapes=dict(problem["shapes"]), baseline_source=str(baseline["source"]), configs=configs,
        scoring=scoring, focus_config=focus, stage_gate=StageGate(gate_ratio, bool(gate.get("strict", False))),
        constraints=lists["constraints"], hints=lists["hints"], references=lists["references"],
        result_keys=list(output.get("result_keys", [c.name for c in configs])))


def _json_numbers(text: str) -> dict[str, float] | None:
    try:
        data = json.loads(text)
    except (json.JSONDecodeError, ValueError, TypeError):
        return None
    if not isinstance(data, dict):
        return None
    # bool is an int subclass in Python; the reference keeps it (float(True) == 1.0)
    return {str(k): float(v) for k, v in data.items() if isinstance(v, (int, float))}


def parse_kernel_output(stdout: str) -> dict[str, float]:
    """Per-config TFLOPS from a bench's stdout (first KERNEL_RESULT line wins)."""
    if not stdout:
        return {}
    m = RESULT_RE.search(stdout)
    if m:
        parsed = _json_numbers(m.group(1))
        if parsed is not None:
            return parsed
    results = {f"Q{q}": float(v) for q, v in _QLEN_RE.findall(stdout)}
    if results:
        return results
    for line in stdout.split("\n"):
        if line.lstrip().startswith("TFLOPS:"):
            for q, v in _QSHORT_RE.findall(line):
                results[f"Q{q}"] = float(v)
    return results


def parse_reference_output(stdout: str) -> dict[str, float]:
    """Per-config reference TFLOPS from the KERNEL_RESULT_REFERENCE line ({} if absent)."""
    if not stdout:
        return {}
    m = REFERENCE_RE.search(stdout)
    if not m:
        return {}
    return _json_numbers(m.group(1)) or {}


def compute_score(results: dict[str, float], reference: dict[str, float], spec: TaskSpec):
    """(aggregate score, per-config ratios); ratio 0 where the reference is missing or <= 0."""
    ratios: dict[str, float] = {}
    for cfg in spec.configs:
        ref = reference.get(cfg.name, 0.0)
        ratios[cfg.name] = results.get(cfg.name, 0.0) / ref if ref > 0 else 0.0
    if not ratios:
        return 0.0, ratios
    if spec.scoring == "min_ratio":
        return min(ratios.values()), ratios
    if spec.scoring == "weighted_avg":
        total = sum(c.weight for c in spec.configs)
        if total <= 0:
            return 0.0, ratios
        return sum(c.weight * ratios[c.name] for c in spec.configs) / total, ratios
    if spec.scoring == "focus":
        return ratios.get(spec.focus_config, 0.0), ratios
    return 0.0, ratios


def should_advance_stage(score: float, ratios: dict[str, float], spec: TaskSpec) -> bool:
    if score < spec.stage_gate.ratio:
        return False
    if spec.stage_gate.strict:
        return all(ratios.get(c.name, 0.0) >= c.target_ratio for c in spec.configs)
    return True
