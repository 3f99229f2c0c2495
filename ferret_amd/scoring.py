"""task.yaml loading and KERNEL_RESULT scoring, behaviour-compatible with ferret.

Mirrors the reference's scoring surface so that bench output from this library is
parsed and scored unchanged:

* ``load_task_spec``      — loads the task.yaml schema of tasks/template.yaml (this
  module's own validator; the reference's is task_spec.py:104-269)
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


# ---------------------------------------------------------------------------- task.yaml

# The task.yaml schema this loader accepts (the keys the reference's task
# files use, tasks/template.yaml): top-level keys with their YAML kinds, the
# required sub-keys of the two nested mappings, and per-config keys with
# defaults.  Everything is checked and every problem is reported in one error.
_TOP_LEVEL = {"name": str, "gpu": str, "arch": str, "precision": str, "problem": dict, "baseline": dict,
              "configs": list}
_NESTED = {"problem": ("description", "shapes"), "baseline": ("source",)}
_CONFIG_DEFAULTS = {"target_ratio": 0.95, "weight": 1.0}
_OPTIONAL_LISTS = ("constraints", "hints", "references")


class _Problems:
    """Collects schema violations; `raise_if_any` turns them into one ValueError."""

    def __init__(self, where: str):
        self.where = where
        self.items: list[str] = []

    def add(self, msg: str) -> None:
        self.items.append(msg)

    def raise_if_any(self) -> None:
        if self.items:
            raise ValueError(f"{self.where}: " + "; ".join(self.items))


def _as_float(value, problems: _Problems, label: str, default: float) -> float:
    try:
        return float(value)
    except (TypeError, ValueError):
        problems.add(f"{label} is not a number ({value!r})")
        return default


def _load_configs(raw, problems: _Problems) -> list[ConfigEntry]:
    configs: list[ConfigEntry] = []
    seen: set[str] = set()
    for idx, entry in enumerate(raw):
        if not isinstance(entry, dict) or "name" not in entry or not isinstance(entry.get("args"), dict):
            problems.add(f"configs entry #{idx} needs a name and an args mapping")
            continue
        name = str(entry["name"])
        if name in seen:
            problems.add(f"config name {name!r} appears twice")
        seen.add(name)
        vals = {k: _as_float(entry.get(k, d), problems, f"{name}.{k}", d) for k, d in _CONFIG_DEFAULTS.items()}
        if vals["target_ratio"] <= 0:
            problems.add(f"{name}.target_ratio has to be positive")
        if vals["weight"] < 0:
            problems.add(f"{name}.weight cannot be negative")
        configs.append(ConfigEntry(name, entry["args"], vals["target_ratio"], vals["weight"]))
    return configs


def load_task_spec(path: str | Path) -> TaskSpec:
    """Parse a task.yaml into a TaskSpec; a file that breaks the schema above
    raises one ValueError naming every problem found."""
    path = Path(path)
    if not path.is_file():
        raise ValueError(f"{path}: no such task file")
    try:
        data = yaml.safe_load(path.read_text())
    except yaml.YAMLError as exc:
        raise ValueError(f"{path}: unreadable YAML ({exc})") from exc
    problems = _Problems(str(path))
    if not isinstance(data, dict):
        problems.add(f"top level is a {type(data).__name__}, not a mapping")
        problems.raise_if_any()

    for key, kind in _TOP_LEVEL.items():
        if key not in data:
            problems.add(f"'{key}' is absent")
        elif kind is not str and not isinstance(data[key], kind):
            problems.add(f"'{key}' should be a {kind.__name__}")
    for key, subkeys in _NESTED.items():
        if isinstance(data.get(key), dict):
            for sub in subkeys:
                if sub not in data[key]:
                    problems.add(f"'{key}.{sub}' is absent")
    if isinstance(data.get("problem"), dict) and "shapes" in data["problem"] \
            and not isinstance(data["problem"]["shapes"], dict):
        problems.add("'problem.shapes' should be a mapping")
    problems.raise_if_any()

    if not data["configs"]:
        problems.add("'configs' is empty")
    configs = _load_configs(data["configs"], problems)
    names = [c.name for c in configs]

    scoring = str(data.get("scoring", SCORING_POLICIES[0]))
    focus = str(data.get("focus_config", ""))
    if scoring not in SCORING_POLICIES:
        problems.add(f"scoring {scoring!r} is not one of {', '.join(SCORING_POLICIES)}")
    elif scoring == "focus" and focus not in names:
        problems.add(f"focus_config {focus!r} has to name one of the configs {names}")
    elif scoring == "weighted_avg" and not any(c.weight > 0 for c in configs):
        problems.add("weighted_avg scoring needs a config with a positive weight")

    gate = data.get("stage_gate") or {}
    output = data.get("output") or {}
    if not isinstance(gate, dict):
        problems.add("'stage_gate' should be a mapping")
        gate = {}
    if not isinstance(output, dict):
        problems.add("'output' should be a mapping")
        output = {}
    gate_ratio = _as_float(gate.get("ratio", 0.9), problems, "stage_gate.ratio", 0.9)
    if gate_ratio <= 0:
        problems.add("stage_gate.ratio has to be positive")
    lists = {key: list(data.get(key) or []) for key in _OPTIONAL_LISTS}
    for key, vals in lists.items():
        if not all(isinstance(v, str) for v in vals):
            problems.add(f"'{key}' should list strings")
    problems.raise_if_any()

    problem = data["problem"]
    return TaskSpec(
        name=str(data["name"]), gpu=str(data["gpu"]), arch=str(data["arch"]), precision=str(data["precision"]),
        description=str(problem["description"]), shapes=dict(problem["shapes"]),
        baseline_source=str(data["baseline"]["source"]), configs=configs, scoring=scoring, focus_config=focus,
        stage_gate=StageGate(gate_ratio, bool(gate.get("strict", False))), constraints=lists["constraints"],
        hints=lists["hints"], references=lists["references"],
        result_keys=list(output.get("result_keys", names)))


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
