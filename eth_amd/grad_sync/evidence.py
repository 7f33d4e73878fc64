"""Per-rank numerical snapshots of a training step.

The record layout of eth/runtime/megatron/grad_sync/evidence.py:158-253
(build_rank_snapshot / save_rank_snapshot / load_rank_snapshot), so the
reference's tools/validation/compare_numerical_evidence.py reads this
build's files: a dict with `version` 1, `phase` (init / pre_sync /
post_sync / post_step), `iteration`, `global_rank`, one record per logical
parameter in logical-id order -- its descriptor as a dict, the model
parameter, its main grad, the optimizer state (`step`, `exp_avg`,
`exp_avg_sq`), the optimizer's fp32 parameter and hyperparameters -- plus
`clock`, `metrics` and `run_metadata`.  Tensors are CPU copies, so the file
loads with `torch.load(..., weights_only=True)`.  Non-finite values are
rejected (a main grad only at `init`: an overflowing step legitimately
holds them before the scaler backs off).
"""

from dataclasses import asdict, is_dataclass
from pathlib import Path

import torch

PHASES = ("init", "pre_sync", "post_sync", "post_step")


def _host(value):
    """Detached CPU copy of tensors inside dicts / lists / tuples."""
    if torch.is_tensor(value):
        return value.detach().to("cpu", copy=True)
    if isinstance(value, dict):
        return {k: _host(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return type(value)(_host(v) for v in value)
    return value


def _require_finite(value, where):
    if torch.is_tensor(value):
        if (value.is_floating_point() or value.is_complex()) and not bool(torch.isfinite(value).all()):
            raise ValueError(f"{where} contains non-finite values")
    elif isinstance(value, dict):
        for k, v in value.items():
            _require_finite(v, f"{where}.{k}")
    elif isinstance(value, (list, tuple)):
        for i, v in enumerate(value):
            _require_finite(v, f"{where}[{i}]")


def _index(items, kind):
    out = {}
    for item in items:
        if item.logical_param_id in out:
            raise ValueError(f"duplicate {kind} for logical_param_id {item.logical_param_id}")
        out[item.logical_param_id] = item
    return out


def build_rank_snapshot(*, phase, iteration, global_rank, descriptors, runtime_bindings,
                        optimizer_state_by_logical=None, optimizer_parameter_by_logical=None,
                        optimizer_hyperparameters_by_logical=None, clock=None, metrics=None, run_metadata=None):
    if phase not in PHASES:
        raise ValueError(f"unsupported evidence phase {phase!r}")
    descs = _index(descriptors, "descriptor")
    binds = _index(runtime_bindings, "runtime binding")
    if set(descs) != set(binds):
        raise ValueError(f"snapshot descriptor/binding IDs differ: {sorted(descs)} != {sorted(binds)}")
    states = optimizer_state_by_logical or {}
    masters = optimizer_parameter_by_logical or {}
    hypers = optimizer_hyperparameters_by_logical or {}
    records = []
    for lid in sorted(descs):
        d, b = descs[lid], binds[lid]
        rec = {
            "descriptor": asdict(d) if is_dataclass(d) else dict(vars(d)),
            "parameter": _host(b.parameter),
            "main_grad": _host(b.main_grad),
            "optimizer_state": _host(states.get(lid, {})),
            "optimizer_parameter": _host(masters.get(lid, b.parameter)),
            "optimizer_hyperparameters": _host(hypers.get(lid, {})),
        }
        checked = ["parameter", "optimizer_parameter", "optimizer_state", "optimizer_hyperparameters"]
        if phase == "init":
            checked.append("main_grad")
        for key in checked:
            _require_finite(rec[key], f"{lid}.{key}")
        records.append(rec)
    snapshot = {
        "version": 1,
        "phase": phase,
        "iteration": int(iteration),
        "global_rank": int(global_rank),
        "records": records,
        "clock": _host(clock or {}),
        "metrics": _host(metrics or {}),
        "run_metadata": dict(run_metadata or {}),
    }
    _require_finite(snapshot["clock"], "clock")
    _require_finite(snapshot["metrics"], "metrics")
    return snapshot


def snapshot_path(output_dir, global_rank, iteration, phase):
    return Path(output_dir) / f"rank-{int(global_rank):05d}" / f"iteration-{int(iteration):06d}-{phase}.pt"


def save_rank_snapshot(output_dir, **snapshot_args):
    snapshot = build_rank_snapshot(**snapshot_args)
    path = snapshot_path(output_dir, snapshot["global_rank"], snapshot["iteration"], snapshot["phase"])
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(snapshot, path)
    return path


def load_rank_snapshot(path):
    snapshot = torch.load(path, map_location="cpu", weights_only=True)
    if snapshot.get("version") != 1:
        raise ValueError(f"unsupported evidence version {snapshot.get('version')!r}")
    return snapshot
