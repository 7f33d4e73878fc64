"""CPU tests of the evidence wire formats: the runtime-evidence JSON of
eth/runtime/megatron/grad_sync/runtime_evidence.py:21-138 (fed with the
oracle's packed payloads) and the rank snapshots of grad_sync/evidence.py:
158-253 (written and read back with a weights-only loader)."""

import hashlib
import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from eth_amd.grad_sync import bucket_plan as bp
from eth_amd.grad_sync.evidence import build_rank_snapshot, load_rank_snapshot, save_rank_snapshot
from eth_amd.grad_sync.planner import CanonicalFragmentPlan, LocalFragmentBindingSpec, ProcessGroupSpec, TensorSegmentSpec
from eth_amd.grad_sync.runtime_evidence import GradientRuntimeEvidenceRecorder
from eth_amd.grad_sync.synthetic import single_rank_descriptor
from oracle import gradsync as og
from tests.helpers import known_answers, named_fragment

KA = known_answers()

REPORT_KEYS = {
    "version", "global_rank", "sync_mode", "global_topology_hash", "global_manifest_hash", "global_fragment_hash",
    "global_plan_hash", "exact_payload_bytes_by_rank", "padding_payload_bytes", "process_group_count",
    "process_group_creation_count", "scratch", "process_group_count_stable", "process_group_creation_count_stable",
    "scratch_stable", "iterations",
}
ITERATION_KEYS = {
    "iteration", "normalization_scale", "collective_count", "payload_bytes", "buckets", "packed_payload_sha256",
    "process_group_count", "process_group_creation_count", "scratch_signature",
}
BUCKET_KEYS = {"bucket_id", "semantic_hash", "process_group_id", "exact_numel", "exact_bytes", "packed_payload_sha256"}


def evidence_plan(rec, mode):
    groups = tuple(ProcessGroupSpec(g, tuple(r), "gradient_sync") for g, r in rec["groups"])
    frags = tuple(named_fragment(fid, lid, gid, n, order) for fid, lid, gid, n, order in rec["fragments"])
    seg = TensorSegmentSpec(0, 2, (2,), 0, 2, 2)
    bindings = tuple(LocalFragmentBindingSpec(0, f.fragment_id, f.logical_param_id, (seg,), 1.0) for f in frags)
    source = CanonicalFragmentPlan(groups, frags, ((0, bindings),), "fragment-hash")
    return bp.build_gradient_sync_plan(source, mode, rec["cap_bytes"], "gpt", "manifest", "topology")


class _Registry:
    group_count = 2
    creation_count = 2


def test_runtime_evidence_records_the_oracle_payloads(tmp_path):
    rec = KA["runtime_evidence_four_to_two"]
    reports = {}
    for mode in ("tensor", "block"):
        plan = evidence_plan(rec, mode)
        scratch = {"torch.float32": torch.zeros(8)}
        recorder = GradientRuntimeEvidenceRecorder(plan, 0, _Registry(), scratch, tmp_path / mode)
        descs = {lid: SimpleNamespace(partition_dim=0) for lid in rec["tensors"]}
        for _ in range(rec["iterations"]):
            grads = {lid: np.asarray(v, dtype=np.float32) for lid, v in rec["tensors"].items()}
            packed = og.execute(plan, 0, descs, grads)
            recorder.begin_execution(1.0)
            for bucket, payload in zip(plan.global_bucket_order, packed):
                recorder.observe_packed_bucket(bucket, torch.from_numpy(payload))
            recorder.finish_execution()
        reports[mode] = json.loads((tmp_path / mode / "rank-00000.json").read_text())
        report = reports[mode]
        assert set(report) == REPORT_KEYS
        it = report["iterations"][0]
        assert set(it) == ITERATION_KEYS and all(set(b) == BUCKET_KEYS for b in it["buckets"])
        assert it["collective_count"] == rec["expected_collectives"][mode]
        assert it["payload_bytes"] == rec["expected_payload_bytes"]
        for b, payload in zip(it["buckets"], packed):
            assert b["packed_payload_sha256"] == hashlib.sha256(payload.tobytes()).hexdigest()
        whole = b"".join(p.tobytes() for p in packed)
        assert it["packed_payload_sha256"] == hashlib.sha256(whole).hexdigest()
        assert report["scratch_stable"] and report["process_group_count_stable"]
        assert report["process_group_creation_count_stable"] and report["padding_payload_bytes"] == 0
        assert [i["iteration"] for i in report["iterations"]] == [1, 2]
    # the same bytes travel in both modes, in fewer collectives in block mode
    for a, b in zip(reports["tensor"]["iterations"], reports["block"]["iterations"]):
        assert a["packed_payload_sha256"] == b["packed_payload_sha256"]
        assert a["payload_bytes"] == b["payload_bytes"]


def test_runtime_evidence_flags_a_moved_scratch(tmp_path):
    rec = KA["runtime_evidence_four_to_two"]
    plan = evidence_plan(rec, "block")
    scratch = {"torch.float32": torch.zeros(8)}
    recorder = GradientRuntimeEvidenceRecorder(plan, 0, _Registry(), scratch, tmp_path)
    recorder.begin_execution(1.0)
    scratch["torch.float32"] = torch.zeros(8)  # a reallocation between steps
    recorder.finish_execution()
    assert not json.loads((tmp_path / "rank-00000.json").read_text())["scratch_stable"]
    with pytest.raises(RuntimeError):
        recorder.finish_execution()


def _snapshot_args(phase="post_step", grad_value=1.0):
    d = single_rank_descriptor("gpt.layers.0.mlp.dense_h_to_4h.bias", (4,), (7, 1, "x"))
    p = torch.nn.Parameter(torch.arange(4, dtype=torch.float32))
    binding = SimpleNamespace(logical_param_id=d.logical_param_id, parameter=p, main_grad=torch.full((4,), grad_value))
    state = {d.logical_param_id: {"step": torch.tensor(3.0), "exp_avg": torch.ones(4), "exp_avg_sq": torch.ones(4)}}
    return dict(
        phase=phase, iteration=3, global_rank=0, descriptors=[d], runtime_bindings=[binding],
        optimizer_state_by_logical=state,
        optimizer_hyperparameters_by_logical={d.logical_param_id: {"beta1": 0.9, "beta2": 0.95, "epsilon": 1e-8,
                                                                   "weight_decay": 0.0}},
        clock={"learning_rate": 1e-4}, metrics={"lm loss": torch.tensor(2.5)}, run_metadata={"precision": "bf16"},
    )


def test_rank_snapshot_round_trips_with_the_reference_layout(tmp_path):
    path = save_rank_snapshot(tmp_path, **_snapshot_args())
    assert path == tmp_path / "rank-00000" / "iteration-000003-post_step.pt"
    snap = load_rank_snapshot(path)  # torch.load(weights_only=True)
    assert set(snap) == {"version", "phase", "iteration", "global_rank", "records", "clock", "metrics", "run_metadata"}
    (r,) = snap["records"]
    assert set(r) == {"descriptor", "parameter", "main_grad", "optimizer_state", "optimizer_parameter",
                      "optimizer_hyperparameters"}
    assert r["descriptor"]["logical_param_id"] == "gpt.layers.0.mlp.dense_h_to_4h.bias"
    assert r["descriptor"]["semantic_order_key"] == (7, 1, "x")
    assert torch.equal(r["parameter"], torch.arange(4, dtype=torch.float32))
    assert torch.equal(r["optimizer_parameter"], r["parameter"])  # defaults to the model parameter
    assert r["optimizer_state"]["step"].item() == 3.0
    assert snap["metrics"]["lm loss"].item() == 2.5


def test_rank_snapshot_rejects_bad_phase_and_non_finite_values():
    with pytest.raises(ValueError, match="phase"):
        build_rank_snapshot(**_snapshot_args(phase="after"))
    # a non-finite main grad is legal after an overflow, but not at init
    build_rank_snapshot(**_snapshot_args(phase="pre_sync", grad_value=float("inf")))
    with pytest.raises(ValueError, match="non-finite"):
        build_rank_snapshot(**_snapshot_args(phase="init", grad_value=float("inf")))
