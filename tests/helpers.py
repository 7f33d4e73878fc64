"""Shared builders for the grad-sync tests (plans over synthetic tensors)."""

import json
from pathlib import Path
from types import SimpleNamespace

from eth_amd.grad_sync.synthetic import descriptors_for, gpt_layer_shapes, single_rank_descriptor  # noqa: F401
from eth_amd.grad_sync.planner import (
    CanonicalFragmentPlan,
    CanonicalGradientFragmentSpec,
    LocalFragmentBindingSpec,
    ProcessGroupSpec,
    TensorSegmentSpec,
)

GOLDEN = Path(__file__).resolve().parent / "golden"


def known_answers():
    return json.loads((GOLDEN / "known_answers.json").read_text())


def fragment(index, group_id, dtype="float32", numel=8, logical=None, norm=True):
    logical = logical or f"param-{index}"
    return CanonicalGradientFragmentSpec(
        fragment_id=f"fragment-{index}",
        logical_param_id=logical,
        canonical_shard_id=0,
        process_group_id=group_id,
        grad_dtype=dtype,
        reduction_semantics="sum",
        logical_region_key=f"region-{index}",
        global_regions=((0, numel),),
        numel=numel,
        semantic_key=(index,),
        optimizer_semantic_id=logical,
        include_in_optimizer_norm=norm,
        norm_owner_rank=0,
    )


def named_fragment(fid, logical, group_id, numel, order, dtype="float32", reduction="sum"):
    return CanonicalGradientFragmentSpec(
        fragment_id=fid,
        logical_param_id=logical,
        canonical_shard_id=0,
        process_group_id=group_id,
        grad_dtype=dtype,
        reduction_semantics=reduction,
        logical_region_key=logical,
        global_regions=((0, numel),),
        numel=numel,
        semantic_key=(order,),
        optimizer_semantic_id=logical,
        include_in_optimizer_norm=True,
        norm_owner_rank=0,
    )


class FakeRegistry:
    def __init__(self):
        self.calls = []

    def handle(self, process_group_id):
        self.calls.append(process_group_id)
        return "cached-pg"


def runtime_binding(logical_id, tensor):
    return SimpleNamespace(logical_param_id=logical_id, main_grad=tensor, device=tensor.device, parameter=None)


__all__ = [
    "CanonicalFragmentPlan",
    "LocalFragmentBindingSpec",
    "ProcessGroupSpec",
    "TensorSegmentSpec",
]
