"""Shared builders for the grad-sync tests (plans over synthetic tensors)."""

import json
from pathlib import Path
from types import SimpleNamespace

from eth_amd.grad_sync.metadata import SerializableGradientDescriptor
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


def single_rank_descriptor(logical_id, shape, order, tensor_parallel=True, partition_dim=0, dtype="torch.float32"):
    return SerializableGradientDescriptor(
        logical_param_id=logical_id,
        shared_weight_id=None,
        shared_weight_root=False,
        logical_region_key=logical_id,
        semantic_order_key=order,
        global_rank=0,
        model_impl="gpt",
        op_manifest_hash="manifest",
        pipeline_id=0,
        stage_id=0,
        model_chunk_id=0,
        global_op_index=order[0],
        manifest_op_name="op",
        runtime_op_name="op",
        relative_parameter_name=logical_id,
        stage_global_op_begin=0,
        stage_global_op_end=1000,
        local_tp_degree=1,
        local_tp_rank=0,
        local_dp_degree=1,
        local_dp_rank=0,
        local_cp_degree=1,
        local_cp_rank=0,
        stage_ranks=(0,),
        local_tp_group_ranks=(0,),
        local_dp_group_ranks=(0,),
        full_shape=tuple(shape),
        local_shape=tuple(shape),
        tensor_parallel=tensor_parallel,
        tp_replica_semantics=None if tensor_parallel else "identical_duplicate",
        partition_dim=partition_dim if tensor_parallel else -1,
        partition_stride=1,
        parameter_dtype=dtype,
        gradient_dtype=dtype,
        requires_grad=True,
    )


class FakeRegistry:
    def __init__(self):
        self.calls = []

    def handle(self, process_group_id):
        self.calls.append(process_group_id)
        return "cached-pg"


def runtime_binding(logical_id, tensor):
    return SimpleNamespace(logical_param_id=logical_id, main_grad=tensor, device=tensor.device, parameter=None)


def gpt_layer_shapes(hidden, ffn, layers):
    """Per-layer parameter list of a GPT stage (TP=1) in op order, with the
    semantics of eth/runtime/megatron/grad_sync/gpt_adapter.py:31-91:
    (logical id, shape, op index, param order, tensor_parallel, partition_dim)."""
    out = []
    for l in range(layers):
        base = 1 + 10 * l
        pre = f"gpt.layers.{l}"
        out += [
            (f"{pre}.attention.input_layernorm.weight", (hidden,), base + 0, 0, False, -1),
            (f"{pre}.attention.input_layernorm.bias", (hidden,), base + 0, 1, False, -1),
            (f"{pre}.attention.query_key_value.weight", (3 * hidden, hidden), base + 1, 0, True, 0),
            (f"{pre}.attention.query_key_value.bias", (3 * hidden,), base + 1, 1, True, 0),
            (f"{pre}.attention.dense.weight", (hidden, hidden), base + 3, 0, True, 1),
            (f"{pre}.attention.dense.bias", (hidden,), base + 3, 1, False, -1),
            (f"{pre}.mlp.input_layernorm.weight", (hidden,), base + 5, 0, False, -1),
            (f"{pre}.mlp.input_layernorm.bias", (hidden,), base + 5, 1, False, -1),
            (f"{pre}.mlp.dense_h_to_4h.weight", (ffn, hidden), base + 6, 0, True, 0),
            (f"{pre}.mlp.dense_h_to_4h.bias", (ffn,), base + 6, 1, True, 0),
            (f"{pre}.mlp.dense_4h_to_h.weight", (hidden, ffn), base + 8, 0, True, 1),
            (f"{pre}.mlp.dense_4h_to_h.bias", (hidden,), base + 8, 1, False, -1),
        ]
    return out


def descriptors_for(shapes):
    return [
        single_rank_descriptor(lid, shape, (op, order, lid), tp, pdim)
        for lid, shape, op, order, tp, pdim in shapes
    ]


__all__ = [
    "CanonicalFragmentPlan",
    "LocalFragmentBindingSpec",
    "ProcessGroupSpec",
    "TensorSegmentSpec",
]
