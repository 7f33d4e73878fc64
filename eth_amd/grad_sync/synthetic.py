"""Synthetic GPT gradient lists for the grad-sync / AdamW workloads
(BASELINE configs[2] and [3]): the per-layer parameters of a TP = 1 GPT in
op order with the semantics of the GPT adapter
(eth/runtime/megatron/grad_sync/gpt_adapter.py:31-91)."""

from .metadata import SerializableGradientDescriptor


def gpt_layer_shapes(hidden, ffn, layers):
    """(logical id, shape, op index, param order, tensor_parallel, partition_dim)."""
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
        stage_global_op_end=1 << 30,
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


def descriptors_for(shapes):
    return [single_rank_descriptor(lid, shape, (op, order, lid), tp, pdim) for lid, shape, op, order, tp, pdim in shapes]
