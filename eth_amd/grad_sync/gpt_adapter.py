"""GPT runtime ops -> canonical gradient descriptors (host, init time).

The parameter schema is the one of
eth/runtime/megatron/grad_sync/gpt_adapter.py:31-91 (op name -> parameter
path, logical id, shared-weight id, root flag, required, TP semantics), and
`semantic_order_key = (op_index, parameter_order, logical_id)` as at
:168-300.  This build runs one rank (TP = DP = CP = 1, stage ranks (0,)),
which fixes every topology field of the descriptor.
"""

import functools

from .metadata import LocalGradientBinding, SerializableGradientDescriptor

# ops without trainable parameters (the flash path's attention pieces, the
# dropouts and the GELU)
PARAMETERLESS_OPS = frozenset(
    {
        "enc-attention-score",
        "enc-attention-softmax",
        "enc-attention-dropout",
        "enc-attention-context",
        "enc-flash-attention",
        "enc-post-attention-dropout",
        "enc-MLP-gelu",
        "enc-post-MLP-dropout",
    }
)

# gradient semantics of a linear's (weight, bias) by the op's `algo`:
# column-parallel splits both along dim 0; row-parallel splits the weight
# along dim 1 and replicates the bias
LINEAR_SEMANTICS = {"column": ("sharded_dim0", "sharded_dim0"), "row": ("sharded_dim1", "replicated")}

# op name -> logical component of its (weight, bias) pair
_NORM_COMPONENTS = {
    "enc-1st-layernorm": "gpt.layers.{layer}.attention.input_layernorm",
    "enc-2nd-layernorm": "gpt.layers.{layer}.mlp.input_layernorm",
    "final-layernorm": "gpt.final_layernorm",
}
_LINEAR_COMPONENTS = {
    "enc-attention-qkv": ("query_key_value", "gpt.layers.{layer}.attention.query_key_value"),
    "enc-attention-dense": ("dense", "gpt.layers.{layer}.attention.dense"),
    "enc-MLP-GEMM-1": ("dense", "gpt.layers.{layer}.mlp.dense_h_to_4h"),
    "enc-MLP-GEMM-2": ("dense", "gpt.layers.{layer}.mlp.dense_4h_to_h"),
}
# entries: (path on the op, logical id, shared-weight id, shared root,
#           required, gradient semantics)
_VOCAB_ENTRIES = {
    "encoder-embedding": (
        ("word_embeddings.weight", "gpt.word_embeddings.weight", "gpt.word_embeddings", True, True, "sharded_dim0"),
        ("position_embeddings.weight", "gpt.position_embeddings.weight", None, False, True, "replicated"),
        ("tokentype_embeddings.weight", "gpt.tokentype_embeddings.weight", None, False, False, "replicated"),
    ),
    "gpt-post-process": (
        ("word_embeddings.weight", "gpt.output_head.word_embeddings.weight", "gpt.word_embeddings", False, True,
         "sharded_dim0"),
    ),
}


def parameter_schema(op, layer_index):
    """The (path, logical id, shared id, root, required, semantics) entries of
    one manifest op, in parameter order."""
    name = op.name
    if name in _VOCAB_ENTRIES:
        return _VOCAB_ENTRIES[name]
    if name in _NORM_COMPONENTS:
        comp = _NORM_COMPONENTS[name].format(layer=layer_index)
        return tuple(
            (f"input_layernorm.{leaf}", f"{comp}.{leaf}", None, False, True, "replicated") for leaf in ("weight", "bias")
        )
    if name in _LINEAR_COMPONENTS:
        module, comp = _LINEAR_COMPONENTS[name]
        comp = comp.format(layer=layer_index)
        algo = "column" if name == "enc-attention-qkv" else getattr(op, "algo", None)
        if algo not in LINEAR_SEMANTICS:
            raise ValueError(f"runtime op {getattr(op, 'op_index', None)} has unsupported linear algo {algo!r}")
        return tuple(
            (f"{module}.{leaf}", f"{comp}.{leaf}", None, False, True, sem)
            for leaf, sem in zip(("weight", "bias"), LINEAR_SEMANTICS[algo])
        )
    if name in PARAMETERLESS_OPS:
        return ()
    raise ValueError(f"unsupported GPT manifest op {name!r}")


def _resolve(root, path):
    """root.a.b.c, or None when any link is missing."""
    return functools.reduce(lambda obj, attr: getattr(obj, attr, None) if obj is not None else None, path.split("."), root)


def collect_stage_metadata(ops, stage_op_begin, stage_op_end, model_impl="gpt", manifest_hash="manifest",
                           global_rank=0):
    """Descriptors and main_grad bindings of every trainable parameter of the
    stage's ops, held by `global_rank` alone (no tensor or data
    parallelism; pipeline stages of one process take ranks 0, 1, ...)."""
    descriptors, bindings = [], []
    for op in ops:
        layer = (op.op_index - 1) // 10 if op.name.startswith("enc-") else None
        seen = set()
        for order, (path, lid, shared_id, shared_root, required, semantics) in enumerate(parameter_schema(op, layer)):
            p = _resolve(op, path)
            if p is None:
                if required:
                    raise ValueError(f"logical_param_id {lid} rank {global_rank} is missing {path}")
                continue
            if id(p) in seen:
                raise ValueError(f"duplicate parameter for logical_param_id {lid} rank {global_rank}")
            seen.add(id(p))
            if not p.requires_grad:
                continue
            mg = getattr(p, "main_grad", None)
            if mg is None:
                raise ValueError(f"logical_param_id {lid} rank {global_rank} is missing main_grad")
            tp = bool(p.tensor_model_parallel)
            pdim = int(p.partition_dim)
            if tp and pdim < 0:
                pdim += p.dim()
            actual = f"sharded_dim{pdim}" if tp else "replicated"
            if actual != semantics:
                raise ValueError(f"logical_param_id {lid} rank {global_rank} expected {semantics}, got {actual}")
            shape = tuple(int(s) for s in p.shape)
            descriptors.append(
                SerializableGradientDescriptor(
                    logical_param_id=lid,
                    shared_weight_id=shared_id,
                    shared_weight_root=shared_root,
                    logical_region_key=lid,
                    semantic_order_key=(op.op_index, order, lid),
                    global_rank=global_rank,
                    model_impl=model_impl,
                    op_manifest_hash=manifest_hash,
                    pipeline_id=0,
                    stage_id=global_rank,
                    model_chunk_id=0,
                    global_op_index=op.op_index,
                    manifest_op_name=op.name,
                    runtime_op_name=op.name,
                    relative_parameter_name=path,
                    stage_global_op_begin=stage_op_begin,
                    stage_global_op_end=stage_op_end,
                    local_tp_degree=1,
                    local_tp_rank=0,
                    local_dp_degree=1,
                    local_dp_rank=0,
                    local_cp_degree=1,
                    local_cp_rank=0,
                    stage_ranks=(global_rank,),
                    local_tp_group_ranks=(global_rank,),
                    local_dp_group_ranks=(global_rank,),
                    full_shape=shape,
                    local_shape=shape,
                    tensor_parallel=tp,
                    tp_replica_semantics=None if tp else "identical_duplicate",
                    partition_dim=pdim if tp else -1,
                    partition_stride=int(p.partition_stride),
                    parameter_dtype=str(p.dtype),
                    gradient_dtype=str(mg.dtype),
                    requires_grad=True,
                )
            )
            bindings.append(LocalGradientBinding(logical_param_id=lid, parameter=p, main_grad=mg, device=p.device))
        unlisted = {id(p) for p in op.parameters() if p.requires_grad} - seen
        if unlisted:
            raise ValueError(f"unlisted trainable parameter on rank {global_rank} op {op.op_index} ({op.name})")
    return tuple(descriptors), tuple(bindings)
