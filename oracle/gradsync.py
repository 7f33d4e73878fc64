"""numpy restatement of the local half of Block-wise All-Reduce (test oracle).

Follows eth/runtime/megatron/grad_sync/executor.py:173-261 (segment views,
pack with contribution scale, all_reduce_sum seam, normalization mul_,
unpack), optimizer/optimizer.py:436-461 (unscale + found_inf) and
grad_sync/optimizer_semantics.py:563-604 (L2 / inf norm, clip, zero count).
"""

import math

import numpy as np


def segment_view(main_grad, descriptor, segment):
    """executor.py:173-197: the whole tensor when replicated, else a narrow."""
    tensor_parallel = getattr(descriptor, "tensor_parallel", descriptor.partition_dim >= 0)
    if not tensor_parallel:
        assert segment.flattened_numel == main_grad.size
        return main_grad
    axis = descriptor.partition_dim % main_grad.ndim
    index = [slice(None)] * main_grad.ndim
    index[axis] = slice(segment.source_dim_offset, segment.source_dim_offset + segment.source_dim_length)
    return main_grad[tuple(index)]


def pack_bucket(bucket, bindings_by_fragment, grads, descriptors):
    """executor.py:199-226 -> payload of one bucket (dtype of the grads)."""
    dtype = None
    parts = []
    for placement in bucket.placements:
        binding = bindings_by_fragment[placement.fragment_id]
        g = grads[binding.logical_param_id]
        dtype = g.dtype
        for seg in binding.source_segments:
            src = segment_view(g, descriptors[binding.logical_param_id], seg).reshape(-1).copy()
            if binding.contribution_scale != 1.0:
                src = (src.astype(np.float32) * np.float32(binding.contribution_scale)).astype(dtype)
            parts.append(src)
    payload = np.concatenate(parts) if parts else np.zeros(0, dtype=np.float32)
    assert payload.size == bucket.exact_numel
    return payload


def unpack_bucket(bucket, bindings_by_fragment, grads, descriptors, payload):
    """executor.py:228-245: copy payload slices back into the segment views."""
    for placement in bucket.placements:
        binding = bindings_by_fragment[placement.fragment_id]
        g = grads[binding.logical_param_id]
        off = placement.destination_offset
        for seg in binding.source_segments:
            view = segment_view(g, descriptors[binding.logical_param_id], seg)
            n = view.size
            view[...] = payload[off : off + n].reshape(view.shape)
            off += n


def execute(plan, rank, descriptors, grads, normalization_scale=1.0, all_reduce_sum=None):
    """executor.py:247-261 for one rank; `grads` (numpy, by logical id) are
    updated in place.  Returns the list of packed payloads (pre-collective)."""
    groups = {g.process_group_id: g for g in plan.process_groups}
    bindings = {b.fragment_id: b for r, bs in plan.local_fragment_bindings_by_rank if r == rank for b in bs}
    packed = []
    for bucket in plan.global_bucket_order:
        if rank not in groups[bucket.process_group_id].ranks:
            continue
        payload = pack_bucket(bucket, bindings, grads, descriptors)
        packed.append(payload.copy())
        if all_reduce_sum is not None:
            all_reduce_sum(payload, bucket.process_group_id)
        if normalization_scale != 1.0:
            payload = (payload.astype(np.float32) * np.float32(normalization_scale)).astype(payload.dtype)
        unpack_bucket(bucket, bindings, grads, descriptors, payload)
    return packed


def unscale_and_check(grads, inv_scale):
    """torch._amp_foreach_non_finite_check_and_unscale_: g *= inv_scale in
    place (fp32), found_inf = any non-finite input."""
    found = False
    inv = np.float32(inv_scale)
    for g in grads:
        found |= not np.all(np.isfinite(g))
        g *= inv
    return found


def l2_norm(grads):
    """Global L2 norm in fp64 (the fp32 accumulation of
    optimizer_semantics.py:584-587 is within 1e-6 relative of this)."""
    return math.sqrt(sum(float(np.dot(g.astype(np.float64).ravel(), g.astype(np.float64).ravel())) for g in grads))


def inf_norm(grads):
    return max((float(np.max(np.abs(g))) for g in grads if g.size), default=0.0)


def clip_coefficient(total_norm, max_norm):
    """optimizer_semantics.py:589-590."""
    return float(max_norm) / (total_norm + 1.0e-6)


def clip(grads, total_norm, max_norm):
    coef = clip_coefficient(total_norm, max_norm)
    if coef < 1.0:
        for g in grads:
            g *= np.float32(coef)
    return coef


def count_zeros(grads):
    return float(sum(g.size - np.count_nonzero(g) for g in grads))
