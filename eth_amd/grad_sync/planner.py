"""Canonical gradient fragment planning (host, init time).

Restates eth/runtime/megatron/grad_sync/planner.py:

* a tensor-parallel parameter is cut into `canonical_tp_degree` canonical
  shards along its partition axis; with partition stride S each shard owns S
  equal intervals (`_rank_intervals`, planner.py:89-101);
* every owner rank binds the parts of its local tensor that overlap a shard
  as TensorSegmentSpec records (`_source_segments`, planner.py:104-133);
* a replicated parameter is one fragment reduced with
  `sum_identical_duplicates` and each TP copy contributes 1/tp
  (`_plan_replicated`, planner.py:360-416);
* fragments are ordered by semantic_key, bindings by fragment order
  (`plan_canonical_fragments`, planner.py:443-507).

Identifiers are SHA-256 of the canonical JSON of the same fields the
reference hashes, so plans built on either side agree.
"""

import hashlib
import json
import math
from dataclasses import asdict, dataclass


def canonical_hash(value):
    payload = json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=True)
    return hashlib.sha256(payload.encode("utf-8")).hexdigest()


@dataclass(frozen=True)
class TensorSegmentSpec:
    source_dim_offset: int
    source_dim_length: int
    source_shape: tuple
    global_coordinate_begin: int
    global_coordinate_end: int
    flattened_numel: int


@dataclass(frozen=True)
class ProcessGroupSpec:
    process_group_id: str
    ranks: tuple
    semantic_kind: str


@dataclass(frozen=True)
class CanonicalGradientFragmentSpec:
    fragment_id: str
    logical_param_id: str
    canonical_shard_id: object
    process_group_id: str
    grad_dtype: str
    reduction_semantics: str
    logical_region_key: str
    global_regions: tuple
    numel: int
    semantic_key: tuple
    optimizer_semantic_id: str
    include_in_optimizer_norm: bool
    norm_owner_rank: object


@dataclass(frozen=True)
class LocalFragmentBindingSpec:
    global_rank: int
    fragment_id: str
    logical_param_id: str
    source_segments: tuple
    contribution_scale: float


@dataclass(frozen=True)
class CanonicalFragmentPlan:
    process_groups: tuple
    fragments: tuple
    local_bindings_by_rank: tuple
    fragment_hash: str

    def bindings_for_rank(self, global_rank):
        for rank, bindings in self.local_bindings_by_rank:
            if rank == global_rank:
                return bindings
        return ()


def numel_of(shape):
    return math.prod(shape) if shape else 1


def group_id_for(ranks):
    return "pg-" + canonical_hash({"ranks": ranks})[:16]


def _axis(descriptor):
    axis = descriptor.partition_dim
    rank = len(descriptor.full_shape)
    if axis < 0:
        axis += rank
    if not 0 <= axis < rank:
        raise ValueError(f"axis mismatch for {descriptor.logical_param_id}: {descriptor.partition_dim}")
    return axis


def shard_intervals(axis_size, tp_degree, tp_rank, stride, logical_id):
    """Intervals of the partition axis owned by `tp_rank` (planner.py:89-101)."""
    parts = tp_degree * stride
    if axis_size % parts:
        raise ValueError(
            f"nondivisible TP layout for {logical_id}: axis {axis_size}, TP {tp_degree}, stride {stride}"
        )
    width = axis_size // parts
    return tuple(
        ((s * tp_degree + tp_rank) * width, (s * tp_degree + tp_rank + 1) * width) for s in range(stride)
    )


def local_segments(descriptor, regions, axis):
    """Pieces of a rank's local tensor covering `regions` exactly, or ()."""
    owned = shard_intervals(
        descriptor.full_shape[axis],
        descriptor.local_tp_degree,
        descriptor.local_tp_rank,
        descriptor.partition_stride,
        descriptor.logical_param_id,
    )
    inner = numel_of(descriptor.full_shape) // descriptor.full_shape[axis]
    pieces = []
    local_base = 0
    for own_lo, own_hi in owned:
        for want_lo, want_hi in regions:
            lo, hi = max(own_lo, want_lo), min(own_hi, want_hi)
            if lo < hi:
                pieces.append(
                    TensorSegmentSpec(
                        source_dim_offset=local_base + lo - own_lo,
                        source_dim_length=hi - lo,
                        source_shape=descriptor.local_shape,
                        global_coordinate_begin=lo,
                        global_coordinate_end=hi,
                        flattened_numel=(hi - lo) * inner,
                    )
                )
        local_base += own_hi - own_lo
    covered = tuple((p.global_coordinate_begin, p.global_coordinate_end) for p in pieces)
    return tuple(pieces) if covered == tuple(regions) else ()


def _check_consistent(logical_id, descriptors):
    first = descriptors[0]
    ranks = set()
    for item in descriptors:
        if item.global_rank in ranks:
            raise ValueError(f"duplicate owner rank {item.global_rank} for {logical_id}")
        ranks.add(item.global_rank)
        for field, message in (
            ("full_shape", "shape mismatch"),
            ("gradient_dtype", "dtype mismatch"),
            ("parameter_dtype", "dtype mismatch"),
            ("tensor_parallel", "replica semantics mismatch"),
            ("partition_stride", "stride mismatch"),
            ("model_impl", "model implementation mismatch"),
            ("op_manifest_hash", "manifest mismatch"),
            ("logical_region_key", "logical region mismatch"),
            ("semantic_order_key", "semantic order mismatch"),
            ("shared_weight_id", "shared weight mismatch"),
            ("shared_weight_root", "shared root mismatch"),
        ):
            if getattr(item, field) != getattr(first, field):
                raise ValueError(f"{message} for {logical_id}")
        if item.tensor_parallel and _axis(item) != _axis(first):
            raise ValueError(f"axis mismatch for {logical_id}")
        if item.local_cp_degree != 1 or item.local_cp_rank != 0:
            raise ValueError(f"CP coordinate mismatch for {logical_id} rank {item.global_rank}")
        for label, group, degree, coord in (
            ("TP", item.local_tp_group_ranks, item.local_tp_degree, item.local_tp_rank),
            ("DP", item.local_dp_group_ranks, item.local_dp_degree, item.local_dp_rank),
        ):
            if tuple(sorted(group)) != tuple(group) or len(group) != degree:
                raise ValueError(f"{label} group mismatch for {logical_id} rank {item.global_rank}")
            if item.global_rank not in group or group.index(item.global_rank) != coord:
                raise ValueError(f"{label} coordinate mismatch for {logical_id} rank {item.global_rank}")
    replicas = {}
    for item in descriptors:
        replicas.setdefault(item.pipeline_id, {}).setdefault(item.local_dp_rank, []).append(item)
    for pipeline_id, by_dp in replicas.items():
        dp = next(iter(by_dp.values()))[0].local_dp_degree
        if set(by_dp) != set(range(dp)):
            raise ValueError(f"missing owner DP replica for {logical_id} pipeline {pipeline_id}")
        for dp_rank, holders in by_dp.items():
            tp = holders[0].local_tp_degree
            if len(holders) != tp or {h.local_tp_rank for h in holders} != set(range(tp)):
                raise ValueError(f"missing owner TP rank for {logical_id} pipeline {pipeline_id} DP {dp_rank}")
    return replicas


def _fragment_id(fields):
    return "fragment-" + canonical_hash(fields)[:20]


def _norm_facts(reference, ranks):
    include = reference.shared_weight_id is None or reference.shared_weight_root
    return include, (min(ranks) if include else None)


def _plan_sharded(logical_id, descriptors, replicas):
    first = descriptors[0]
    axis = _axis(first)
    degree = max(d.local_tp_degree for d in descriptors)
    shard_intervals(first.full_shape[axis], degree, 0, first.partition_stride, logical_id)
    for d in descriptors:
        if degree % d.local_tp_degree:
            raise ValueError(f"nondivisible canonical TP degree for {logical_id}: {degree} % {d.local_tp_degree}")
        expect = list(first.full_shape)
        expect[axis] //= d.local_tp_degree
        if tuple(d.local_shape) != tuple(expect):
            raise ValueError(f"shape mismatch for {logical_id} rank {d.global_rank}")
    inner = numel_of(first.full_shape) // first.full_shape[axis]
    groups, fragments, bindings = [], [], []
    for shard in range(degree):
        regions = shard_intervals(first.full_shape[axis], degree, shard, first.partition_stride, logical_id)
        owners = []
        for pipeline_id in sorted(replicas):
            for dp_rank in sorted(replicas[pipeline_id]):
                hits = [
                    (d, segs)
                    for d in replicas[pipeline_id][dp_rank]
                    for segs in (local_segments(d, regions, axis),)
                    if segs
                ]
                if len(hits) != 1:
                    raise ValueError(f"missing owner for {logical_id} shard {shard} pipeline {pipeline_id} DP {dp_rank}")
                owners.append(hits[0])
        ranks = tuple(sorted(d.global_rank for d, _ in owners))
        pg = group_id_for(ranks)
        groups.append(ProcessGroupSpec(pg, ranks, "gradient_sync"))
        include, owner = _norm_facts(first, ranks)
        semantic_key = (first.semantic_order_key, shard, regions)
        fid = _fragment_id(
            {
                "logical_param_id": logical_id,
                "canonical_shard_id": shard,
                "process_group_id": pg,
                "grad_dtype": first.gradient_dtype,
                "global_regions": regions,
                "semantic_key": semantic_key,
            }
        )
        fragments.append(
            CanonicalGradientFragmentSpec(
                fragment_id=fid,
                logical_param_id=logical_id,
                canonical_shard_id=shard,
                process_group_id=pg,
                grad_dtype=first.gradient_dtype,
                reduction_semantics="sum",
                logical_region_key=first.logical_region_key,
                global_regions=regions,
                numel=sum(hi - lo for lo, hi in regions) * inner,
                semantic_key=semantic_key,
                optimizer_semantic_id=first.shared_weight_id or logical_id,
                include_in_optimizer_norm=include,
                norm_owner_rank=owner,
            )
        )
        for d, segs in owners:
            bindings.append(LocalFragmentBindingSpec(d.global_rank, fid, logical_id, segs, 1.0))
    for d in descriptors:
        mine = sorted(
            (s.source_dim_offset, s.source_dim_offset + s.source_dim_length)
            for b in bindings
            if b.global_rank == d.global_rank
            for s in b.source_segments
        )
        cursor = 0
        for lo, hi in mine:
            if lo != cursor or hi <= lo:
                raise ValueError(f"local coverage overlap or gap for {logical_id} rank {d.global_rank}")
            cursor = hi
        if cursor != d.local_shape[axis]:
            raise ValueError(f"local coverage gap for {logical_id} rank {d.global_rank}")
    return groups, fragments, bindings


def _plan_replicated(logical_id, descriptors):
    first = descriptors[0]
    for d in descriptors:
        if d.tp_replica_semantics != "identical_duplicate":
            raise ValueError(f"replica semantics invalid for {logical_id}")
        if tuple(d.local_shape) != tuple(d.full_shape):
            raise ValueError(f"shape mismatch for replicated {logical_id}")
    ranks = tuple(sorted(d.global_rank for d in descriptors))
    pg = group_id_for(ranks)
    regions = ((0, first.full_shape[0] if first.full_shape else 1),)
    include, owner = _norm_facts(first, ranks)
    semantic_key = (first.semantic_order_key, None, regions)
    fid = _fragment_id(
        {
            "logical_param_id": logical_id,
            "canonical_shard_id": None,
            "process_group_id": pg,
            "grad_dtype": first.gradient_dtype,
            "global_regions": regions,
            "semantic_key": semantic_key,
        }
    )
    fragment = CanonicalGradientFragmentSpec(
        fragment_id=fid,
        logical_param_id=logical_id,
        canonical_shard_id=None,
        process_group_id=pg,
        grad_dtype=first.gradient_dtype,
        reduction_semantics="sum_identical_duplicates",
        logical_region_key=first.logical_region_key,
        global_regions=regions,
        numel=numel_of(first.full_shape),
        semantic_key=semantic_key,
        optimizer_semantic_id=first.shared_weight_id or logical_id,
        include_in_optimizer_norm=include,
        norm_owner_rank=owner,
    )
    bindings = tuple(
        LocalFragmentBindingSpec(
            d.global_rank,
            fid,
            logical_id,
            (
                TensorSegmentSpec(
                    0,
                    d.local_shape[0] if d.local_shape else 1,
                    d.local_shape,
                    0,
                    d.full_shape[0] if d.full_shape else 1,
                    numel_of(d.local_shape),
                ),
            ),
            1.0 / d.local_tp_degree,
        )
        for d in sorted(descriptors, key=lambda x: x.global_rank)
    )
    return (ProcessGroupSpec(pg, ranks, "gradient_sync"),), (fragment,), bindings


def plan_canonical_fragments(descriptors, expected_pipeline_ids):
    descriptors = tuple(descriptors)
    if len({d.model_impl for d in descriptors}) > 1:
        raise ValueError("model implementation mismatch across descriptors")
    if len({d.op_manifest_hash for d in descriptors}) > 1:
        raise ValueError("manifest mismatch across descriptors")
    by_id = {}
    for d in descriptors:
        if not d.requires_grad:
            raise ValueError(f"non-trainable descriptor {d.logical_param_id}")
        by_id.setdefault(d.logical_param_id, []).append(d)
    expected = set(expected_pipeline_ids)
    if not expected:
        raise ValueError("expected_pipeline_ids must not be empty")
    shared = {}
    for lid, ds in by_id.items():
        if ds[0].shared_weight_id is not None:
            shared.setdefault(ds[0].shared_weight_id, []).append((lid, ds[0]))
    for sid, members in shared.items():
        roots = [lid for lid, d in members if d.shared_weight_root]
        if len(roots) != 1:
            raise ValueError(f"shared root mismatch for {sid}: expected one root, got {roots}")
    groups, fragments, bindings = {}, [], []
    for lid in sorted(by_id):
        ds = sorted(by_id[lid], key=lambda d: (d.pipeline_id, d.local_dp_rank, d.local_tp_rank, d.global_rank))
        present = {d.pipeline_id for d in ds}
        if present != expected:
            raise ValueError(f"missing owner pipeline {sorted(expected - present)} for {lid}")
        replicas = _check_consistent(lid, ds)
        if ds[0].tensor_parallel:
            g, f, b = _plan_sharded(lid, ds, replicas)
        else:
            g, f, b = _plan_replicated(lid, ds)
        for item in g:
            old = groups.get(item.process_group_id)
            if old is not None and old.ranks != item.ranks:
                raise ValueError(f"process group hash collision for {item.ranks}")
            groups[item.process_group_id] = item
        fragments.extend(f)
        bindings.extend(b)
    fragments.sort(key=lambda f: f.semantic_key)
    order = {f.fragment_id: i for i, f in enumerate(fragments)}
    per_rank = {}
    for b in bindings:
        per_rank.setdefault(b.global_rank, []).append(b)
    frozen = tuple(
        (rank, tuple(sorted(bs, key=lambda b: order[b.fragment_id]))) for rank, bs in sorted(per_rank.items())
    )
    return CanonicalFragmentPlan(
        process_groups=tuple(sorted(groups.values(), key=lambda g: g.ranks)),
        fragments=tuple(fragments),
        local_bindings_by_rank=frozen,
        fragment_hash=canonical_hash([asdict(f) for f in fragments]),
    )
