"""Canonical gradient fragments: which part of which tensor every rank
contributes to which reduction (host, init time).

Behaviour of eth/runtime/megatron/grad_sync/planner.py:443-507
(plan_canonical_fragments) with the record types of :18-74; the algorithm
here is a closed form rather than an interval search.

Partition arithmetic.  Megatron splits a tensor-parallel parameter along its
partition axis into `degree * stride` equal blocks and gives TP rank r the
blocks r, r + degree, r + 2*degree, ... (stride > 1 is the interleaved QKV
layout).  Ranks of one parameter may run different TP degrees (one
pipeline at TP 2, another at TP 4); the canonical degree D is the largest of
them and every degree must divide it.  On the fine grid of D * stride blocks
of width w, canonical shard c is the blocks {c + k*D}.  For a rank of degree
d, fine block c + k*D lies inside its coarse block floor(c*d/D) + k*d, so

* shard c is held whole by TP rank t = floor(c*d/D), and
* its k-th block sits at offset k*W + w*(c - t*D/d) of that rank's local
  partition axis, where W = w*D/d is the rank's own block width.

Every rank's segments therefore follow from (c, d, k) directly; a rank's
segments tile its local axis exactly once by construction (checked anyway).
A replicated parameter is one fragment whose every holder contributes 1/d
of its copy (reduction `sum_identical_duplicates`).

Identifiers are the first hex digits of SHA-256 over a canonical JSON of the
fragment's defining fields (sorted keys, no whitespace), so plans built by
different processes -- or by the reference's planner -- compare equal.
"""

import hashlib
import json
import math
from dataclasses import asdict, dataclass, replace


def plan_digest(value):
    """SHA-256 hex of `value` as canonical JSON (sorted keys, compact)."""
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=True)
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


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
        return dict(self.local_bindings_by_rank).get(global_rank, ())


def _numel(shape):
    return math.prod(shape) if shape else 1


def group_id_for(ranks):
    return "pg-" + plan_digest({"ranks": ranks})[:16]


def canonical_regions(axis_size, degree, shard, stride, logical_id="parameter"):
    """Global [begin, end) intervals of the partition axis that make up
    canonical shard `shard` of `degree` with partition `stride`."""
    blocks = degree * stride
    if axis_size % blocks:
        raise ValueError(
            f"nondivisible TP layout for {logical_id}: axis of {axis_size} does not split into "
            f"TP {degree} x stride {stride} blocks"
        )
    width = axis_size // blocks
    return tuple(((shard + k * degree) * width, (shard + k * degree + 1) * width) for k in range(stride))


# fields every holder of one logical parameter must agree on -> error phrase
_AGREED = {
    "gradient_dtype": "dtype mismatch",
    "parameter_dtype": "dtype mismatch",
    "tensor_parallel": "replica semantics mismatch",
    "partition_stride": "stride mismatch",
    "model_impl": "model implementation mismatch",
    "op_manifest_hash": "manifest mismatch",
    "logical_region_key": "logical region mismatch",
    "semantic_order_key": "semantic order mismatch",
    "shared_weight_id": "shared weight mismatch",
    "shared_weight_root": "shared root mismatch",
}


class _Holders:
    """All descriptors of one logical parameter, checked and arranged as one
    (DP rank x TP rank) grid per pipeline."""

    def __init__(self, logical_id, descriptors):
        self.lid = logical_id
        self.items = sorted(descriptors, key=lambda d: (d.pipeline_id, d.local_dp_rank, d.local_tp_rank, d.global_rank))
        self.head = self.items[0]
        self._check_agreement()
        self.grids = self._arrange()

    @property
    def tensor_parallel(self):
        return self.head.tensor_parallel

    @property
    def axis(self):
        return self._axis_of(self.head)

    def _axis_of(self, d):
        ndim = len(d.full_shape)
        axis = d.partition_dim + ndim if d.partition_dim < 0 else d.partition_dim
        if axis not in range(ndim):
            raise ValueError(f"axis mismatch for {d.logical_param_id}: partition_dim {d.partition_dim} of {ndim}-d")
        return axis

    def _check_agreement(self):
        ranks = [d.global_rank for d in self.items]
        if len(set(ranks)) != len(ranks):
            dup = sorted(r for r in set(ranks) if ranks.count(r) > 1)
            raise ValueError(f"duplicate owner rank {dup[0]} for {self.lid}")
        if len({d.full_shape for d in self.items}) > 1:
            layouts = ", ".join(
                f"rank={d.global_rank} full={d.full_shape} local={d.local_shape} tp={d.local_tp_rank}/{d.local_tp_degree}"
                for d in self.items
            )
            raise ValueError(f"shape mismatch for {self.lid}: {layouts}")
        for field, phrase in _AGREED.items():
            if len({getattr(d, field) for d in self.items}) > 1:
                raise ValueError(f"{phrase} for {self.lid} ({field} differs between holders)")
        if self.head.tensor_parallel and len({self._axis_of(d) for d in self.items}) > 1:
            raise ValueError(f"axis mismatch for {self.lid}: holders split different axes")
        for d in self.items:
            where = f"{self.lid} rank {d.global_rank}"
            if (d.local_cp_degree, d.local_cp_rank) != (1, 0):
                raise ValueError(f"CP coordinate mismatch for {where}: context parallelism is not planned")
            for label, group, degree, coord in (
                ("TP", d.local_tp_group_ranks, d.local_tp_degree, d.local_tp_rank),
                ("DP", d.local_dp_group_ranks, d.local_dp_degree, d.local_dp_rank),
            ):
                if list(group) != sorted(group) or len(group) != degree:
                    raise ValueError(f"{label} group mismatch for {where}: {group} for degree {degree}")
                if d.global_rank not in group or group.index(d.global_rank) != coord:
                    raise ValueError(f"{label} coordinate mismatch for {where}: coordinate {coord} in {group}")
            if list(d.stage_ranks) != sorted(d.stage_ranks) or d.global_rank not in d.stage_ranks:
                raise ValueError(f"stage ranks mismatch for {where}")

    def _arrange(self):
        """{pipeline: {(dp_rank, tp_rank): descriptor}} with every grid
        complete and its TP rows / DP columns matching the declared groups."""
        grids = {}
        for d in self.items:
            grids.setdefault(d.pipeline_id, {})[(d.local_dp_rank, d.local_tp_rank)] = d
        for pipeline, grid in grids.items():
            cells = list(grid.values())
            dp = cells[0].local_dp_degree
            if any(c.local_dp_degree != dp for c in cells):
                raise ValueError(f"DP degree mismatch for {self.lid} pipeline {pipeline}")
            if {r for r, _ in grid} != set(range(dp)):
                raise ValueError(f"missing owner DP replica for {self.lid} pipeline {pipeline}")
            for r in range(dp):
                row = [c for (dr, _), c in sorted(grid.items()) if dr == r]
                tp = row[0].local_tp_degree
                if len(row) != tp or {c.local_tp_rank for c in row} != set(range(tp)):
                    raise ValueError(f"missing owner TP rank for {self.lid} pipeline {pipeline} DP {r}")
                if any(c.local_tp_degree != tp for c in row):
                    raise ValueError(f"TP degree mismatch for {self.lid}")
                ranks = tuple(sorted(c.global_rank for c in row))
                if any(tuple(c.local_tp_group_ranks) != ranks for c in row):
                    raise ValueError(f"TP group mismatch for {self.lid}")
            tp = cells[0].local_tp_degree
            if any(c.local_tp_degree != tp for c in cells):
                raise ValueError(f"TP degree mismatch for {self.lid} pipeline {pipeline}")
            for t in range(tp):
                column = tuple(grid[(r, t)].global_rank for r in range(dp))
                if any(tuple(grid[(r, t)].local_dp_group_ranks) != column for r in range(dp)):
                    raise ValueError(f"DP group mismatch for {self.lid} pipeline {pipeline}")
        return grids

    def replicas(self):
        """(pipeline, dp_rank, {tp_rank: descriptor}) in canonical order."""
        for pipeline in sorted(self.grids):
            grid = self.grids[pipeline]
            for r in sorted({dr for dr, _ in grid}):
                yield pipeline, r, {t: d for (dr, t), d in grid.items() if dr == r}


def _fragment(holders, shard, regions, group_id, numel, reduction):
    head = holders.head
    semantic_key = (head.semantic_order_key, shard, regions)
    fid = "fragment-" + plan_digest(
        {
            "logical_param_id": holders.lid,
            "canonical_shard_id": shard,
            "process_group_id": group_id,
            "grad_dtype": head.gradient_dtype,
            "global_regions": regions,
            "semantic_key": semantic_key,
        }
    )[:20]
    counted = head.shared_weight_id is None or head.shared_weight_root
    return CanonicalGradientFragmentSpec(
        fragment_id=fid,
        logical_param_id=holders.lid,
        canonical_shard_id=shard,
        process_group_id=group_id,
        grad_dtype=head.gradient_dtype,
        reduction_semantics=reduction,
        logical_region_key=head.logical_region_key,
        global_regions=regions,
        numel=numel,
        semantic_key=semantic_key,
        optimizer_semantic_id=head.shared_weight_id or holders.lid,
        include_in_optimizer_norm=counted,
        norm_owner_rank=None,  # filled once the group is known
    )


def _with_owner(fragment, ranks):
    """The lowest rank of the reduction group owns a counted fragment's norm."""
    return replace(fragment, norm_owner_rank=min(ranks) if fragment.include_in_optimizer_norm else None)


def _plan_sharded(holders):
    head, lid, axis = holders.head, holders.lid, holders.axis
    size, stride = head.full_shape[axis], head.partition_stride
    degree = max(d.local_tp_degree for d in holders.items)
    canonical_regions(size, degree, 0, stride, lid)  # divisibility of the fine grid
    for d in holders.items:
        if degree % d.local_tp_degree:
            raise ValueError(
                f"nondivisible canonical TP degree for {lid}: {degree} is not a multiple of {d.local_tp_degree}"
            )
        expected = tuple(n // d.local_tp_degree if i == axis else n for i, n in enumerate(head.full_shape))
        if tuple(d.local_shape) != expected:
            raise ValueError(f"shape mismatch for {lid} rank {d.global_rank}: local {d.local_shape}, expected {expected}")
    width = size // (degree * stride)
    inner = _numel(head.full_shape) // size
    groups, fragments, bindings = [], [], []
    for shard in range(degree):
        regions = canonical_regions(size, degree, shard, stride, lid)
        owners = []
        for _pipeline, _dp, row in holders.replicas():
            d_local = len(row)
            t = shard * d_local // degree
            owner = row[t]
            block = width * degree // d_local  # the owner's block width W
            base = width * (shard - t * (degree // d_local))
            segments = tuple(
                TensorSegmentSpec(
                    source_dim_offset=k * block + base,
                    source_dim_length=width,
                    source_shape=owner.local_shape,
                    global_coordinate_begin=lo,
                    global_coordinate_end=hi,
                    flattened_numel=width * inner,
                )
                for k, (lo, hi) in enumerate(regions)
            )
            owners.append((owner, segments))
        ranks = tuple(sorted(o.global_rank for o, _ in owners))
        gid = group_id_for(ranks)
        groups.append(ProcessGroupSpec(gid, ranks, "gradient_sync"))
        frag = _with_owner(_fragment(holders, shard, regions, gid, width * stride * inner, "sum"), ranks)
        fragments.append(frag)
        bindings.extend(LocalFragmentBindingSpec(o.global_rank, frag.fragment_id, lid, segs, 1.0) for o, segs in owners)
    _check_tiling(holders, bindings, axis)
    return groups, fragments, bindings


def _check_tiling(holders, bindings, axis):
    """Each holder's segments cover its local partition axis once, in order."""
    spans = {}
    for b in bindings:
        spans.setdefault(b.global_rank, []).extend(
            (s.source_dim_offset, s.source_dim_offset + s.source_dim_length) for s in b.source_segments
        )
    for d in holders.items:
        edges = sorted(spans.get(d.global_rank, []))
        flat = [x for span in edges for x in span]
        if not edges or flat[0] != 0 or flat[-1] != d.local_shape[axis] or any(
            flat[i] != flat[i + 1] for i in range(1, len(flat) - 1, 2)
        ):
            raise ValueError(f"local coverage overlap or gap for {holders.lid} rank {d.global_rank}")


def _plan_replicated(holders):
    head, lid = holders.head, holders.lid
    for d in holders.items:
        if d.tp_replica_semantics != "identical_duplicate":
            raise ValueError(f"replica semantics invalid for {lid}: {d.tp_replica_semantics!r}")
        if tuple(d.local_shape) != tuple(d.full_shape):
            raise ValueError(f"shape mismatch for replicated {lid} rank {d.global_rank}")
    ranks = tuple(sorted(d.global_rank for d in holders.items))
    gid = group_id_for(ranks)
    extent = head.full_shape[0] if head.full_shape else 1
    regions = ((0, extent),)
    frag = _with_owner(_fragment(holders, None, regions, gid, _numel(head.full_shape), "sum_identical_duplicates"), ranks)
    whole = TensorSegmentSpec(0, extent, head.local_shape, 0, extent, _numel(head.local_shape))
    bindings = [
        LocalFragmentBindingSpec(d.global_rank, frag.fragment_id, lid, (whole,), 1.0 / d.local_tp_degree)
        for d in sorted(holders.items, key=lambda x: x.global_rank)
    ]
    return [ProcessGroupSpec(gid, ranks, "gradient_sync")], [frag], bindings


def _check_shared_weights(by_id):
    shared = {}
    for lid, items in by_id.items():
        if items[0].shared_weight_id is not None:
            shared.setdefault(items[0].shared_weight_id, []).append(items[0])
    for sid, heads in shared.items():
        roots = sorted(h.logical_param_id for h in heads if h.shared_weight_root)
        if len(roots) != 1:
            raise ValueError(f"shared root mismatch for {sid}: expected one root, got {roots}")
        first = heads[0]
        for h in heads[1:]:
            for field in ("full_shape", "parameter_dtype", "gradient_dtype", "tensor_parallel", "partition_dim",
                          "partition_stride"):
                if getattr(h, field) != getattr(first, field):
                    raise ValueError(f"shared copy mismatch for {sid} at {h.logical_param_id} ({field})")


def plan_canonical_fragments(descriptors, expected_pipeline_ids):
    """CanonicalFragmentPlan of every rank's descriptors (the same on every
    rank, independent of the order the descriptors arrive in)."""
    descriptors = tuple(descriptors)
    for field, phrase in (("model_impl", "model implementation"), ("op_manifest_hash", "manifest")):
        if len({getattr(d, field) for d in descriptors}) > 1:
            raise ValueError(f"{phrase} mismatch across descriptors")
    expected = set(expected_pipeline_ids)
    if not expected:
        raise ValueError("expected_pipeline_ids must not be empty")
    by_id = {}
    for d in descriptors:
        if not d.requires_grad:
            raise ValueError(f"non-trainable descriptor {d.logical_param_id}")
        by_id.setdefault(d.logical_param_id, []).append(d)
    _check_shared_weights(by_id)
    groups, fragments, bindings = {}, [], []
    for lid in sorted(by_id):
        present = {d.pipeline_id for d in by_id[lid]}
        if present != expected:
            raise ValueError(f"missing owner pipeline {sorted(expected - present)} for {lid}")
        holders = _Holders(lid, by_id[lid])
        planned = _plan_sharded(holders) if holders.tensor_parallel else _plan_replicated(holders)
        for group in planned[0]:
            known = groups.setdefault(group.process_group_id, group)
            if known.ranks != group.ranks:
                raise ValueError(f"process group hash collision for {group.ranks}")
        fragments.extend(planned[1])
        bindings.extend(planned[2])
    fragments.sort(key=lambda f: f.semantic_key)
    position = {f.fragment_id: i for i, f in enumerate(fragments)}
    per_rank = {}
    for b in sorted(bindings, key=lambda b: position[b.fragment_id]):
        per_rank.setdefault(b.global_rank, []).append(b)
    return CanonicalFragmentPlan(
        process_groups=tuple(sorted(groups.values(), key=lambda g: g.ranks)),
        fragments=tuple(fragments),
        local_bindings_by_rank=tuple((rank, tuple(bs)) for rank, bs in sorted(per_rank.items())),
        fragment_hash=plan_digest([asdict(f) for f in fragments]),
    )
