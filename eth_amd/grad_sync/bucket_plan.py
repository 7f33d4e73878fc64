"""Bucket placement and the process-group registry (host, init time).

Behaviour of eth/runtime/megatron/grad_sync/bucket_plan.py:77-280 with its
record types (:28-74).  How buckets are formed:

1. fragments are ordered by (process group index, dtype index, reduction
   semantics, semantic key) -- groups by their rank tuples, dtypes by name;
2. that order is cut into runs of equal (group, dtype, semantics): a bucket
   never mixes them, since each bucket is one collective on one group;
3. `tensor` mode makes every fragment its own bucket; `block` mode cuts each
   run greedily: a bucket takes fragments while its byte total stays within
   the cap, a fragment is never split, and one larger than the cap becomes
   a bucket of its own, flagged `oversized`;
4. a bucket's payload is its fragments back to back (destination offsets are
   prefix sums, no padding), and the scratch a rank needs per dtype is its
   largest bucket.

Bucket and plan identifiers are digests of canonical JSON (planner.plan_digest).
"""

import itertools
from dataclasses import asdict, dataclass

from .planner import plan_digest

_ELEMENT_BYTES = {"float16": 2, "bfloat16": 2, "float32": 4, "float64": 8}


def dtype_bytes(dtype):
    """Bytes per element of a gradient dtype name ("float32" or "torch.float32")."""
    size = _ELEMENT_BYTES.get(str(dtype).removeprefix("torch."))
    if size is None:
        raise ValueError(f"unsupported gradient dtype {dtype!r}")
    return size


@dataclass(frozen=True)
class BucketFragmentPlacement:
    fragment_id: str
    destination_offset: int


@dataclass(frozen=True)
class CommunicationBucketSpec:
    bucket_id: str
    process_group_id: str
    grad_dtype: str
    reduction_semantics: str
    placements: tuple
    exact_numel: int
    exact_bytes: int
    logical_region_begin: str
    logical_region_end: str
    semantic_hash: str
    oversized: bool


@dataclass(frozen=True)
class GradientSyncPlan:
    version: int
    sync_mode: str
    bucket_cap_bytes: int
    model_impl: str
    op_manifest_hash: str
    process_groups: tuple
    process_group_index_by_id: tuple
    canonical_fragments: tuple
    local_fragment_bindings_by_rank: tuple
    global_bucket_order: tuple
    max_scratch_numel_by_rank_and_dtype: tuple
    exact_payload_bytes_by_rank: tuple
    padding_payload_bytes: int
    global_topology_hash: str
    global_manifest_hash: str
    global_fragment_hash: str
    global_plan_hash: str


def _greedy_cuts(sizes, cap):
    """[lo, hi) index ranges of consecutive items whose sizes sum to at most
    `cap`, taken greedily; an item above the cap is a range of its own."""
    lo, total = 0, 0
    for i, size in enumerate(sizes):
        if i > lo and total + size > cap:
            yield lo, i
            lo, total = i, 0
        total += size
        if size > cap:
            yield lo, i + 1
            lo, total = i + 1, 0
    if lo < len(sizes):
        yield lo, len(sizes)


def _seal(fragments, cap_bytes, ranks):
    """The bucket holding `fragments` back to back."""
    head, tail = fragments[0], fragments[-1]
    starts = [0, *itertools.accumulate(f.numel for f in fragments)]
    placements = tuple(BucketFragmentPlacement(f.fragment_id, off) for f, off in zip(fragments, starts))
    numel = starts[-1]
    nbytes = numel * dtype_bytes(head.grad_dtype)
    digest = plan_digest(
        {
            "version": 1,
            "process_group_id": head.process_group_id,
            "process_group_ranks": ranks,
            "grad_dtype": head.grad_dtype,
            "reduction_semantics": head.reduction_semantics,
            "fragments": [asdict(f) for f in fragments],
            "placements": [asdict(p) for p in placements],
            "exact_numel": numel,
            "exact_bytes": nbytes,
        }
    )
    return CommunicationBucketSpec(
        bucket_id="bucket-" + digest[:20],
        process_group_id=head.process_group_id,
        grad_dtype=head.grad_dtype,
        reduction_semantics=head.reduction_semantics,
        placements=placements,
        exact_numel=numel,
        exact_bytes=nbytes,
        logical_region_begin=head.logical_region_key,
        logical_region_end=tail.logical_region_key,
        semantic_hash=digest,
        oversized=nbytes > cap_bytes,
    )


def bucketize(fragments, sync_mode, cap_bytes, groups):
    """Buckets of `fragments` (already in placement order); `groups` maps a
    process group id to its ProcessGroupSpec."""
    if sync_mode not in ("tensor", "block"):
        raise ValueError(f"unsupported sync mode {sync_mode!r}")
    if cap_bytes <= 0:
        raise ValueError("bucket_cap_bytes must be positive")
    buckets = []
    same_collective = lambda f: (f.process_group_id, f.grad_dtype, f.reduction_semantics)  # noqa: E731
    for (gid, _dtype, _sem), run in itertools.groupby(fragments, key=same_collective):
        run = tuple(run)
        if sync_mode == "tensor":
            cuts = [(i, i + 1) for i in range(len(run))]
        else:
            cuts = _greedy_cuts([f.numel * dtype_bytes(f.grad_dtype) for f in run], cap_bytes)
        buckets.extend(_seal(run[lo:hi], cap_bytes, groups[gid].ranks) for lo, hi in cuts)
    return tuple(buckets)


def build_gradient_sync_plan(fragment_plan, sync_mode, bucket_cap_bytes, model_impl, manifest_hash, topology_hash):
    groups = tuple(sorted(fragment_plan.process_groups, key=lambda g: g.ranks))
    group_rank = {g.process_group_id: i for i, g in enumerate(groups)}
    fragments = tuple(sorted(fragment_plan.fragments, key=lambda f: f.semantic_key))
    dtype_rank = {name: i for i, name in enumerate(sorted({f.grad_dtype for f in fragments}))}
    order = sorted(
        fragments,
        key=lambda f: (group_rank[f.process_group_id], dtype_rank[f.grad_dtype], f.reduction_semantics, f.semantic_key),
    )
    by_id = {g.process_group_id: g for g in groups}
    buckets = bucketize(tuple(order), sync_mode, bucket_cap_bytes, by_id)

    payload_bytes, scratch = {}, {}
    for b in buckets:
        for rank in by_id[b.process_group_id].ranks:
            payload_bytes[rank] = payload_bytes.get(rank, 0) + b.exact_bytes
            scratch[(rank, b.grad_dtype)] = max(scratch.get((rank, b.grad_dtype), 0), b.exact_numel)

    fragment_records = [asdict(f) for f in fragments]
    binding_records = [(rank, [asdict(b) for b in bs]) for rank, bs in fragment_plan.local_bindings_by_rank]
    fragment_hash = plan_digest(
        {"canonical_fragments": fragment_records, "local_fragment_bindings_by_rank": binding_records}
    )
    plan_hash = plan_digest(
        {
            "version": 1,
            "sync_mode": sync_mode,
            "bucket_cap_bytes": bucket_cap_bytes,
            "model_impl": model_impl,
            "manifest_hash": manifest_hash,
            "topology_hash": topology_hash,
            "fragment_hash": fragment_hash,
            "process_groups": [asdict(g) for g in groups],
            "canonical_fragments": fragment_records,
            "local_fragment_bindings_by_rank": binding_records,
            "buckets": [asdict(b) for b in buckets],
        }
    )
    return GradientSyncPlan(
        version=1,
        sync_mode=sync_mode,
        bucket_cap_bytes=bucket_cap_bytes,
        model_impl=model_impl,
        op_manifest_hash=manifest_hash,
        process_groups=groups,
        process_group_index_by_id=tuple(group_rank.items()),
        canonical_fragments=fragments,
        local_fragment_bindings_by_rank=fragment_plan.local_bindings_by_rank,
        global_bucket_order=buckets,
        max_scratch_numel_by_rank_and_dtype=tuple(sorted(scratch.items())),
        exact_payload_bytes_by_rank=tuple(sorted(payload_bytes.items())),
        padding_payload_bytes=0,
        global_topology_hash=topology_hash,
        global_manifest_hash=manifest_hash,
        global_fragment_hash=fragment_hash,
        global_plan_hash=plan_hash,
    )


class ProcessGroupRegistry:
    """Creates the plan's process groups once, in rank-tuple order, after
    checking the whole list (so a bad plan creates no group at all)."""

    def __init__(self, process_groups, create_group):
        self._specs = tuple(sorted(process_groups, key=lambda g: g.ranks))
        self._create_group = create_group
        self._handles = {}
        self._created = 0

    def _validate(self):
        ids = [g.process_group_id for g in self._specs]
        rank_sets = [g.ranks for g in self._specs]
        for g in self._specs:
            if ids.count(g.process_group_id) > 1:
                raise ValueError(f"duplicate process group id {g.process_group_id}")
            if rank_sets.count(g.ranks) > 1:
                raise ValueError(f"duplicate process group ranks {g.ranks}")
            if tuple(g.ranks) != tuple(sorted(set(g.ranks))):
                raise ValueError(f"process group ranks must be sorted and unique: {g.ranks}")

    def initialize(self):
        if self._handles:
            return
        self._validate()
        for g in self._specs:
            self._handles[g.process_group_id] = self._create_group(g.ranks)
            self._created += 1

    @property
    def group_count(self):
        return len(self._handles)

    @property
    def creation_count(self):
        return self._created

    def handle(self, process_group_id):
        try:
            return self._handles[process_group_id]
        except KeyError:
            raise KeyError(f"process group {process_group_id} is not initialized") from None
