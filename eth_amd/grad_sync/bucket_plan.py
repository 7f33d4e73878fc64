"""Bucket placement and the process-group registry (host, init time).

Restates eth/runtime/megatron/grad_sync/bucket_plan.py:77-280:

* fragments are placed in (group index, dtype index, reduction semantics,
  semantic key) order (`build_gradient_sync_plan`, :155-241);
* `tensor` mode gives one fragment per bucket; `block` mode fills a bucket
  greedily while the group/dtype/semantics key is unchanged and the bytes stay
  within the cap; a fragment is never split and one larger than the cap gets
  a bucket of its own, flagged `oversized` (`_bucketize`, :115-152);
* destination offsets are running element counts, there is no padding, and
  the scratch per (rank, dtype) is the largest bucket (:196-206).
"""

from dataclasses import asdict, dataclass

from .planner import canonical_hash

DTYPE_BYTES = {
    "float16": 2,
    "bfloat16": 2,
    "float32": 4,
    "float64": 8,
    "torch.float16": 2,
    "torch.bfloat16": 2,
    "torch.float32": 4,
    "torch.float64": 8,
}


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


def dtype_bytes(dtype):
    if dtype not in DTYPE_BYTES:
        raise ValueError(f"unsupported gradient dtype {dtype!r}")
    return DTYPE_BYTES[dtype]


def _bucket(fragments, cap_bytes, groups):
    head = fragments[0]
    width = dtype_bytes(head.grad_dtype)
    placements, offset = [], 0
    for frag in fragments:
        placements.append(BucketFragmentPlacement(frag.fragment_id, offset))
        offset += frag.numel
    nbytes = offset * width
    digest = canonical_hash(
        {
            "version": 1,
            "process_group_id": head.process_group_id,
            "process_group_ranks": groups[head.process_group_id].ranks,
            "grad_dtype": head.grad_dtype,
            "reduction_semantics": head.reduction_semantics,
            "fragments": [asdict(f) for f in fragments],
            "placements": [asdict(p) for p in placements],
            "exact_numel": offset,
            "exact_bytes": nbytes,
        }
    )
    return CommunicationBucketSpec(
        bucket_id="bucket-" + digest[:20],
        process_group_id=head.process_group_id,
        grad_dtype=head.grad_dtype,
        reduction_semantics=head.reduction_semantics,
        placements=tuple(placements),
        exact_numel=offset,
        exact_bytes=nbytes,
        logical_region_begin=head.logical_region_key,
        logical_region_end=fragments[-1].logical_region_key,
        semantic_hash=digest,
        oversized=nbytes > cap_bytes,
    )


def bucketize(fragments, sync_mode, cap_bytes, groups):
    if sync_mode not in ("tensor", "block"):
        raise ValueError(f"unsupported sync mode {sync_mode!r}")
    if cap_bytes <= 0:
        raise ValueError("bucket_cap_bytes must be positive")
    if sync_mode == "tensor":
        return tuple(_bucket((f,), cap_bytes, groups) for f in fragments)
    out, run, run_bytes, run_key = [], [], 0, None
    for frag in fragments:
        size = frag.numel * dtype_bytes(frag.grad_dtype)
        key = (frag.process_group_id, frag.grad_dtype, frag.reduction_semantics)
        if run and (key != run_key or run_bytes + size > cap_bytes):
            out.append(_bucket(tuple(run), cap_bytes, groups))
            run, run_bytes = [], 0
        run.append(frag)
        run_bytes += size
        run_key = key
        if size > cap_bytes:
            # an oversized fragment closes its own bucket
            out.append(_bucket(tuple(run), cap_bytes, groups))
            run, run_bytes, run_key = [], 0, None
    if run:
        out.append(_bucket(tuple(run), cap_bytes, groups))
    return tuple(out)


def build_gradient_sync_plan(fragment_plan, sync_mode, bucket_cap_bytes, model_impl, manifest_hash, topology_hash):
    groups = tuple(sorted(fragment_plan.process_groups, key=lambda g: g.ranks))
    fragments = tuple(sorted(fragment_plan.fragments, key=lambda f: f.semantic_key))
    by_id = {g.process_group_id: g for g in groups}
    group_index = {g.process_group_id: i for i, g in enumerate(groups)}
    dtype_index = {d: i for i, d in enumerate(sorted({f.grad_dtype for f in fragments}))}
    placed = tuple(
        sorted(
            fragments,
            key=lambda f: (group_index[f.process_group_id], dtype_index[f.grad_dtype], f.reduction_semantics, f.semantic_key),
        )
    )
    buckets = bucketize(placed, sync_mode, bucket_cap_bytes, by_id)
    payload_bytes, scratch = {}, {}
    for b in buckets:
        for rank in by_id[b.process_group_id].ranks:
            payload_bytes[rank] = payload_bytes.get(rank, 0) + b.exact_bytes
            key = (rank, b.grad_dtype)
            scratch[key] = max(scratch.get(key, 0), b.exact_numel)
    bindings_payload = [
        (rank, [asdict(b) for b in bindings]) for rank, bindings in fragment_plan.local_bindings_by_rank
    ]
    fragment_hash = canonical_hash(
        {"canonical_fragments": [asdict(f) for f in fragments], "local_fragment_bindings_by_rank": bindings_payload}
    )
    plan_hash = canonical_hash(
        {
            "version": 1,
            "sync_mode": sync_mode,
            "bucket_cap_bytes": bucket_cap_bytes,
            "model_impl": model_impl,
            "manifest_hash": manifest_hash,
            "topology_hash": topology_hash,
            "fragment_hash": fragment_hash,
            "process_groups": [asdict(g) for g in groups],
            "canonical_fragments": [asdict(f) for f in fragments],
            "local_fragment_bindings_by_rank": bindings_payload,
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
        process_group_index_by_id=tuple((g.process_group_id, i) for i, g in enumerate(groups)),
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
    """Creates each process group exactly once (bucket_plan.py:244-280)."""

    def __init__(self, process_groups, create_group):
        self._groups = tuple(sorted(process_groups, key=lambda g: g.ranks))
        self._create_group = create_group
        self._handles = {}
        self._creation_count = 0

    def initialize(self):
        if self._handles:
            return
        ids, rank_sets = set(), set()
        for g in self._groups:
            if g.process_group_id in ids:
                raise ValueError(f"duplicate process group id {g.process_group_id}")
            if g.ranks in rank_sets:
                raise ValueError(f"duplicate process group ranks {g.ranks}")
            if g.ranks != tuple(sorted(set(g.ranks))):
                raise ValueError(f"process group ranks must be sorted and unique: {g.ranks}")
            ids.add(g.process_group_id)
            rank_sets.add(g.ranks)
            self._handles[g.process_group_id] = self._create_group(g.ranks)
            self._creation_count += 1

    @property
    def group_count(self):
        return len(self._handles)

    @property
    def creation_count(self):
        return self._creation_count

    def handle(self, process_group_id):
        if process_group_id not in self._handles:
            raise KeyError(f"process group {process_group_id} is not initialized")
        return self._handles[process_group_id]
