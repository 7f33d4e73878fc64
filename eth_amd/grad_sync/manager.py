"""Gradient-sync lifecycle (single process group owner per rank).

Mirrors eth/runtime/megatron/grad_sync/manager.py:31-32,122-214: plan the
canonical fragments from every rank's descriptors, build the bucket plan,
cross-check the plan hash, create each process group once and hand back a
manager whose `execute(normalization_scale)` runs the executor.  The
descriptor exchange is a callable (`all_gather_object`) so the same code runs
at world size 1 without torch.distributed.
"""

from .bucket_plan import ProcessGroupRegistry, build_gradient_sync_plan
from .executor import GradientBucketExecutor, local_all_reduce_sum
from .planner import plan_canonical_fragments


class GradientSyncManager:
    def __init__(self, plan, executor, registry):
        self.plan = plan
        self.executor = executor
        self.registry = registry

    def execute(self, normalization_scale=1.0):
        if hasattr(normalization_scale, "item"):
            normalization_scale = float(normalization_scale.item())
        self.executor.execute(normalization_scale)


def _single_rank_all_gather(obj):
    return [obj]


def initialize_gradient_sync(
    descriptors,
    bindings,
    global_rank,
    expected_pipeline_ids,
    sync_mode="block",
    bucket_cap_bytes=32 * 1024 * 1024,
    model_impl="gpt",
    manifest_hash="manifest",
    topology_hash="topology",
    all_gather_object=_single_rank_all_gather,
    create_group=lambda ranks: ranks,
    all_reduce_sum=local_all_reduce_sum,
    runtime_evidence_dir=None,
):
    """Plan, verify and bind gradient synchronization for this rank."""
    gathered = all_gather_object(tuple(descriptors))
    all_descriptors = tuple(d for part in gathered for d in part)
    fragment_plan = plan_canonical_fragments(all_descriptors, expected_pipeline_ids)
    plan = build_gradient_sync_plan(fragment_plan, sync_mode, bucket_cap_bytes, model_impl, manifest_hash, topology_hash)
    hashes = all_gather_object(plan.global_plan_hash)
    if len(set(hashes)) != 1:
        raise ValueError(f"gradient sync plan hash mismatch across ranks: {sorted(set(hashes))}")
    registry = ProcessGroupRegistry(plan.process_groups, create_group)
    registry.initialize()
    executor = GradientBucketExecutor(
        plan, global_rank, tuple(descriptors), tuple(bindings), registry, all_reduce_sum,
        runtime_evidence_dir=runtime_evidence_dir,
    )
    return GradientSyncManager(plan, executor, registry)
