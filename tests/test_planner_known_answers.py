"""CPU tests of the fragment planner (eth_amd/grad_sync/planner.py) on the
multi-rank layouts of the reference's planner tests
(tests/test_gradient_fragment_planner.py:94-278): mixed TP degrees between
pipelines, stride-2 partitions, replicated parameters, shared weights and
the rejected layouts.  The planner runs per rank in a deployment; here all
ranks' descriptors are planned at once, as the reference's tests do."""

import random
from dataclasses import replace

import pytest

from eth_amd.grad_sync.metadata import SerializableGradientDescriptor
from eth_amd.grad_sync.planner import canonical_regions, plan_canonical_fragments


def desc(lid, rank, pipeline, tp_degree, tp_rank, full, local, tensor_parallel, partition_dim, stride=1,
         dtype="float32", dp_degree=1, dp_rank=0, shared_id=None, shared_root=False, tp_group=None, dp_group=None,
         stage_ranks=None):
    start = rank - tp_rank
    tp_group = tp_group or tuple(range(start, start + tp_degree))
    dp_group = dp_group or (rank,)
    stage_ranks = stage_ranks or tuple(sorted(set(tp_group + dp_group)))
    return SerializableGradientDescriptor(
        logical_param_id=lid, shared_weight_id=shared_id, shared_weight_root=shared_root, logical_region_key=lid,
        semantic_order_key=(0, 0, lid), global_rank=rank, model_impl="gpt", op_manifest_hash="manifest",
        pipeline_id=pipeline, stage_id=0, model_chunk_id=0, global_op_index=1, manifest_op_name="op",
        runtime_op_name="op", relative_parameter_name="weight", stage_global_op_begin=0, stage_global_op_end=1,
        local_tp_degree=tp_degree, local_tp_rank=tp_rank, local_dp_degree=dp_degree, local_dp_rank=dp_rank,
        local_cp_degree=1, local_cp_rank=0, stage_ranks=stage_ranks, local_tp_group_ranks=tp_group,
        local_dp_group_ranks=dp_group, full_shape=full, local_shape=local, tensor_parallel=tensor_parallel,
        tp_replica_semantics=None if tensor_parallel else "identical_duplicate", partition_dim=partition_dim,
        partition_stride=stride, parameter_dtype="float16", gradient_dtype=dtype, requires_grad=True,
    )


def _mixed_dim0():
    return [
        desc("weight", 0, 0, 1, 0, (8, 2), (8, 2), True, 0),
        desc("weight", 1, 1, 2, 0, (8, 2), (4, 2), True, 0),
        desc("weight", 2, 1, 2, 1, (8, 2), (4, 2), True, 0),
    ]


def test_canonical_regions_with_stride():
    assert canonical_regions(8, 2, 0, 2) == ((0, 2), (4, 6))
    assert canonical_regions(8, 2, 1, 2) == ((2, 4), (6, 8))
    assert canonical_regions(12, 1, 0, 3) == ((0, 4), (4, 8), (8, 12))
    with pytest.raises(ValueError, match="nondivisible"):
        canonical_regions(6, 4, 0, 1)


def test_dim0_mixed_tp_layouts_give_canonical_shards_and_bindings():
    plan = plan_canonical_fragments(_mixed_dim0(), (0, 1))
    assert [g.ranks for g in plan.process_groups] == [(0, 1), (0, 2)]
    assert [f.canonical_shard_id for f in plan.fragments] == [0, 1]
    assert [f.numel for f in plan.fragments] == [8, 8]
    rank0 = plan.bindings_for_rank(0)
    assert [(b.source_segments[0].source_dim_offset, b.source_segments[0].source_dim_length) for b in rank0] == [
        (0, 4), (4, 4)]
    # the TP-2 ranks each hold one whole canonical shard at local offset 0
    for rank, shard in ((1, 0), (2, 1)):
        (b,) = plan.bindings_for_rank(rank)
        assert b.fragment_id == plan.fragments[shard].fragment_id
        assert b.source_segments[0].source_dim_offset == 0 and b.source_segments[0].source_dim_length == 4


def test_dim1_stride_two_keeps_both_global_intervals():
    ds = []
    for pipeline, start in enumerate((0, 2)):
        ds += [desc("weight", start, pipeline, 2, 0, (2, 8), (2, 4), True, 1, 2),
               desc("weight", start + 1, pipeline, 2, 1, (2, 8), (2, 4), True, 1, 2)]
    plan = plan_canonical_fragments(ds, (0, 1))
    assert plan.fragments[0].global_regions == ((0, 2), (4, 6))
    b = plan.bindings_for_rank(0)[0]
    assert [(s.source_dim_offset, s.source_dim_length) for s in b.source_segments] == [(0, 2), (2, 2)]


def test_stride_two_between_tp1_and_tp2_maps_local_offsets():
    """TP 1 holds the whole axis; TP 2 rank r holds blocks r and r + 2 of
    four.  Canonical shard 1 is global [2,4) + [6,8): local offsets 2 and 6
    on the TP-1 rank, 0 and 2 on TP rank 1."""
    ds = [desc("weight", 0, 0, 1, 0, (8, 3), (8, 3), True, 0, 2),
          desc("weight", 1, 1, 2, 0, (8, 3), (4, 3), True, 0, 2),
          desc("weight", 2, 1, 2, 1, (8, 3), (4, 3), True, 0, 2)]
    plan = plan_canonical_fragments(ds, (0, 1))
    shard1 = plan.fragments[1]
    assert shard1.global_regions == ((2, 4), (6, 8)) and shard1.numel == 12
    segs = {b.global_rank: [(s.source_dim_offset, s.source_dim_length, s.flattened_numel) for s in b.source_segments]
            for rank in range(3) for b in plan.bindings_for_rank(rank) if b.fragment_id == shard1.fragment_id}
    assert segs == {0: [(2, 2, 6), (6, 2, 6)], 2: [(0, 2, 6), (2, 2, 6)]}


def test_replicated_parameter_scales_every_tp_holder():
    ds = [desc("bias", 0, 0, 1, 0, (4,), (4,), False, -1),
          desc("bias", 1, 1, 2, 0, (4,), (4,), False, -1),
          desc("bias", 2, 1, 2, 1, (4,), (4,), False, -1)]
    plan = plan_canonical_fragments(ds, (0, 1))
    assert plan.process_groups[0].ranks == (0, 1, 2)
    assert plan.fragments[0].canonical_shard_id is None
    assert plan.fragments[0].reduction_semantics == "sum_identical_duplicates"
    assert [plan.bindings_for_rank(r)[0].contribution_scale for r in range(3)] == [1.0, 0.5, 0.5]


def test_shared_root_is_the_only_norm_fragment():
    ds = [desc("embedding", 0, 0, 1, 0, (4,), (4,), False, -1, shared_id="shared", shared_root=True),
          desc("embedding", 1, 1, 1, 0, (4,), (4,), False, -1, shared_id="shared", shared_root=True),
          desc("head", 0, 0, 1, 0, (4,), (4,), False, -1, shared_id="shared"),
          desc("head", 1, 1, 1, 0, (4,), (4,), False, -1, shared_id="shared")]
    by_id = {f.logical_param_id: f for f in plan_canonical_fragments(ds, (0, 1)).fragments}
    assert by_id["embedding"].include_in_optimizer_norm and by_id["embedding"].norm_owner_rank == 0
    assert not by_id["head"].include_in_optimizer_norm and by_id["head"].norm_owner_rank is None
    assert by_id["head"].optimizer_semantic_id == "shared"


def test_groups_are_shared_and_pipelines_dp_and_roots_are_validated():
    mixed = []
    for rank, pipeline in ((0, 0), (1, 1)):
        mixed += [desc("weight", rank, pipeline, 1, 0, (4,), (4,), True, 0),
                  desc("bias", rank, pipeline, 1, 0, (4,), (4,), False, -1)]
    plan = plan_canonical_fragments(mixed, (0, 1))
    assert len(plan.process_groups) == 1 and len(plan.fragments) == 2
    with pytest.raises(ValueError, match="missing owner pipeline.*1"):
        plan_canonical_fragments(mixed[:2], (0, 1))
    dp = [desc("bias", r, r // 2, 1, 0, (4,), (4,), False, -1, dp_degree=2, dp_rank=r % 2,
               dp_group=(2 * (r // 2), 2 * (r // 2) + 1), stage_ranks=(2 * (r // 2), 2 * (r // 2) + 1))
          for r in range(4)]
    assert plan_canonical_fragments(dp, (0, 1)).process_groups[0].ranks == (0, 1, 2, 3)
    no_root = [desc("head", r, r, 1, 0, (4,), (4,), False, -1, shared_id="shared") for r in (0, 1)]
    with pytest.raises(ValueError, match="shared root mismatch"):
        plan_canonical_fragments(no_root, (0, 1))
    two_roots = no_root + [desc(n, r, r, 1, 0, (4,), (4,), False, -1, shared_id="shared", shared_root=True)
                           for n in ("embedding", "other_root") for r in (0, 1)]
    with pytest.raises(ValueError, match="shared root mismatch"):
        plan_canonical_fragments(two_roots, (0, 1))


def test_shape_mismatch_reports_every_rank_layout():
    ds = [desc("weight", 0, 0, 1, 0, (8, 2), (8, 2), True, 0), desc("weight", 1, 1, 1, 0, (4, 2), (4, 2), True, 0)]
    with pytest.raises(ValueError, match=r"shape mismatch for weight: .*rank=0.*full=\(8, 2\).*rank=1.*full=\(4, 2\)"):
        plan_canonical_fragments(ds, (0, 1))


def test_rejected_layouts_and_input_order_independence():
    valid = _mixed_dim0()
    shuffled = list(valid)
    random.Random(7).shuffle(shuffled)
    assert plan_canonical_fragments(valid, (0, 1)) == plan_canonical_fragments(shuffled, (0, 1))
    cases = {
        "nondivisible": [desc("weight", r, 0, 3, r, (8, 2), (3, 2), True, 0) for r in range(3)],
        "axis mismatch": [valid[0], desc("weight", 1, 1, 1, 0, (8, 2), (8, 2), True, 1)],
        "dtype mismatch": [valid[0], desc("weight", 1, 1, 1, 0, (8, 2), (8, 2), True, 0, dtype="float16")],
        "shape mismatch": [desc("weight", r, 0, 2, r, (2, 8, 3), (3, 4, 2), True, 1) for r in range(2)],
        "replica semantics": [replace(desc("bias", 0, 0, 1, 0, (4,), (4,), False, -1), tp_replica_semantics="replicated")],
    }
    for phrase, case in cases.items():
        expected = (0, 1) if len({d.pipeline_id for d in case}) > 1 else (0,)
        with pytest.raises(ValueError, match=phrase):
            plan_canonical_fragments(case, expected)
