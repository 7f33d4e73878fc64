"""CPU tests: bucket planning / fragment planning (product host code) and the
grad-sync + AdamW oracle, against the reference tests' known answers."""

import math

import numpy as np
import pytest
import torch

from eth_amd.grad_sync import bucket_plan as bp
from eth_amd.grad_sync.planner import (
    CanonicalFragmentPlan,
    LocalFragmentBindingSpec,
    ProcessGroupSpec,
    TensorSegmentSpec,
    plan_canonical_fragments,
)
from oracle import adamw as oadam
from oracle import gradsync as og
from tests.helpers import (
    descriptors_for,
    fragment,
    gpt_layer_shapes,
    known_answers,
    named_fragment,
    single_rank_descriptor,
)

KA = known_answers()


def _plan_from(record, mode, cap):
    groups = tuple(ProcessGroupSpec(g, tuple(r), "gradient_sync") for g, r in record["groups"])
    frags = tuple(fragment(i, g, d, n) for i, g, d, n in record["fragments"])
    return bp.build_gradient_sync_plan(CanonicalFragmentPlan(groups, frags, (), "h"), mode, cap, "gpt", "m", "t")


def test_tensor_and_block_modes_share_semantics():
    rec = KA["bucket_plan_tensor_vs_block"]
    tensor = _plan_from(rec, "tensor", rec["cap_bytes"])
    block = _plan_from(rec, "block", rec["cap_bytes"])
    assert len(tensor.global_bucket_order) == rec["expected_tensor_buckets"]
    assert len(block.global_bucket_order) == rec["expected_block_buckets"]
    assert tensor.canonical_fragments == block.canonical_fragments
    assert tensor.global_fragment_hash == block.global_fragment_hash
    assert tensor.exact_payload_bytes_by_rank == block.exact_payload_bytes_by_rank
    assert tensor.padding_payload_bytes == block.padding_payload_bytes == 0
    assert tensor.global_plan_hash != block.global_plan_hash


def test_cap_dtype_group_boundaries_never_split():
    rec = KA["bucket_plan_boundaries"]
    plan = _plan_from(rec, "block", rec["cap_bytes"])
    assert len(plan.global_bucket_order) == rec["expected_block_buckets"]
    last = plan.global_bucket_order[-1]
    assert last.oversized is rec["expected_last_oversized"]
    assert last.exact_numel == rec["expected_last_numel"]
    assert all(b.placements[0].destination_offset == 0 for b in plan.global_bucket_order)


def test_plan_is_independent_of_input_order():
    rec = KA["bucket_plan_tensor_vs_block"]
    groups = tuple(ProcessGroupSpec(g, tuple(r), "gradient_sync") for g, r in rec["groups"])
    frags = tuple(fragment(i, g, d, n) for i, g, d, n in rec["fragments"])
    for cap_mib in (1, 32, 256):
        a = bp.build_gradient_sync_plan(CanonicalFragmentPlan(groups, frags, (), "h"), "block", cap_mib << 20, "gpt", "m", "t")
        b = bp.build_gradient_sync_plan(
            CanonicalFragmentPlan(tuple(reversed(groups)), tuple(reversed(frags)), (), "h"), "block", cap_mib << 20, "gpt", "m", "t"
        )
        assert a == b


def test_bucketize_rejects_bad_mode_and_cap():
    with pytest.raises(ValueError):
        bp.bucketize((), "ring", 16, {})
    with pytest.raises(ValueError):
        bp.bucketize((), "block", 0, {})


def test_gpt_1p3b_grad_list_gives_121_block_and_288_tensor_buckets():
    # 24 layers of hidden 2048, fp32 grads, 32 MiB buckets
    shapes = gpt_layer_shapes(2048, 8192, 24)
    fplan = plan_canonical_fragments(descriptors_for(shapes), (0,))
    numel = sum(math.prod(s[1]) for s in shapes)
    assert numel == 1_208_598_528
    block = bp.build_gradient_sync_plan(fplan, "block", 32 << 20, "gpt", "m", "t")
    tensor = bp.build_gradient_sync_plan(fplan, "tensor", 32 << 20, "gpt", "m", "t")
    assert len(tensor.global_bucket_order) == 288
    assert len(block.global_bucket_order) == 121
    assert sum(b.oversized for b in block.global_bucket_order) == 72
    dup = [b for b in block.global_bucket_order if b.reduction_semantics == "sum_identical_duplicates"]
    assert len(dup) == 1 and dup[0].exact_numel == 294_912
    assert dict(block.max_scratch_numel_by_rank_and_dtype)[(0, "torch.float32")] == 16_777_216
    assert sum(b.exact_numel for b in block.global_bucket_order) == numel
    for b in block.global_bucket_order:  # offsets are contiguous, no padding
        off = 0
        for p in b.placements:
            assert p.destination_offset == off
            off += next(f.numel for f in block.canonical_fragments if f.fragment_id == p.fragment_id)
        assert off == b.exact_numel


def test_replicated_tp2_contributes_half_and_sharded_tp2_splits():
    # two TP ranks of one pipeline: a column weight [4,2] split on dim 0 and
    # a replicated bias; checks the planner's segments and scales
    def desc(rank, lid, full, local, tp, pdim):
        d = single_rank_descriptor(lid, local, (1, 0 if "w" in lid else 1, lid), tp, pdim)
        return d.__class__(
            **{
                **d.__dict__,
                "global_rank": rank,
                "local_tp_degree": 2,
                "local_tp_rank": rank,
                "local_tp_group_ranks": (0, 1),
                "local_dp_group_ranks": (rank,),
                "stage_ranks": (0, 1),
                "full_shape": full,
                "local_shape": local,
            }
        )

    ds = [desc(r, "w", (4, 2), (2, 2), True, 0) for r in range(2)] + [desc(r, "b", (2,), (2,), False, -1) for r in range(2)]
    plan = plan_canonical_fragments(ds, (0,))
    rep = [f for f in plan.fragments if f.logical_param_id == "b"]
    assert len(rep) == 1 and rep[0].reduction_semantics == "sum_identical_duplicates"
    for rank in range(2):
        bs = {b.logical_param_id: b for b in plan.bindings_for_rank(rank)}
        assert bs["b"].contribution_scale == 0.5
        w = [b for b in plan.bindings_for_rank(rank) if b.logical_param_id == "w"]
        assert len(w) == 1 and w[0].source_segments[0].flattened_numel == 4


# ------------------------------------------------------------- oracle pins --
def _strided_plan(rec):
    group = ProcessGroupSpec("pg", (0, 1), "gradient_sync")
    frags, bindings = [], []
    for f in rec["fragments"]:
        frags.append(named_fragment(f["id"], "weight", "pg", f["numel"], f["order"]))
        segs = tuple(TensorSegmentSpec(o, l, tuple(rec["main_grad_shape"]), o, o + l, l * 3) for o, l in f["segments"])
        bindings.append(LocalFragmentBindingSpec(0, f["id"], "weight", segs, 1.0))
    fplan = CanonicalFragmentPlan((group,), tuple(frags), ((0, tuple(bindings)),), "h")
    return bp.build_gradient_sync_plan(fplan, rec["mode"], rec["cap_bytes"], "gpt", "m", "t")


def test_oracle_strided_pack_known_answer():
    rec = KA["executor_strided_pack"]
    plan = _strided_plan(rec)
    grads = {"weight": np.arange(12, dtype=np.float32).reshape(4, 3)}
    desc = {"weight": type("D", (), {"partition_dim": 0})()}
    packed = og.execute(plan, 0, desc, grads, rec["normalization_scale"], lambda p, h: p.__imul__(2))
    assert [p.tolist() for p in packed] == rec["expected_packed"]
    assert grads["weight"].ravel().tolist() == rec["expected_main_grad"]


def test_oracle_clip_known_answer():
    rec = KA["canonical_clip"]
    grads = [np.asarray(g, dtype=np.float32) for g in rec["owned_grads"]]
    norm = og.l2_norm(grads)
    assert norm == pytest.approx(rec["expected_norm"], rel=1e-12)
    assert og.count_zeros(grads) == rec["expected_zeros"]
    og.clip(grads, norm, rec["max_norm"])
    np.testing.assert_allclose(grads[0], rec["expected_clipped"][0], rtol=1e-6)
    assert og.inf_norm(grads) == pytest.approx(rec["expected_inf_norm"], rel=1e-6)


def test_oracle_unscale_flags_nonfinite():
    g = [np.array([1.0, np.inf, 2.0], dtype=np.float32), np.array([4.0], dtype=np.float32)]
    assert og.unscale_and_check(g, 0.5)
    assert g[1][0] == 2.0
    g = [np.array([1.0, 2.0], dtype=np.float32)]
    assert not og.unscale_and_check(g, 2.0**-16)
    assert g[0][1] == 2.0 * 2.0**-16  # power-of-two scale is exact


def test_oracle_adamw_step1_closed_form_and_torch():
    rec = KA["adamw_step1"]
    p = np.asarray(rec["param"], dtype=np.float64)
    g = np.asarray(rec["grad"], dtype=np.float64)
    norm = og.l2_norm([g])
    assert norm == pytest.approx(rec["expected_norm"])
    coef = og.clip_coefficient(norm, rec["max_norm"])
    assert coef == pytest.approx(1.0 / (5.0 + 1e-6))
    gc = g * coef
    b1, b2 = rec["betas"]
    np_, m, v = oadam.adamw_step(p, gc, np.zeros(2), np.zeros(2), 1, rec["lr"], b1, b2, rec["eps"], rec["weight_decay"])
    np.testing.assert_allclose(m, gc * rec["expected_exp_avg_over_grad"], rtol=1e-12)
    np.testing.assert_allclose(v, gc * gc * rec["expected_exp_avg_sq_over_grad_sq"], rtol=1e-12)
    tp = torch.nn.Parameter(torch.tensor(rec["param"], dtype=torch.float64))
    opt = torch.optim.AdamW([tp], lr=rec["lr"], betas=(b1, b2), eps=rec["eps"], weight_decay=rec["weight_decay"])
    tp.grad = torch.tensor(gc)
    opt.step()
    np.testing.assert_allclose(np_, tp.detach().numpy(), rtol=1e-14)
    # step-1 update is -lr*sign(g) up to eps, after decay
    np.testing.assert_allclose(np_, p * (1 - rec["lr"] * rec["weight_decay"]) - rec["lr"] * np.sign(g), rtol=1e-6)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_oracle_adamw_matches_torch_over_steps(dtype):
    rng = np.random.default_rng(0)
    n = 1000
    p = rng.normal(0, 0.02, n).astype(dtype)
    m = np.zeros(n, dtype)
    v = np.zeros(n, dtype)
    tp = torch.nn.Parameter(torch.tensor(p))
    opt = torch.optim.AdamW([tp], lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
    for step in range(1, 4):
        g = rng.normal(0, 1e-3, n).astype(dtype)
        p, m, v = oadam.adamw_step(p, g, m, v, step, 1e-4, 0.9, 0.95, 1e-8, 0.1)
        tp.grad = torch.tensor(g)
        opt.step()
    st = opt.state[tp]
    if dtype == np.float32:
        # moments bit-exact (same fma structure as torch's CPU kernels); the
        # parameter within 1e-6 relative because torch's vectorized CPU sqrt
        # is not correctly rounded while the oracle's (and the GPU's) is
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-6, atol=2e-8)
        np.testing.assert_array_equal(m, st["exp_avg"].numpy())
        np.testing.assert_array_equal(v, st["exp_avg_sq"].numpy())
    else:
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(m, st["exp_avg"].numpy(), rtol=1e-13, atol=1e-18)
        np.testing.assert_allclose(v, st["exp_avg_sq"].numpy(), rtol=1e-13, atol=1e-21)


def test_oracle_bf16_rounding():
    x = np.array([1.0, 1.00390625, 1.01171875, -3.5, np.inf], dtype=np.float32)
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(oadam.to_bf16(x), ref)


def test_shadowed_prefixes_and_chunk_marks():
    """The payload prefix a later bucket of the same dtype packs over, per
    bucket in plan order, and the chunks marked inside it (hand-worked)."""
    from collections import namedtuple

    from eth_amd import _native as nat
    from eth_amd.grad_sync.executor import mark_shadowed, shadowed_prefixes

    B = namedtuple("B", "grad_dtype exact_numel")
    buckets = [B("f32", 10), B("bf16", 50), B("f32", 30), B("f32", 20), B("bf16", 5), B("f32", 4)]
    assert shadowed_prefixes(buckets) == [30, 5, 20, 4, 0, 0]
    assert shadowed_prefixes([]) == []
    # (src, dst, stride, rows, row_len, scale, flags): payload ranges [0, 8), [8, 20), [20, 30)
    entries = [(0, 0, 8, 1, 8, 1.0, nat.CHUNK_NORM), (0, 8, 4, 3, 4, 1.0, 0), (0, 20, 10, 1, 10, 1.0, 0)]
    flags = [e[6] for e in mark_shadowed(entries, 20)]
    assert flags == [nat.CHUNK_NORM | nat.CHUNK_SHADOWED, nat.CHUNK_SHADOWED, 0]
    assert [e[6] for e in mark_shadowed(entries, 19)] == [nat.CHUNK_NORM | nat.CHUNK_SHADOWED, 0, 0]
    assert mark_shadowed(entries, 0) == entries
