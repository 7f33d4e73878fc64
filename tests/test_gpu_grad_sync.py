"""GPU parity: GradientBucketExecutor (HIP pack/unpack) against the oracle
and the reference tests' known answers.  Bit-exact for every copy/scale;
norm within 1e-6 relative of the fp64 oracle."""

import math

import numpy as np
import pytest
import torch

from eth_amd.grad_sync import bucket_plan as bp
from eth_amd.grad_sync.executor import GradientBucketExecutor, GradientStatistics, local_all_reduce_sum
from eth_amd.grad_sync.planner import (
    CanonicalFragmentPlan,
    LocalFragmentBindingSpec,
    ProcessGroupSpec,
    TensorSegmentSpec,
    plan_canonical_fragments,
)
from eth_amd.grad_sync.synthetic import single_rank_descriptor
from oracle import gradsync as og
from tests.conftest import announce
from tests.helpers import (
    FakeRegistry,
    descriptors_for,
    gpt_layer_shapes,
    known_answers,
    named_fragment,
    runtime_binding,
)

pytestmark = pytest.mark.gpu
KA = known_answers()


class Desc:
    def __init__(self, lid, pdim, tp=None):
        self.logical_param_id = lid
        self.partition_dim = pdim
        if tp is not None:
            self.tensor_parallel = tp


def test_strided_pack_known_answer(cuda):
    announce("grad_sync strided pack known answer")
    rec = KA["executor_strided_pack"]
    group = ProcessGroupSpec("pg", (0, 1), "gradient_sync")
    frags, bindings = [], []
    for f in rec["fragments"]:
        frags.append(named_fragment(f["id"], "weight", "pg", f["numel"], f["order"]))
        segs = tuple(TensorSegmentSpec(o, l, (4, 3), o, o + l, l * 3) for o, l in f["segments"])
        bindings.append(LocalFragmentBindingSpec(0, f["id"], "weight", segs, 1.0))
    fplan = CanonicalFragmentPlan((group,), tuple(frags), ((0, tuple(bindings)),), "h")
    plan = bp.build_gradient_sync_plan(fplan, "block", rec["cap_bytes"], "gpt", "m", "t")
    main_grad = torch.arange(12, dtype=torch.float32, device=cuda).view(4, 3)
    packed = []

    def all_reduce_sum(payload, handle):
        assert handle == "cached-pg"
        packed.append(payload.clone())
        payload.mul_(2)

    reg = FakeRegistry()
    ex = GradientBucketExecutor(plan, 0, (Desc("weight", 0),), (runtime_binding("weight", main_grad),), reg, all_reduce_sum)
    ex.execute(normalization_scale=rec["normalization_scale"])
    torch.cuda.synchronize()
    assert reg.calls == ["pg"]
    assert packed[0].cpu().tolist() == rec["expected_packed"][0]
    assert main_grad.cpu().reshape(-1).tolist() == rec["expected_main_grad"]


def test_scratch_reuse_leaves_short_bucket_tail(cuda):
    announce("grad_sync scratch tail known answer")
    rec = KA["executor_scratch_tail"]
    group = ProcessGroupSpec("pg", (0,), "gradient_sync")
    frags = (named_fragment("large", "large-param", "pg", 8, 0), named_fragment("small", "small-param", "pg", 4, 1))
    bindings = (
        LocalFragmentBindingSpec(0, "large", "large-param", (TensorSegmentSpec(0, 8, (8,), 0, 8, 8),), 1.0),
        LocalFragmentBindingSpec(0, "small", "small-param", (TensorSegmentSpec(0, 4, (4,), 0, 4, 4),), 1.0),
    )
    plan = bp.build_gradient_sync_plan(CanonicalFragmentPlan((group,), frags, ((0, bindings),), "h"), "tensor", 1024, "gpt", "m", "t")
    large = torch.zeros(8, device=cuda)
    small = torch.zeros(4, device=cuda)
    seen = []

    def all_reduce_sum(payload, handle):
        seen.append(payload.numel())
        payload.add_(100)

    ex = GradientBucketExecutor(
        plan,
        0,
        (Desc("large-param", 0), Desc("small-param", 0)),
        (runtime_binding("large-param", large), runtime_binding("small-param", small)),
        FakeRegistry(),
        all_reduce_sum,
    )
    for _ in range(rec["iterations"]):
        large.copy_(torch.tensor(rec["tensors"]["large-param"], dtype=torch.float32))
        small.copy_(torch.tensor(rec["tensors"]["small-param"], dtype=torch.float32))
        ex.execute()
        torch.cuda.synchronize()
        assert ex.scratch("float32")[4:].cpu().tolist() == rec["expected_scratch_tail"]
    assert seen == rec["expected_numels"]


@pytest.mark.parametrize("large_first", [True, False])
@pytest.mark.parametrize("local", [True, False])
def test_normalized_pass_leaves_the_reference_scratch(cuda, large_first, local):
    """With a normalization scale the reference multiplies each bucket's
    payload in place before its unpack (executor.py:247-261), so a pass
    leaves the scratch holding, at every offset, the normalized payload of
    the last bucket reaching it.  The unpack skips the write-back of chunks a
    later bucket packs over; the scratch a pass leaves is still exactly that
    (8- and 4-element buckets in both orders, both seams)."""
    announce(f"grad_sync normalized scratch, large_first={large_first} local={local}")
    group = ProcessGroupSpec("pg", (0,), "gradient_sync")
    order = (0, 1) if large_first else (1, 0)
    frags = (named_fragment("large", "large-param", "pg", 8, order[0]),
             named_fragment("small", "small-param", "pg", 4, order[1]))
    bindings = (
        LocalFragmentBindingSpec(0, "large", "large-param", (TensorSegmentSpec(0, 8, (8,), 0, 8, 8),), 1.0),
        LocalFragmentBindingSpec(0, "small", "small-param", (TensorSegmentSpec(0, 4, (4,), 0, 4, 4),), 1.0),
    )
    plan = bp.build_gradient_sync_plan(CanonicalFragmentPlan((group,), frags, ((0, bindings),), "h"), "tensor", 1024, "gpt", "m", "t")
    large = torch.arange(1, 9, dtype=torch.float32, device=cuda) * 3.0
    small = -torch.arange(1, 5, dtype=torch.float32, device=cuda)
    add = 0.0 if local else 100.0

    def all_reduce_sum(payload, handle):
        payload.add_(add)

    seam = local_all_reduce_sum if local else all_reduce_sum
    ex = GradientBucketExecutor(plan, 0, (Desc("large-param", 0), Desc("small-param", 0)),
                                (runtime_binding("large-param", large), runtime_binding("small-param", small)),
                                FakeRegistry(), seam)
    assert ex.n_buckets == 2
    l0, s0 = large.clone(), small.clone()
    scale = 0.3701
    ex.execute(scale)
    torch.cuda.synchronize()
    ln, sn = (l0 + add) * scale, (s0 + add) * scale
    assert torch.equal(large, ln) and torch.equal(small, sn)
    sizes = [t[0].exact_numel for t in ex._tables]  # buckets in execution order
    assert sizes == ([8, 4] if large_first else [4, 8])
    want = torch.cat([sn, ln[4:]]) if large_first else ln.clone()
    assert torch.equal(ex.scratch("float32")[:8], want)


def test_replicated_half_contribution_scale(cuda):
    announce("grad_sync replicated fp16 x0.5")
    rec = KA["executor_replicated_half"]
    group = ProcessGroupSpec("pg", (0, 1), "gradient_sync")
    frag = named_fragment("f", "bias", "pg", 4, 0, dtype="float16", reduction="sum_identical_duplicates")
    binding = LocalFragmentBindingSpec(0, "f", "bias", (TensorSegmentSpec(0, 4, (4,), 0, 4, 4),), rec["contribution_scale"])
    plan = bp.build_gradient_sync_plan(CanonicalFragmentPlan((group,), (frag,), ((0, (binding,)),), "h"), "tensor", 1024, "gpt", "m", "t")
    g = torch.zeros(4, dtype=torch.float16, device=cuda)

    def all_reduce_sum(payload, handle):
        assert payload.dtype == torch.float16
        payload.mul_(2)

    ex = GradientBucketExecutor(plan, 0, (Desc("bias", 0),), (runtime_binding("bias", g),), FakeRegistry(), all_reduce_sum)
    ex.execute()
    torch.cuda.synchronize()
    assert torch.equal(g.cpu(), torch.zeros(4, dtype=torch.float16))
    g.copy_(torch.tensor(rec["main_grad"], dtype=torch.float16))
    ex.execute()
    torch.cuda.synchronize()
    assert g.cpu().tolist() == rec["expected_main_grad"]


def test_validation_errors_carry_bucket_context(cuda):
    group = ProcessGroupSpec("pg", (0,), "gradient_sync")
    frag = named_fragment("f", "w", "pg", 4, 0)
    binding = LocalFragmentBindingSpec(0, "f", "w", (TensorSegmentSpec(0, 4, (4,), 0, 4, 4),), 1.0)
    plan = bp.build_gradient_sync_plan(CanonicalFragmentPlan((group,), (frag,), ((0, (binding,)),), "h"), "tensor", 1024, "gpt", "m", "t")
    bad = torch.zeros(5, device=cuda)
    with pytest.raises(ValueError, match=r"bucket bucket-\w+ rank 0 logical_param_id w fragment f: main_grad shape mismatch"):
        GradientBucketExecutor(plan, 0, (Desc("w", 0),), (runtime_binding("w", bad),), FakeRegistry(), lambda p, h: None)


def _gpt_setup(cuda, hidden, ffn, layers, cap_bytes, mode, seed, dtype=torch.float32):
    shapes = gpt_layer_shapes(hidden, ffn, layers)
    if dtype == torch.float32:
        descs = descriptors_for(shapes)
    else:
        descs = [single_rank_descriptor(lid, shape, (op, order, lid), tp, pdim, dtype=str(dtype))
                 for lid, shape, op, order, tp, pdim in shapes]
    fplan = plan_canonical_fragments(descs, (0,))
    plan = bp.build_gradient_sync_plan(fplan, mode, cap_bytes, "gpt", "m", "t")
    gen = torch.Generator().manual_seed(seed)
    # one contiguous main-grad buffer carved from the end, as LocalDDP does
    total = sum(math.prod(s[1]) for s in shapes)
    buf = torch.empty(total, dtype=dtype, device=cuda)
    grads, off = {}, total
    for lid, shape, *_ in shapes:
        n = math.prod(shape)
        off -= n
        grads[lid] = buf[off : off + n].view(shape)
        grads[lid].copy_(torch.randn(shape, generator=gen) * 1e-3)
    bindings = [runtime_binding(lid, grads[lid]) for lid, *_ in shapes]
    return plan, descs, grads, bindings


@pytest.mark.parametrize("mode,cap", [("block", 1 << 16), ("tensor", 1 << 16), ("block", 1 << 12)])
def test_gpt_grad_list_bit_exact_vs_oracle(cuda, mode, cap):
    announce(f"grad_sync gpt list mode={mode} cap={cap}")
    plan, descs, grads, bindings = _gpt_setup(cuda, 64, 256, 3, cap, mode, seed=1234)
    host = {k: v.cpu().numpy().copy() for k, v in grads.items()}
    packed = []

    def all_reduce_sum(payload, handle):
        packed.append(payload.cpu().numpy().copy())

    ex = GradientBucketExecutor(plan, 0, descs, bindings, FakeRegistry(), all_reduce_sum)
    norm_scale = 0.3701
    ex.execute(norm_scale)
    torch.cuda.synchronize()
    ref_packed = og.execute(plan, 0, {d.logical_param_id: d for d in descs}, host, norm_scale)
    assert len(packed) == len(ref_packed) == len(plan.global_bucket_order)
    for a, b in zip(packed, ref_packed):
        np.testing.assert_array_equal(a, b)
    for lid, g in grads.items():
        np.testing.assert_array_equal(g.cpu().numpy(), host[lid])


def test_fused_unscale_flag_and_norm(cuda):
    announce("grad_sync fused unscale/flag/norm")
    plan, descs, grads, bindings = _gpt_setup(cuda, 64, 256, 2, 1 << 14, "block", seed=7)
    for g in grads.values():
        g.mul_(65536.0)
    host = {k: v.cpu().numpy().copy() for k, v in grads.items()}
    ex = GradientBucketExecutor(plan, 0, descs, bindings, FakeRegistry(), lambda p, h: None)
    stats = GradientStatistics(ex.n_partials, cuda)
    ex.bind_statistics(stats)
    inv = 2.0**-16
    ex.set_inv_loss_scale(inv)
    ex.execute(1.0)
    stats.finalize(1.0)
    torch.cuda.synchronize()
    og.execute(plan, 0, {d.logical_param_id: d for d in descs}, host, 1.0)
    ref = [host[lid] for lid in grads]
    found = og.unscale_and_check(ref, inv)
    assert stats.found_inf.item() == float(found) == 0.0
    for lid, r in zip(grads, ref):
        np.testing.assert_array_equal(grads[lid].cpu().numpy(), r)
    norm = og.l2_norm(ref)
    assert stats.stats[1].item() == pytest.approx(norm, rel=1e-6)
    assert stats.stats[2].item() == pytest.approx(og.clip_coefficient(norm, 1.0), rel=1e-6)

    # 0.1% of one tensor forced to +inf -> flag raised
    victim = next(iter(grads.values()))
    idx = torch.randperm(victim.numel(), generator=torch.Generator().manual_seed(3))[: max(1, victim.numel() // 1000)]
    victim.view(-1)[idx.to(cuda)] = float("inf")
    ex.execute(1.0)
    torch.cuda.synchronize()
    assert stats.found_inf.item() == 1.0


def test_strided_tp_segments_vs_oracle(cuda):
    """Row-parallel style fragments: column halves of a [6, 8] tensor
    (narrow on dim 1) -> strided chunks."""
    announce("grad_sync strided dim-1 segments")
    group = ProcessGroupSpec("pg", (0,), "gradient_sync")
    frags = (named_fragment("lo", "w", "pg", 24, 0), named_fragment("hi", "w", "pg", 24, 1))
    bindings = (
        LocalFragmentBindingSpec(0, "lo", "w", (TensorSegmentSpec(0, 4, (6, 8), 0, 4, 24),), 1.0),
        LocalFragmentBindingSpec(0, "hi", "w", (TensorSegmentSpec(4, 4, (6, 8), 4, 8, 24),), 0.5),
    )
    plan = bp.build_gradient_sync_plan(CanonicalFragmentPlan((group,), frags, ((0, bindings),), "h"), "block", 1 << 20, "gpt", "m", "t")
    g = torch.randn(6, 8, generator=torch.Generator().manual_seed(5)).to(cuda)
    host = {"w": g.cpu().numpy().copy()}
    packed = []
    ex = GradientBucketExecutor(
        plan, 0, (Desc("w", 1),), (runtime_binding("w", g),), FakeRegistry(), lambda p, h: packed.append(p.cpu().numpy().copy())
    )
    ex.execute(2.0)
    torch.cuda.synchronize()
    ref = og.execute(plan, 0, {"w": Desc("w", 1)}, host, 2.0)
    np.testing.assert_array_equal(packed[0], ref[0])
    np.testing.assert_array_equal(g.cpu().numpy(), host["w"])


@pytest.mark.parametrize("scale", [0.3701, 1.0])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_local_pass_matches_the_per_bucket_calls(cuda, dtype, scale):
    """eth_bucket_sync_local (the identity seam, one native call for the
    pass; each bucket staged in one of two halves, one launch unpacking a
    bucket while it packs the next) against run_bucket's two launches per
    bucket through a seam that is not the identity object: main grads, the
    whole scratch buffer, found_inf and every L2 partial bit for bit, with
    and without a normalization scale, an unscale (fp32 only) and an inf
    planted on the second call."""
    announce(f"grad_sync local pass vs per-bucket calls, {dtype}, scale {scale}")
    setups = [_gpt_setup(cuda, 64, 256, 3, 1 << 13, "block", seed=21, dtype=dtype) for _ in range(2)]
    exs, sts = [], []
    for seam, (plan, descs, grads, bindings) in zip((local_all_reduce_sum, lambda p, h: None), setups):
        for g in grads.values():
            g.mul_(4096.0)
        ex = GradientBucketExecutor(plan, 0, descs, bindings, FakeRegistry(), seam)
        st = GradientStatistics(ex.n_partials, cuda)
        ex.bind_statistics(st)
        if dtype == torch.float32:
            ex.set_inv_loss_scale(2.0**-12)
        exs.append(ex)
        sts.append(st)
    assert exs[0].n_buckets > 4
    for call in range(2):
        if call == 1:
            for _, _, grads, _ in setups:
                next(iter(grads.values())).view(-1)[17] = float("inf")
        for ex in exs:
            ex.execute(scale)
        torch.cuda.synchronize()
        for a, b in zip(setups[0][2].values(), setups[1][2].values()):
            assert torch.equal(a.view(torch.int16 if dtype != torch.float32 else torch.int32),
                               b.view(torch.int16 if dtype != torch.float32 else torch.int32))
        name = exs[0].scratch_dtypes[0]
        assert torch.equal(exs[0].scratch(name), exs[1].scratch(name))
        assert sts[0].found_inf.item() == sts[1].found_inf.item() == float(call)
        assert torch.equal(sts[0].partials, sts[1].partials)


def test_local_pass_rejects_a_bad_entry_before_launching(cuda):
    """A bad bucket entry (unsupported dtype) raises before any launch, so
    the payload is left untouched."""
    import ctypes

    from eth_amd import _native as nat

    announce("grad_sync local pass bad entry")
    plan, descs, grads, bindings = _gpt_setup(cuda, 64, 256, 1, 1 << 13, "block", seed=5)
    ex = GradientBucketExecutor(plan, 0, descs, bindings, FakeRegistry(), local_all_reduce_sum)
    name = ex.scratch_dtypes[0]
    ex.scratch(name).fill_(-7.0)
    entries = ex._local_pass.copy()
    entries[-1]["dtype"] = 9
    with pytest.raises(ValueError, match="unsupported dtype"):
        nat.call("eth_bucket_sync_local", ctypes.c_void_p(entries.ctypes.data), len(entries), 1.0, 1.0, 0,
                 None, None, nat.ptr(ex._staging), ex._staging_half, nat.stream_ptr(cuda))
    torch.cuda.synchronize()
    assert bool((ex.scratch(name) == -7.0).all())


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 7, 8, 1023, 1024 * 4 + 3, 1 << 20, (1 << 20) + 5])
def test_fill_every_alignment_and_length(cuda, n):
    """eth_fill_f32 writes exactly [0, n) at each 4-byte offset from a 16-byte
    boundary (a scalar head, 16-byte stores, a scalar tail) and nothing either
    side of it."""
    from eth_amd import _native as nat

    for off in range(4):
        announce(f"fill n={n} offset={off}")
        buf = torch.full((n + 16,), -1.0, dtype=torch.float32, device=cuda)
        view = buf[off:off + n]
        nat.call("eth_fill_f32", nat.ptr(view), n, 2.5, nat.stream_ptr(cuda))
        host = buf.cpu()
        assert torch.all(host[off:off + n] == 2.5)
        assert torch.all(host[:off] == -1.0) and torch.all(host[off + n:] == -1.0)
