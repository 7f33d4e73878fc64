"""GPU property tests of the grad-sync and AdamW legs at the size BASELINE
configs[2] and [3] state: the 24-layer hidden-2048 GPT gradient list
(1,208,598,528 fp32 elements, eth/runtime/megatron/grad_sync/gpt_adapter.py
schema) in 32 MiB block buckets (bucket_plan.py:155-241).  At this size the
oracle cannot replay everything, so the checks are size-independent
properties: the bucket count of the plan, the overflow flag with and without
the 0.1 % +inf set, the unscale by the exact power of two 2^-16 against
torch's own multiply on the GPU, the L2 norm against a float64 reduction,
and three clipped AdamW steps with sampled slices against the oracle."""

import math

import numpy as np
import pytest
import torch

from eth_amd.grad_sync import bucket_plan as bp
from eth_amd.grad_sync.executor import GradientBucketExecutor, GradientStatistics
from eth_amd.grad_sync.planner import plan_canonical_fragments
from eth_amd.grad_sync.synthetic import descriptors_for, gpt_layer_shapes
from eth_amd.optimizer.grad_scaler import ConstantGradScaler
from eth_amd.optimizer.optimizer import Float16OptimizerWithFloat16Params
from oracle import adamw as oadam
from oracle import gradsync as og
from tests.conftest import announce
from tests.helpers import FakeRegistry, runtime_binding

pytestmark = pytest.mark.gpu

H, FFN, LAYERS = 2048, 8192, 24
N_ELEMENTS = 1_208_598_528
CAP = 32 << 20
SCALE = 2.0**16


def _layout(cuda):
    """The tensor list, its plan, and main grads as views of one fp32 buffer
    carved from the end (model/distributed.py:93-105)."""
    shapes = gpt_layer_shapes(H, FFN, LAYERS)
    total = sum(math.prod(s[1]) for s in shapes)
    assert total == N_ELEMENTS
    descs = descriptors_for(shapes)
    plan = bp.build_gradient_sync_plan(plan_canonical_fragments(descs, (0,)), "block", CAP, "gpt", "m", "t")
    buf = torch.empty(total, dtype=torch.float32, device=cuda)
    grads, off = {}, total
    for lid, shape, *_ in shapes:
        n = math.prod(shape)
        off -= n
        grads[lid] = buf[off : off + n].view(shape)
    return shapes, descs, plan, buf, grads


def _sum_sq_f64(buf, chunk=1 << 27):
    """Sum of squares in float64, a chunk at a time (bounded temporaries)."""
    total = 0.0
    for i in range(0, buf.numel(), chunk):
        total += float(buf[i : i + chunk].double().square().sum().item())
    return total


def test_grad_sync_at_configs_2_size(cuda):
    announce("grad sync at full C3 size (1.2 G fp32, 32 MiB buckets)")
    shapes, descs, plan, buf, grads = _layout(cuda)
    assert len(plan.global_bucket_order) == 121
    ex = GradientBucketExecutor(plan, 0, descs, [runtime_binding(l, grads[l]) for l, *_ in shapes], FakeRegistry(),
                                lambda payload, handle: None)
    st = GradientStatistics(ex.n_partials, cuda)
    ex.bind_statistics(st)
    ex.set_inv_loss_scale(2.0**-16)
    g = torch.Generator(device=cuda).manual_seed(1234)
    buf.normal_(0, 1e-3, generator=g).mul_(SCALE)  # loss-scaled gradients (x 2^16 is exact)
    expect = buf * 2.0**-16  # torch's own multiply by the exact power of two
    ex.execute(1.0)
    st.finalize(1.0)
    torch.cuda.synchronize()
    assert st.found_inf.item() == 0.0
    assert torch.equal(buf, expect)
    ref_sq = _sum_sq_f64(expect)
    norm = float(st.stats[1].item())
    assert norm == pytest.approx(math.sqrt(ref_sq), rel=1e-6)
    assert float(st.stats[2].item()) == pytest.approx(og.clip_coefficient(math.sqrt(ref_sq), 1.0), rel=1e-6)
    # the overflow variant: 0.1 % of the elements +inf (a seeded index set)
    buf.copy_(expect).mul_(SCALE)
    del expect
    idx = torch.randint(0, N_ELEMENTS, (N_ELEMENTS // 1000,), generator=g, device=cuda)
    buf[idx] = float("inf")
    ex.execute(1.0)
    torch.cuda.synchronize()
    assert st.found_inf.item() == 1.0
    # the finite elements are still unscaled bit for bit; the +inf stay +inf
    assert bool(torch.isinf(buf[idx]).all())
    del idx, ex, st, buf, grads
    torch.cuda.empty_cache()


def test_adamw_at_configs_3_size(cuda):
    """Three steps of the Megatron bf16 optimizer over the full list:
    grad sync with the fused unscale (2^-16) / flag / L2, clip at 1.0 (active:
    the norm is ~35), AdamW lr 1e-4, betas .9/.95, eps 1e-8, wd 0.1 on the 96
    weight matrices and 0 on the 192 LayerNorm / bias tensors, bf16 model
    copies.  Every step applies with a finite norm matching a float64
    reduction; the fp32 masters stay finite; slices of four tensors equal
    the oracle's AdamW chain bit for bit, and their bf16 copies its
    rounding."""
    announce("AdamW at full C4 size, 3 clipped steps")
    shapes, descs, plan, buf, grads = _layout(cuda)
    g = torch.Generator(device=cuda).manual_seed(99)
    params = {}
    for lid, shape, *_ in shapes:
        p = torch.nn.Parameter(torch.empty(shape, device=cuda).normal_(0, 0.02, generator=g).to(torch.bfloat16))
        p.main_grad = grads[lid]
        params[lid] = p
    wd_ids = [l for l, s, *_ in shapes if len(s) == 2]
    rest = [l for l, *_ in shapes if l not in wd_ids]
    assert (len(wd_ids), len(rest)) == (96, 192)
    ex = GradientBucketExecutor(plan, 0, descs, [runtime_binding(l, grads[l]) for l, *_ in shapes], FakeRegistry(),
                                lambda payload, handle: None)
    opt = Float16OptimizerWithFloat16Params(
        [{"params": [params[l] for l in wd_ids]}, {"params": [params[l] for l in rest], "weight_decay": 0.0}],
        1e-4, (0.9, 0.95), 1e-8, 0.1, clip_grad=1.0, bf16=True, grad_scaler=ConstantGradScaler(SCALE))
    opt.bind_gradient_sync(ex)
    # sampled slices: the first layer's QKV weight, the last layer's fc2
    # weight, a LayerNorm bias and an fc1 bias
    samples = {
        "gpt.layers.0.attention.query_key_value.weight": slice(1_000_000, 2_000_000),
        "gpt.layers.23.mlp.dense_4h_to_h.weight": slice(0, 1_000_000),
        "gpt.layers.11.mlp.input_layernorm.bias": slice(0, H),
        "gpt.layers.5.mlp.dense_h_to_4h.bias": slice(0, FFN),
    }
    host = {l: params[l].detach().float().reshape(-1)[s].cpu().numpy() for l, s in samples.items()}
    m = {l: np.zeros_like(v) for l, v in host.items()}
    v_ = {l: np.zeros_like(v) for l, v in host.items()}
    for step in range(1, 4):
        buf.normal_(0, 1e-3, generator=g).mul_(SCALE)
        raw = {l: grads[l].reshape(-1)[s].cpu().numpy() for l, s in samples.items()}
        ex.execute(1.0)
        ok, norm, _ = opt.step()
        torch.cuda.synchronize()
        assert ok and norm is not None and np.isfinite(norm)
        # the main grads now hold the unscaled gradients the step used
        ref_norm = math.sqrt(_sum_sq_f64(buf))
        assert norm == pytest.approx(ref_norm, rel=1e-6)
        coef = float(opt._statistics.stats[2].item())
        assert coef < 0.1 and coef == pytest.approx(og.clip_coefficient(ref_norm, 1.0), rel=1e-6)
        for l in samples:
            gs = raw[l] * np.float32(2.0**-16)
            wd = 0.1 if l in wd_ids else 0.0
            host[l], m[l], v_[l] = oadam.adamw_step(host[l], gs, m[l], v_[l], step, 1e-4, 0.9, 0.95, 1e-8, wd,
                                                    clip_coef=coef)
    for l, s in samples.items():
        master = opt.optimizer_parameter_for_model_parameter(params[l]).detach().reshape(-1)[s].cpu().numpy()
        np.testing.assert_array_equal(master, host[l], err_msg=l)
        np.testing.assert_array_equal(params[l].detach().float().reshape(-1)[s].cpu().numpy(), oadam.to_bf16(host[l]))
    for l, p in params.items():
        assert bool(torch.isfinite(opt.optimizer_parameter_for_model_parameter(p)).all()), l
    del opt, ex, params, buf, grads
    torch.cuda.empty_cache()
