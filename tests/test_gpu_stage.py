"""GPU parity of one middle pipeline stage (whole transformer layers):
forward output, input gradient and every parameter's main_grad against the
fp32 CPU oracle on the same bf16 weights and inputs, then one full training
step (grad sync + clip + AdamW) against the oracle's AdamW on the GPU's own
gradients.

Bar: loss-side quantities and per-tensor gradient
norms within 2e-2 relative for bf16/fp16."""

import math

import numpy as np
import pytest
import torch

from eth_amd.model.flex_ops import GPTConfig
from eth_amd.stage import MiddleStageTrainer
from oracle import adamw as oadam
from oracle import gradsync as og
from oracle import layer as ol
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return (a - b).norm().item() / (b.norm().item() + 1e-30)


def _stage_parity(cuda, dtype, hidden, heads, ffn, layers, seq, mb, seed):
    cfg = GPTConfig(hidden_size=hidden, num_attention_heads=heads, ffn_hidden_size=ffn, num_layers=layers,
                    seq_length=seq, micro_batch_size=mb, params_dtype=dtype, device="cuda", seed=seed)
    tr = MiddleStageTrainer(cfg, lr=1e-4, weight_decay=0.1, clip_grad=1.0)
    gen = torch.Generator().manual_seed(77)
    x = torch.randn(seq, mb, hidden, generator=gen).to(dtype)
    dy = (torch.randn(seq, mb, hidden, generator=gen) * 1e-2).to(dtype)
    params = tr.layer_parameters()
    # give biases / LN params non-trivial values so their paths are exercised
    with torch.no_grad():
        for layer in params:
            for k, p in layer.items():
                if k.endswith("_b"):
                    p.copy_((torch.randn(p.shape, generator=gen) * 0.02).to(dtype))
                elif k.startswith("ln"):
                    p.copy_((1 + torch.randn(p.shape, generator=gen) * 0.05).to(dtype))
        tr.optimizer.reload_model_params()
    host = [{k: p.detach().float().cpu() for k, p in layer.items()} for layer in params]
    tr.ddp.zero_grad_buffer()
    out, dx = tr.forward_backward(x.to(cuda), dy.to(cuda))
    torch.cuda.synchronize()
    ref_out, ref_dx, ref_grads = ol.middle_stage_fwd_bwd(x.float(), host, heads, dy.float())
    assert _rel(out, ref_out) < 2e-2
    assert _rel(dx, ref_dx) < 2e-2
    for li, (layer, ref) in enumerate(zip(params, ref_grads)):
        for k, p in layer.items():
            g = p.main_grad
            assert p.grad is None
            gn, rn = g.double().norm().item(), ref[k].double().norm().item()
            assert abs(gn - rn) <= 2e-2 * rn + 1e-12, f"layer {li} {k}: |g| {gn} vs {rn}"
            assert _rel(g, ref[k]) < 5e-2, f"layer {li} {k}: rel err {_rel(g, ref[k])}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_middle_stage_matches_fp32_oracle(cuda, dtype):
    announce(f"middle stage parity {dtype}")
    _stage_parity(cuda, dtype, hidden=256, heads=4, ffn=1024, layers=2, seq=128, mb=2, seed=5)


def test_middle_stage_with_head_dim_80_and_a_ragged_sequence(cuda):
    """The head width of the reference's "2_6B" profiler model (hidden 2560,
    32 heads: 80, eth/profiler/model_configs.py:19) at a sequence that is not
    a multiple of the attention block, on a narrower stage (4 heads of 80)."""
    announce("middle stage parity, head_dim 80, seq 200")
    _stage_parity(cuda, torch.bfloat16, hidden=320, heads=4, ffn=1280, layers=1, seq=200, mb=2, seed=6)


def test_middle_stage_layer_at_bench_shape_matches_fp32_oracle(cuda):
    """One layer at the benchmarked shape (hidden 2048, 16 heads of 128,
    FFN 8192, seq 2048, micro-batch 4, bf16): the widths that select the
    production GEMM tiles, the 128-wide attention kernels and the
    1025-2048-column LayerNorm backward."""
    announce("middle stage parity at the bench shape (1 layer, 8192 tokens)")
    _stage_parity(cuda, torch.bfloat16, hidden=2048, heads=16, ffn=8192, layers=1, seq=2048, mb=4, seed=5)


def test_deferred_zero_matches_eager_zero(cuda):
    """zero_grad_buffer(defer=True) over a buffer full of garbage, then two
    micro-batches (the first gradient into each main_grad stores, the
    second adds) and settle: every main_grad equals zero-then-accumulate of
    the same two micro-batches bit for bit."""
    announce("deferred main-grad zero vs eager zero")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2,
                    seq_length=128, micro_batch_size=2, params_dtype=torch.bfloat16, device="cuda", seed=21)
    tr = MiddleStageTrainer(cfg, lr=1e-4, weight_decay=0.1, clip_grad=1.0)
    gen = torch.Generator().manual_seed(8)
    xs = [torch.randn(128, 2, 256, generator=gen).to(torch.bfloat16).to(cuda) for _ in range(2)]
    dys = [(torch.randn(128, 2, 256, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda) for _ in range(2)]
    (buf,) = tr.ddp.grad_buffers.values()
    tr.ddp.zero_grad_buffer()
    for x, dy in zip(xs, dys):
        tr.forward_backward(x, dy)
    eager = buf.data.clone()
    buf.data.fill_(123.0)
    tr.ddp.zero_grad_buffer(defer=True)
    for x, dy in zip(xs, dys):
        tr.forward_backward(x, dy)
    tr.ddp.settle_grad_buffer()
    torch.cuda.synchronize()
    assert torch.equal(buf.data, eager)
    # a parameter no kernel wrote is zero-filled by settle
    buf.data.fill_(5.0)
    tr.ddp.zero_grad_buffer(defer=True)
    tr.ddp.settle_grad_buffer()
    assert torch.count_nonzero(buf.data).item() == 0


def test_overlapped_weight_gradients_match_single_stream(cuda):
    """forward_backward runs the weight-gradient GEMMs on a side stream
    (joined before it returns); the buffer equals a plain single-stream
    backward of the same micro-batch bit for bit."""
    announce("side-stream weight gradients vs single stream")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2,
                    seq_length=128, micro_batch_size=2, params_dtype=torch.bfloat16, device="cuda", seed=33)
    tr = MiddleStageTrainer(cfg, lr=1e-4, weight_decay=0.1, clip_grad=1.0)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(128, 2, 256, generator=gen).to(torch.bfloat16).to(cuda)
    dy = (torch.randn(128, 2, 256, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda)
    (buf,) = tr.ddp.grad_buffers.values()
    tr.ddp.zero_grad_buffer()
    xi = x.detach().requires_grad_(True)
    tr.model.set_input_tensor({"hidden_states": xi})
    out, _ = tr.model(None, {})
    torch.autograd.backward(out["hidden_states"], dy)
    single = buf.data.clone()
    tr.ddp.zero_grad_buffer()
    _, dx = tr.forward_backward(x, dy)
    overlapped = buf.data.clone()
    torch.cuda.synchronize()
    assert torch.equal(overlapped, single)
    assert torch.equal(dx, xi.grad)


def _check_step_against_oracle(tr, x, dy, masters_before, step, lr, clip):
    """After tr.train_step: the main grads the step used (the synced,
    unscaled gradients the unpack wrote back) against the fp32 layer oracle
    on the pre-step weights, and the fp32 masters against the oracle's
    L2 norm / clip / AdamW chain applied to those gradients (1e-6)."""
    layers = tr.layer_parameters()
    # the model's 16-bit weights before the step are the bf16 rounding of the masters
    host = [{k: torch.from_numpy(oadam.to_bf16(masters_before[li][k])) for k in layer} for li, layer in enumerate(layers)]
    _, _, ref_grads = ol.middle_stage_fwd_bwd(x.float().cpu(), host, 4, dy.float().cpu())
    grads = [{k: p.main_grad.detach().cpu().numpy().copy() for k, p in layer.items()} for layer in layers]
    for li, layer in enumerate(grads):
        for k, g in layer.items():
            assert _rel(torch.from_numpy(g), ref_grads[li][k]) < 5e-2, (li, k)
    ref_norm = og.l2_norm([g for layer in grads for g in layer.values()])
    coef = og.clip_coefficient(ref_norm, clip)
    for li, layer in enumerate(layers):
        for k, p in layer.items():
            wd = 0.1 if k.endswith("_w") and not k.startswith("ln") else 0.0
            m_prev, v_prev = masters_before[li][k + ".m"], masters_before[li][k + ".v"]
            ref_p, _, _ = oadam.adamw_step(masters_before[li][k], grads[li][k], m_prev, v_prev, step, lr, 0.9, 0.95,
                                           1e-8, wd, clip_coef=coef)
            got = tr.optimizer.optimizer_parameter_for_model_parameter(p).detach().cpu().numpy()
            np.testing.assert_allclose(got, ref_p, rtol=1e-6, atol=1e-9, err_msg=f"layer {li} {k}")
    return ref_norm


def _optimizer_snapshot(tr):
    """fp32 masters and AdamW moments per layer and oracle name (numpy)."""
    snap = []
    for layer in tr.layer_parameters():
        d = {}
        for k, p in layer.items():
            d[k] = tr.optimizer.optimizer_parameter_for_model_parameter(p).detach().cpu().numpy().copy()
            st = tr.optimizer.state_for_model_parameter(p)
            d[k + ".m"] = st["exp_avg"].detach().cpu().numpy().copy() if "exp_avg" in st else np.zeros_like(d[k])
            d[k + ".v"] = st["exp_avg_sq"].detach().cpu().numpy().copy() if "exp_avg_sq" in st else np.zeros_like(d[k])
        snap.append(d)
    return snap


def test_streamed_grad_sync_matches_sync_after_backward(cuda):
    """Two identical stages, two steps each: buckets synced during the
    backward (streamed, the default) and the whole sync after it (the
    reference order) give bit-identical norms, master weights and bf16
    weights; and each streamed step matches the oracle chain: its gradients
    the fp32 layer oracle, its norm, clip and AdamW update the grad-sync and
    AdamW oracles applied to those gradients."""
    announce("streamed grad sync vs sync after backward")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2,
                    seq_length=128, micro_batch_size=2, params_dtype=torch.bfloat16, device="cuda", seed=41)
    trs = [MiddleStageTrainer(cfg, lr=1e-3, weight_decay=0.1, clip_grad=0.5, bucket_cap_bytes=1 << 19) for _ in range(2)]
    assert trs[0].grad_sync.executor.n_buckets > 4
    gen = torch.Generator().manual_seed(6)
    batches = [(torch.randn(128, 2, 256, generator=gen).to(torch.bfloat16).to(cuda),
                (torch.randn(128, 2, 256, generator=gen) * 1e-1).to(torch.bfloat16).to(cuda)) for _ in range(2)]
    norms = [[], []]
    for step, (x, dy) in enumerate(batches, start=1):
        before = _optimizer_snapshot(trs[0])
        for i, tr in enumerate(trs):
            _, _, ok, norm = tr.train_step(x, dy, streamed_sync=(i == 0))
            assert ok
            norms[i].append(norm)
        torch.cuda.synchronize()
        ref_norm = _check_step_against_oracle(trs[0], x, dy, before, step, 1e-3, 0.5)
        assert norms[0][-1] == pytest.approx(ref_norm, rel=1e-6)
    assert norms[0] == norms[1]
    for pa, pb in zip(trs[0].model.parameters(), trs[1].model.parameters()):
        assert torch.equal(pa, pb)
        ma = trs[0].optimizer.optimizer_parameter_for_model_parameter(pa)
        mb = trs[1].optimizer.optimizer_parameter_for_model_parameter(pb)
        assert torch.equal(ma, mb)


def test_middle_stage_training_step(cuda):
    """zero -> fwd/bwd -> grad sync (fused stats) -> clip -> AdamW -> bf16
    copy; the update must equal the oracle AdamW applied to the GPU's own
    gradients with the oracle's clip coefficient (1e-6 relative)."""
    announce("middle stage training step")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=1,
                    seq_length=128, micro_batch_size=2, params_dtype=torch.bfloat16, device="cuda", seed=9)
    tr = MiddleStageTrainer(cfg, lr=1e-3, weight_decay=0.1, clip_grad=0.05, bucket_cap_bytes=1 << 18)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(128, 2, 256, generator=gen).to(torch.bfloat16).to(cuda)
    dy = (torch.randn(128, 2, 256, generator=gen) * 1e-1).to(torch.bfloat16).to(cuda)
    layer = tr.layer_parameters()[0]
    masters = {k: tr.optimizer.optimizer_parameter_for_model_parameter(p).detach().cpu().numpy().copy() for k, p in layer.items()}
    tr.ddp.zero_grad_buffer()
    tr.forward_backward(x, dy)
    grads = {k: p.main_grad.detach().cpu().numpy().copy() for k, p in layer.items()}
    tr.grad_sync.execute(1.0)
    ok, norm, _ = tr.optimizer.step()
    torch.cuda.synchronize()
    assert ok
    ref_norm = og.l2_norm(list(grads.values()))
    assert norm == pytest.approx(ref_norm, rel=1e-6)
    coef = og.clip_coefficient(ref_norm, 0.05)
    assert coef < 1.0
    for k, p in layer.items():
        wd = 0.1 if k.endswith("_w") and not k.startswith("ln") else 0.0
        ref_p, _, _ = oadam.adamw_step(masters[k], grads[k], np.zeros_like(grads[k]), np.zeros_like(grads[k]), 1,
                                       1e-3, 0.9, 0.95, 1e-8, wd, clip_coef=coef)
        got = tr.optimizer.optimizer_parameter_for_model_parameter(p).detach().cpu().numpy()
        np.testing.assert_allclose(got, ref_p, rtol=1e-6, atol=1e-9)
        np.testing.assert_array_equal(p.detach().float().cpu().numpy(), oadam.to_bf16(got))


@pytest.mark.parametrize("dropout", [0.0, 0.1])
def test_fused_dropout_layernorm_pairs_match_the_separate_ops(cuda, dropout):
    """Each bias-dropout-add followed in the stage by a LayerNorm runs as one
    kernel (BiasDropoutAddLayerNormFn) whose LayerNorm result the next op
    takes over.  With the pairs undone the stage gives the same output, input
    gradient and main grads bit for bit, with and without dropout (same mask
    from the same per-call seed)."""
    from eth_amd.model.flex_ops import ParallelDropoutOp

    announce(f"fused dropout+LayerNorm pairs vs separate ops, p={dropout}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2,
                    seq_length=128, micro_batch_size=2, params_dtype=torch.bfloat16, device="cuda", seed=51,
                    hidden_dropout=dropout)
    tr = MiddleStageTrainer(cfg, lr=1e-4, weight_decay=0.1, clip_grad=1.0)
    ops = list(tr.model.language_model.ops)
    drops = [op for op in ops if isinstance(op, ParallelDropoutOp)]
    paired = {id(op): op.fused_layernorm_op for op in drops}
    # post-attention -> 2nd LN in both layers, post-MLP of layer 0 -> layer 1's 1st LN; the last
    # dropout ends the stage
    assert sum(v is not None for v in paired.values()) == 3 and drops[-1].fused_layernorm_op is None
    # the LayerNorm stays registered once: no parameter reached through the pairing
    names = [n for n, _ in tr.model.named_parameters()]
    assert not any("fused_layernorm_op" in n for n in names)
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(128, 2, 256, generator=gen).to(torch.bfloat16).to(cuda)
    dy = (torch.randn(128, 2, 256, generator=gen) * 1e-2).to(torch.bfloat16).to(cuda)
    (buf,) = tr.ddp.grad_buffers.values()
    calls = {id(op): op._calls for op in drops}

    def run():
        for op in drops:
            op._calls = calls[id(op)]
        tr.ddp.zero_grad_buffer()
        out, dx = tr.forward_backward(x, dy)
        torch.cuda.synchronize()
        return out.clone(), dx.clone(), buf.data.clone()

    fused = run()
    for op in drops:
        object.__setattr__(op, "fused_layernorm_op", None)
    separate = run()
    for op in drops:
        object.__setattr__(op, "fused_layernorm_op", paired[id(op)])
    for a, b in zip(fused, separate):
        assert torch.equal(a, b)
