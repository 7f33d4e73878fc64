"""GPU tests of the reference's default fp16 contract (training without
--accumulate-allreduce-grads-in-fp32): fp16 main grads that receive each
gradient rounded to fp16 and add it with a second rounding
(eth/runtime/megatron/model/distributed.py:69-123), fp16 bucket payloads,
and the optimizer's fp32 copy before unscaling (optimizer/optimizer.py:
388-461)."""

import hashlib
import json

import numpy as np
import pytest
import torch
from torch import nn

from eth_amd import kernels as K
from eth_amd.loss import global_normalization_scale
from eth_amd.model.distributed import DistributedDataParallel
from eth_amd.model.flex_ops import GPTConfig
from eth_amd.model.functional import LinearFn
from eth_amd.stage import FirstLastStageTrainer
from oracle import gradsync as og
from tests.conftest import announce

pytestmark = pytest.mark.gpu


class _Linear(nn.Module):
    def __init__(self, n_in, n_out, gen):
        super().__init__()
        self.weight = nn.Parameter((torch.randn(n_out, n_in, generator=gen) * 0.02).half().cuda())
        self.bias = nn.Parameter((torch.randn(n_out, generator=gen) * 0.02).half().cuda())

    def forward(self, x):
        return LinearFn.apply(x, self.weight, self.bias)


@pytest.mark.parametrize("defer", [False, True])
def test_linear_adds_the_rounded_gradient_into_fp16_main_grads(cuda, defer):
    """Two microbatches: main_grad == fp16(dW1 + dW2) where each dW_i is the
    fp32 product rounded once to fp16 (what the reference's fp16 autograd
    matmul returns as param.grad), bit for bit; the bias likewise from the
    fp32 column sums.  A deferred zero over a garbage buffer gives the same
    bits (the first contribution is stored)."""
    announce(f"fp16 main grads, linear, defer={defer}")
    gen = torch.Generator().manual_seed(3)
    lin = _Linear(256, 384, gen)
    ddp = DistributedDataParallel(lin, accumulate_allreduce_grads_in_fp32=False)
    assert lin.weight.main_grad.dtype == torch.float16
    xs = [(torch.randn(128, 256, generator=gen)).half().cuda() for _ in range(2)]
    dys = [(torch.randn(128, 384, generator=gen) * 1e-2).half().cuda() for _ in range(2)]
    if defer:
        for buf in ddp.grad_buffers.values():
            buf.data.fill_(-3.0)
        ddp.zero_grad_buffer(defer=True)
    else:
        ddp.zero_grad_buffer()
    for x, dy in zip(xs, dys):
        lin(x).backward(dy)
    ddp.settle_grad_buffer()
    torch.cuda.synchronize()
    dws, dbs = [], []
    for x, dy in zip(xs, dys):
        dws.append(K.gemm(dy.t(), x, out_dtype=torch.float16))
        acc = torch.empty(384, dtype=torch.float32, device=cuda)
        K.col_sum(dy, acc, accumulate=False)
        dbs.append(acc.half())
    want_w = (dws[0].float() + dws[1].float()).half()
    want_b = (dbs[0].float() + dbs[1].float()).half()
    assert torch.equal(lin.weight.main_grad, want_w)
    assert torch.equal(lin.bias.main_grad, want_b)
    assert lin.weight.grad is None and lin.bias.grad is None


def test_first_last_stage_in_the_reference_fp16_contract(cuda, tmp_path):
    """fp16 main grads end to end on the first+last stage: the buckets carry
    fp16, each packed payload is bit for bit the oracle's packing of the
    pre-sync fp16 main grads (SHA-256 of the runtime evidence), the synced
    gradients match the fp64 oracle, and the step (fp32 copy, unscale,
    clip, AdamW) applies with the tied copies kept equal."""
    from tests.test_gpu_full_stage import _check_first_last_gradients

    announce("first+last stage, fp16 main grads")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=torch.float16, device="cuda", seed=11)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                               initial_loss_scale=1024.0, accumulate_allreduce_grads_in_fp32=False,
                               runtime_evidence_dir=tmp_path)
    assert {b.grad_dtype for b in tr.grad_sync.plan.global_bucket_order} == {"torch.float16"}
    assert all(p.main_grad.dtype == torch.float16 for p in tr.model.parameters())
    # the packed bytes: one forward/backward, host copy of the fp16 main
    # grads, then the sync records the SHA-256 of every packed payload
    tr.ddp.zero_grad_buffer()
    _, lo = tr.forward_backward([3, 8])
    torch.cuda.synchronize()
    host = {b.logical_param_id: b.main_grad.detach().cpu().numpy().copy() for b in tr.bindings}
    assert all(g.dtype == np.float16 for g in host.values())
    tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
    torch.cuda.synchronize()
    descs = {d.logical_param_id: d for d in tr.descriptors}
    packed = og.execute(tr.grad_sync.plan, 0, descs, host)
    report = json.loads((tmp_path / "rank-00000.json").read_text())
    got = [b["packed_payload_sha256"] for b in report["iterations"][-1]["buckets"]]
    assert got == [hashlib.sha256(p.tobytes()).hexdigest() for p in packed]
    assert report["iterations"][-1]["payload_bytes"] == sum(p.nbytes for p in packed)
    # gradients against the fp64 oracle (same tolerances as the fp32-accumulate mode)
    _check_first_last_gradients(tr, [3, 8], 4)
    ok, norm, _ = tr.optimizer.step()
    assert ok and norm is not None and np.isfinite(norm)
    assert torch.equal(tr.embedding.word_embeddings.weight, tr.post.word_embeddings.weight)
    # a packaged step runs too, and the next one reuses the fp32 gradient buffer
    _, _, ok2, norm2 = tr.train_step([5, 9])
    assert ok2 and np.isfinite(norm2)


def test_fp16_main_grads_are_widened_unscaled_and_measured_in_one_pass(cuda):
    """The optimizer's fp32 copy of fp16 main grads (main_grad.float(),
    optimizer.py:392-397) is made by the statistics pass itself: after the
    step every master's grad is the fp16 main grad widened and multiplied by
    1/loss_scale, bit for bit as torch computes it; the norm is the oracle's
    L2 over the norm-owned grads (the tied head copy excluded); a +inf in an
    fp16 main grad skips the step."""
    announce("fp16 main grads: widening fused with unscale and statistics")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=torch.float16, device="cuda", seed=19)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                               initial_loss_scale=1024.0, accumulate_allreduce_grads_in_fp32=False)
    opt = tr.optimizer
    for attempt in ("finite", "overflow"):
        tr.ddp.zero_grad_buffer()
        _, lo = tr.forward_backward([3, 8])
        tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
        tr.tie_gradients()
        if attempt == "overflow":
            qkv = next(op for op in tr.model.language_model.ops if op.name == "enc-attention-qkv")
            qkv.query_key_value.weight.main_grad[1, 2] = float("inf")
        torch.cuda.synchronize()
        host = {name: p.main_grad.detach().cpu().clone() for name, p in tr.model.named_parameters()}
        ok, norm, _ = opt.step()
        torch.cuda.synchronize()
        if attempt == "overflow":
            assert (ok, norm) == (False, None)
            continue
        assert ok and norm is not None
        owned, seen = [], set()
        for name, p in tr.model.named_parameters():
            m = opt.optimizer_parameter_for_model_parameter(p)
            assert m.grad.dtype == torch.float32
            want = host[name].float() * torch.tensor(1.0 / 1024.0)
            assert torch.equal(m.grad.cpu(), want), name
            if id(m) not in seen and opt._norm_owned(m):
                owned.append(want.numpy())
            seen.add(id(m))
        # the tied head copy adds nothing to the norm: it shares the root's
        # master (and would not be norm-owned as a master of its own)
        assert len(owned) == len(host) - 1
        assert norm == pytest.approx(og.l2_norm(owned), rel=1e-6)
