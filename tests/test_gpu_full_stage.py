"""GPU parity of the first+last stage (embedding, layers, final LN, tied LM
head, vocab cross entropy, loss contract, tied-gradient sum) against the fp64
CPU oracle on BASELINE configs[0] shapes (h 256, 2 layers, 4 heads, FFN 1024,
seq 128, micro-batch 2, vocab 50257 padded to 50304, labels = 0 as the
reference's post-process builds them), and the vocabulary kernels alone."""

import numpy as np
import pytest
import torch

from eth_amd import kernels as K
from eth_amd.loss import synthetic_gpt_batch
from eth_amd.model.flex_ops import GPTConfig
from eth_amd.stage import FirstLastStageTrainer
from oracle import layer as ol
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return (a - b).norm().item() / (b.norm().item() + 1e-30)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_cross_entropy_and_embedding_kernels(cuda, dtype):
    announce(f"vocab kernels {dtype}")
    gen = torch.Generator().manual_seed(0)
    rows, V = 96, 50304
    z = (torch.randn(rows, V, generator=gen) * 3).to(dtype)
    lab = torch.randint(0, V, (rows,), generator=gen)
    bad = torch.zeros(1, dtype=torch.int32, device=cuda)
    loss, lse = K.xent_fwd(z.to(cuda), lab.to(cuda), bad)
    zr = z.double().requires_grad_(True)
    ref = ol.vocab_cross_entropy(zr, lab).double()
    assert torch.allclose(loss.cpu().double(), ref, rtol=1e-4, atol=1e-4)
    g = torch.rand(rows, generator=gen)
    ref.backward(g.double())
    dz = K.xent_bwd(z.to(cuda), lab.to(cuda), lse, g.to(cuda))
    tol = 2**-7 if dtype == torch.bfloat16 else 2**-10
    assert (dz.cpu().double() - zr.grad).abs().max().item() <= tol * zr.grad.abs().max().item()
    assert bad.item() == 0
    # embedding
    b, s, h = 2, 16, 64
    word = (torch.randn(V, h, generator=gen) * 0.02).to(dtype)
    pos = (torch.randn(s, h, generator=gen) * 0.02).to(dtype)
    tok = torch.randint(0, V, (b, s), generator=gen)
    tok[0, 1] = tok[1, 3]  # a repeated token accumulates twice
    pid = torch.arange(s).expand(b, s).contiguous()
    out = K.embedding_fwd(tok.to(cuda), pid.to(cuda), word.to(cuda), pos.to(cuda), bad)
    ref = (word[tok] + pos[pid]).transpose(0, 1)  # same dtype: one rounded add
    assert torch.equal(out.cpu(), ref)
    dout = torch.randn(s, b, h, generator=gen).to(dtype)
    dw = torch.zeros(V, h, device=cuda)
    dp = torch.zeros(s, h, device=cuda)
    K.embedding_bwd(tok.to(cuda), pid.to(cuda), dout.to(cuda), dw, dp)
    ref_w = torch.zeros(V, h, dtype=torch.float64).index_add_(0, tok.reshape(-1), dout.transpose(0, 1).reshape(-1, h).double())
    ref_p = torch.zeros(s, h, dtype=torch.float64).index_add_(0, pid.reshape(-1), dout.transpose(0, 1).reshape(-1, h).double())
    assert torch.allclose(dw.cpu().double(), ref_w, atol=1e-5)
    assert torch.allclose(dp.cpu().double(), ref_p, atol=1e-5)
    # out-of-range ids are flagged, never read out of bounds
    tok[0, 0] = V + 5
    K.embedding_fwd(tok.to(cuda), pid.to(cuda), word.to(cuda), pos.to(cuda), bad)
    assert bad.item() == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_first_last_stage_matches_fp64_oracle(cuda, dtype):
    announce(f"first+last stage parity {dtype}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=11)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                               initial_loss_scale=1024.0)
    ops = tr.model.language_model.ops
    layers = tr_layer_params(tr)
    params = {
        "word": tr.embedding.word_embeddings.weight.detach().float().cpu(),
        "pos": tr.embedding.position_embeddings.weight.detach().float().cpu(),
        "lnf_w": ops[-2].input_layernorm.weight.detach().float().cpu(),
        "lnf_b": ops[-2].input_layernorm.bias.detach().float().cpu(),
        "layers": [{k: p.detach().float().cpu() for k, p in lp.items()} for lp in layers],
    }
    sample_ids = [3, 8]
    tr.ddp.zero_grad_buffer()
    losses, lo = tr.forward_backward(sample_ids)
    from eth_amd.loss import global_normalization_scale
    tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
    tr.tie_gradients()
    torch.cuda.synchronize()
    tokens, mask, positions, _ = synthetic_gpt_batch(sample_ids, 128, 50257, "cpu")
    ref_losses, ref_mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, 4)
    assert _rel(losses, ref_losses) < 2e-2
    scale = tr.optimizer.get_loss_scale().item()
    # main grads hold d(sum(loss*mask)/sum(mask)) * loss_scale after the sync
    checks = [(tr.embedding.word_embeddings.weight, grads["word"]), (tr.embedding.position_embeddings.weight, grads["pos"]),
              (tr.post.word_embeddings.weight, grads["word"]), (ops[-2].input_layernorm.weight, grads["lnf_w"]),
              (ops[-2].input_layernorm.bias, grads["lnf_b"])]
    for lp, gl in zip(layers, grads["layers"]):
        for k, p in lp.items():
            checks.append((p, gl[k]))
    for p, ref in checks:
        g = p.main_grad.double().cpu() / scale
        rn = ref.norm().item()
        assert abs(g.norm().item() - rn) <= 2e-2 * rn + 1e-12, (p.shape, g.norm().item(), rn)
    ok, norm, _ = tr.optimizer.step()
    assert ok and norm is not None and np.isfinite(norm)
    # the tied copies stay identical after the update
    assert torch.equal(tr.embedding.word_embeddings.weight, tr.post.word_embeddings.weight)
    # deferred zeroing (what train_step uses) over a garbage buffer gives the
    # eager buffer bit for bit: embedding scatter-add, LM head and layers
    (buf,) = tr.ddp.grad_buffers.values()
    tr.ddp.zero_grad_buffer()
    tr.forward_backward(sample_ids)
    eager = buf.data.clone()
    buf.data.fill_(-7.0)
    tr.ddp.zero_grad_buffer(defer=True)
    tr.forward_backward(sample_ids)
    tr.ddp.settle_grad_buffer()
    torch.cuda.synchronize()
    assert torch.equal(buf.data, eager)


def tr_layer_params(tr):
    names = {
        "enc-1st-layernorm": (("input_layernorm.weight", "ln1_w"), ("input_layernorm.bias", "ln1_b")),
        "enc-attention-qkv": (("query_key_value.weight", "qkv_w"), ("query_key_value.bias", "qkv_b")),
        "enc-attention-dense": (("dense.weight", "proj_w"), ("dense.bias", "proj_b")),
        "enc-2nd-layernorm": (("input_layernorm.weight", "ln2_w"), ("input_layernorm.bias", "ln2_b")),
        "enc-MLP-GEMM-1": (("dense.weight", "fc1_w"), ("dense.bias", "fc1_b")),
        "enc-MLP-GEMM-2": (("dense.weight", "fc2_w"), ("dense.bias", "fc2_b")),
    }
    layers = {}
    for op in tr.model.language_model.ops:
        if op.name not in names:
            continue
        layer = layers.setdefault((op.op_index - 1) // 10, {})
        for path, key in names[op.name]:
            obj = op
            for part in path.split("."):
                obj = getattr(obj, part)
            layer[key] = obj
    return [layers[k] for k in sorted(layers)]
