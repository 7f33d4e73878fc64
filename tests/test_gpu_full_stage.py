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
def test_embedding_backward_is_deterministic_with_repeated_tokens(cuda, dtype):
    """Heavily repeated ids (most tokens from 6 values, so runs of ~600
    rows) into a non-zero fp32 main grad: bit-exact against the oracle's
    ordered fp32 sum, and the same bits on a second run."""
    announce(f"embedding backward determinism {dtype}")
    gen = torch.Generator().manual_seed(21)
    b, s, h, V = 4, 1024, 256, 50304
    tok = torch.randint(0, 6, (b, s), generator=gen)
    tok[:, ::7] = torch.randint(0, V, (b, (s + 6) // 7), generator=gen)
    pid = torch.arange(s).expand(b, s).contiguous()
    dout = torch.randn(s, b, h, generator=gen).to(dtype)
    start = torch.randn(V, h, generator=gen) * 0.01
    ref_w = start.numpy().copy()
    ref_p = np.zeros((s, h), dtype=np.float32)
    ol.embedding_grad_ordered(tok.numpy(), pid.numpy(), dout.float().numpy(), ref_w, ref_p)
    outs = []
    for _ in range(2):
        dw, dp = start.to(cuda), torch.zeros(s, h, device=cuda)
        K.embedding_bwd(tok.to(cuda), pid.to(cuda), dout.to(cuda), dw, dp)
        outs.append((dw.cpu(), dp.cpu()))
    assert torch.equal(outs[0][0], torch.from_numpy(ref_w))
    assert torch.equal(outs[0][1], torch.from_numpy(ref_p))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    # one table only
    dw = start.to(cuda)
    K.embedding_bwd(tok.to(cuda), pid.to(cuda), dout.to(cuda), dw, None)
    assert torch.equal(dw.cpu(), outs[0][0])


@pytest.mark.parametrize("b,s", [(3, 12000), (32, 2048)])
def test_embedding_backward_beyond_one_sort_chunk(cuda, b, s):
    """More tokens than one LDS sort holds (32768): consecutive chunks of
    whole sequence positions, bit-exact against the oracle's chunked
    ordered sum, with heavily repeated ids across the chunk edges (b 32,
    s 2048 is a first stage at micro-batch 32)."""
    announce(f"embedding backward in chunks b {b} s {s}")
    gen = torch.Generator().manual_seed(22)
    h, V = 64, 50304
    tok = torch.randint(0, 5, (b, s), generator=gen)
    tok[:, ::3] = torch.randint(0, V, (b, (s + 2) // 3), generator=gen)
    pid = torch.arange(s).expand(b, s).contiguous()
    dout = torch.randn(s, b, h, generator=gen).to(torch.bfloat16)
    start = torch.randn(V, h, generator=gen) * 0.01
    ref_w = start.numpy().copy()
    ref_p = np.zeros((s, h), dtype=np.float32)
    ol.embedding_grad_ordered(tok.numpy(), pid.numpy(), dout.float().numpy(), ref_w, ref_p)
    dw, dp = start.to(cuda), torch.zeros(s, h, device=cuda)
    K.embedding_bwd(tok.to(cuda), pid.to(cuda), dout.to(cuda), dw, dp)
    torch.cuda.synchronize()
    assert torch.equal(dw.cpu(), torch.from_numpy(ref_w))
    assert torch.equal(dp.cpu(), torch.from_numpy(ref_p))


def _lcg_batch_exact(ids, seq, vocab):
    """The synthetic batch by Python integers: the int64 products wrap in
    two's complement, the residues are floor-mod (non-negative)."""
    def wrap(x):
        x &= (1 << 64) - 1
        return x - (1 << 64) if x >= 1 << 63 else x

    tokens = [[wrap(i * 1103515245 + p * 12345) % vocab for p in range(seq)] for i in ids]
    mask = [[1.0 if wrap(i + p) % 4 else 0.0 for p in range(seq)] for i in ids]
    return tokens, mask


def test_synthetic_batch_kernel_matches_the_host_batch(cuda):
    """eth_synthetic_batch: the reference's known answers, the torch path on
    the CPU (ragged sequence, more than one 64-sample launch), and products
    past 2^63 against exact integer arithmetic."""
    from tests.helpers import known_answers

    announce("synthetic batch kernel")
    for case in known_answers()["synthetic_gpt_batch"]["cases"]:
        tokens, mask, positions, attn = synthetic_gpt_batch(case["ids"], case["seq"], case["vocab"], "cuda")
        assert tokens.tolist() == case["tokens"]
        assert mask.tolist() == case["mask"]
        assert positions.tolist() == [list(range(case["seq"]))] * len(case["ids"])
        assert attn.shape == (len(case["ids"]), 1, case["seq"], case["seq"]) and attn.is_cuda
    ids = list(range(5, 5 + 3 * 67, 3))  # 67 samples: two launches
    for seq, vocab in ((7, 50257), (2048, 50304), (33, 4)):
        g = synthetic_gpt_batch(ids, seq, vocab, "cuda", attention_mask=False)
        c = synthetic_gpt_batch(ids, seq, vocab, "cpu", attention_mask=False)
        assert g[3] is None and c[3] is None
        for a, b in zip(g[:3], c[:3]):
            assert a.dtype == b.dtype and torch.equal(a.cpu(), b)
    big = [0, 1, 2**40 + 7, 2**62 - 1, 9_000_000_000_000_000_000]
    tokens, mask, _, _ = synthetic_gpt_batch(big, 19, 50257, "cuda", attention_mask=False)
    ref_t, ref_m = _lcg_batch_exact(big, 19, 50257)
    assert tokens.tolist() == ref_t
    assert mask.tolist() == ref_m


def test_cross_entropy_backward_beyond_one_launch(cuda):
    """70,000 rows (past the 65,535 rows of one launch's grid) against the
    fp64 oracle's gradient, every row including the last launch's."""
    announce("cross entropy backward, 70000 rows")
    gen = torch.Generator().manual_seed(23)
    rows, V = 70000, 64
    z = (torch.randn(rows, V, generator=gen) * 2).to(torch.bfloat16)
    lab = torch.randint(0, V, (rows,), generator=gen)
    bad = torch.zeros(1, dtype=torch.int32, device=cuda)
    loss, lse = K.xent_fwd(z.to(cuda), lab.to(cuda), bad)
    g = torch.rand(rows, generator=gen)
    dz = K.xent_bwd(z.to(cuda), lab.to(cuda), lse, g.to(cuda)).cpu()
    zr = z.double().requires_grad_(True)
    ol.vocab_cross_entropy(zr, lab).backward(g.double())
    err = (dz.double() - zr.grad).abs().amax(dim=1)
    assert (err <= 2**-7 * zr.grad.abs().amax(dim=1) + 1e-30).all()
    assert bad.item() == 0


def test_embedding_dropout_draws_a_mask_per_call_and_backward_replays_it(cuda):
    announce("embedding dropout masks")
    from eth_amd.model.embedding import gen_embedding_op

    p = 0.5
    cfg = GPTConfig(hidden_size=64, num_attention_heads=2, ffn_hidden_size=256, num_layers=1, seq_length=32,
                    micro_batch_size=2, padded_vocab_size=512, hidden_dropout=p, params_dtype=torch.bfloat16,
                    device="cuda", seed=3)
    op = gen_embedding_op("encoder-embedding", 0, cfg).train()
    with torch.no_grad():  # every embedded value is 1.5, so a zero output means dropped
        op.word_embeddings.weight.fill_(1.0)
        op.position_embeddings.weight.fill_(0.5)
    gen = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 512, (2, 32), generator=gen).to(cuda)
    pos = torch.arange(32).expand(2, 32).contiguous().to(cuda)
    outs = [op({"enc_input_ids": ids, "enc_position_ids": pos}, {}, {})["hidden_states"] for _ in range(2)]
    keeps = [o != 0 for o in outs]
    assert not torch.equal(keeps[0], keeps[1])
    for o, keep in zip(outs, keeps):
        kept = keep.float().mean().item()
        assert 0.4 < kept < 0.6
        (g,) = torch.autograd.grad(o.float().sum(), op.position_embeddings.weight, retain_graph=True)
        # d(sum)/d pos[s] = sum over the batch of keep / (1 - p): small integers
        assert torch.equal(g.float(), (keep.float() / (1 - p)).sum(1))


def _oracle_params(tr):
    ops = tr.model.language_model.ops
    return {
        "word": tr.embedding.word_embeddings.weight.detach().float().cpu(),
        "pos": tr.embedding.position_embeddings.weight.detach().float().cpu(),
        "lnf_w": ops[-2].input_layernorm.weight.detach().float().cpu(),
        "lnf_b": ops[-2].input_layernorm.bias.detach().float().cpu(),
        "layers": [{k: p.detach().float().cpu() for k, p in lp.items()} for lp in tr_layer_params(tr)],
    }


def _check_first_last_gradients(tr, sample_ids, heads, unpadded_vocab=50257):
    """One forward/backward + grad sync + tied sum of the trainer against the
    fp64 oracle: per-token losses within 2e-2, and for every main grad both
    its norm within 2e-2 and its element-wise relative error within 5e-2."""
    from eth_amd.loss import global_normalization_scale

    params = _oracle_params(tr)
    ops = tr.model.language_model.ops
    tr.ddp.zero_grad_buffer()
    losses, lo = tr.forward_backward(sample_ids)
    tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
    tr.tie_gradients()
    torch.cuda.synchronize()
    tokens, mask, positions, _ = synthetic_gpt_batch(sample_ids, tr.cfg.seq_length, unpadded_vocab, "cpu")
    ref_losses, ref_mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, heads)
    assert _rel(losses, ref_losses) < 2e-2
    # main grads hold d(sum(loss*mask)/sum(mask)) after the sync, times the
    # loss scale unless the sync's unpack unscaled them
    scale = 1.0 if tr.optimizer.grads_unscaled_by_sync else tr.optimizer.get_loss_scale().item()
    checks = [("word", tr.embedding.word_embeddings.weight, grads["word"]),
              ("pos", tr.embedding.position_embeddings.weight, grads["pos"]),
              ("head", tr.post.word_embeddings.weight, grads["word"]),
              ("lnf_w", ops[-2].input_layernorm.weight, grads["lnf_w"]),
              ("lnf_b", ops[-2].input_layernorm.bias, grads["lnf_b"])]
    for i, (lp, gl) in enumerate(zip(tr_layer_params(tr), grads["layers"])):
        for k, p in lp.items():
            checks.append((f"layer{i}.{k}", p, gl[k]))
    for name, p, ref in checks:
        g = p.main_grad.double().cpu() / scale
        rn = ref.norm().item()
        assert abs(g.norm().item() - rn) <= 2e-2 * rn + 1e-12, (name, g.norm().item(), rn)
        assert _rel(g, ref) < 5e-2, (name, _rel(g, ref))
    return losses


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_first_last_stage_matches_fp64_oracle(cuda, dtype):
    announce(f"first+last stage parity {dtype}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=11)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                               initial_loss_scale=1024.0)
    sample_ids = [3, 8]
    _check_first_last_gradients(tr, sample_ids, 4)
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


# GPT-6.7B first+last stage widths, fp16, loss scale 2^16
C5_WIDTHS = dict(hidden_size=4096, num_attention_heads=32, ffn_hidden_size=16384, padded_vocab_size=50304,
                 params_dtype=torch.float16, device="cuda")


def _c5_trainer(cfg):
    return FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0,
                                 bucket_cap_bytes=32 << 20, initial_loss_scale=2.0**16)


def test_c5_widths_at_a_short_sequence_match_fp64_oracle(cuda):
    """h 4096, 32 heads (hn 128), FFN 16384, V 50304, fp16 with loss scale
    2^16 -- the production tiles, the 128-wide attention kernels, the
    4096-column LayerNorm and the full-vocabulary cross entropy -- at s 256,
    b 1, one layer, against the fp64 oracle; then the step applies and the
    tied copies stay equal."""
    announce("C5 widths, s 256, b 1, 1 layer, fp16 parity")
    cfg = GPTConfig(num_layers=1, seq_length=256, micro_batch_size=1, seed=5, **C5_WIDTHS)
    tr = _c5_trainer(cfg)
    _check_first_last_gradients(tr, [5], 32)
    ok, norm, _ = tr.optimizer.step()
    torch.cuda.synchronize()
    assert ok and norm is not None and np.isfinite(norm)
    assert torch.equal(tr.embedding.word_embeddings.weight, tr.post.word_embeddings.weight)


def test_c5_full_shape_trains(cuda):
    """configs[4] at its full shape (2 layers, s 2048, b 2, T 4096): two
    training steps apply without overflow, with a finite loss near its
    value at initialisation, finite per-tensor main grads and a finite norm, and the
    tied embedding / head copies identical after each step."""
    announce("C5 full shape, 2 steps")
    import math

    cfg = GPTConfig(num_layers=2, seq_length=2048, micro_batch_size=2, seed=1234, **C5_WIDTHS)
    tr = _c5_trainer(cfg)
    # uniform labels: with the reference's labels = 0 every gradient of the
    # step pushes the same logit up, and AdamW's first (sign-like) update
    # across 4096-wide layers already saturates the fp16 softmax, leaving
    # the second step with a zero loss and zero gradients
    gen = torch.Generator(device="cuda").manual_seed(7)
    for step in range(2):
        labels = torch.randint(0, 50257, (2, 2048), generator=gen, device="cuda")
        losses, lo, ok, norm = tr.train_step([2 * step, 2 * step + 1], labels)
        torch.cuda.synchronize()
        assert ok, f"step {step} overflowed at loss scale {tr.optimizer.get_loss_scale().item()}"
        assert norm is not None and np.isfinite(norm) and norm > 0
        assert bool(torch.isfinite(losses).all())
        mean = (lo.local_loss_sum / lo.local_loss_weight).item()
        if step == 0:
            # unit-variance LN output against N(0, 0.02) head rows: logits of
            # variance 0.02^2 * 4096, so the expected loss is ln V + var / 2
            assert abs(mean - (math.log(50304) + 0.5 * 0.02**2 * 4096)) < 1.0, mean
            first = mean
        else:
            assert np.isfinite(mean) and mean < first + 1.0, (first, mean)
        for name, p in tr.model.named_parameters():
            assert bool(torch.isfinite(p.main_grad).all()), name
        assert torch.equal(tr.embedding.word_embeddings.weight, tr.post.word_embeddings.weight)
    assert tr.optimizer.get_loss_scale().item() == 2.0**16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_first_last_update_overlapped_with_the_next_forward_is_bit_identical(cuda, dtype):
    """The first+last stage with its AdamW update split into parts
    (embedding; the first layer's attention and MLP halves; the next layer;
    the final LayerNorm with the tied head copy) launched under the next
    forward: three steps give the losses, norms and parameters of the in-line
    update bit for bit, and the tied copies stay equal."""
    announce(f"first+last overlapped update {dtype}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=13)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=0.05, initial_loss_scale=1024.0)
    plain, over = FirstLastStageTrainer(cfg, **kw), FirstLastStageTrainer(cfg, overlap_optimizer=True, **kw)
    assert len(over.optimizer._overlap[1]) == 5
    for step in range(3):
        ids = [3 + step, 8 + step]
        l_p, _, ok_p, n_p = plain.train_step(ids)
        l_o, _, ok_o, n_o = over.train_step(ids)
        assert ok_p and ok_o and n_p == n_o, (step, n_p, n_o)
        assert torch.equal(l_p, l_o), step
    over.optimizer.join_overlapped_update()
    torch.cuda.synchronize()
    for (n1, p1), (_, p2) in zip(plain.model.named_parameters(), over.model.named_parameters()):
        assert torch.equal(p1, p2), n1
    assert torch.equal(over.embedding.word_embeddings.weight, over.post.word_embeddings.weight)


@pytest.mark.parametrize("misalign", [0, 1])
def test_tied_sum_with_statistics_equals_the_sum_then_the_statistics(cuda, misalign):
    """eth_tied_grad_sum_stats against eth_tied_grad_sum followed by
    eth_grad_stats(ETH_STATS_SCALED_OVERFLOW) on the same chunk table: equal
    sums in both copies, equal per-chunk partials and flags, with a ragged
    length, a copy 16-byte aligned or not, and an element whose loss-scaled
    sum overflows fp32."""
    from eth_amd import _native as nat
    from eth_amd.grad_sync.executor import chunk_table, split_block

    announce(f"tied sum + statistics, copy misaligned by {misalign}")
    n, scale = 100_003, 1024.0
    gen = torch.Generator(device="cuda").manual_seed(21)
    c0 = (n + 3) // 4 * 4 + 4 + misalign  # the copy's first element (16-byte aligned when misalign is 0)
    base = torch.randn(c0 + n, generator=gen, device="cuda")
    for overflow in (False, True):
        a, b = base.clone(), base.clone()
        if overflow:
            for buf in (a, b):
                buf[12_345] = 2e35
                buf[c0 + 12_345] = 2e35  # sum 4e35, x 1024 > fp32 max
        results = []
        for buf, fused in ((a, False), (b, True)):
            root, copy = buf[:n], buf[c0 : c0 + n]
            entries = []
            split_block(root.data_ptr(), 4, 1, n, n, 0, 1.0, nat.CHUNK_NORM, entries)
            table = nat.table_to_device(chunk_table(entries), cuda)
            flag = torch.zeros(1, device="cuda")
            part = torch.full((len(entries) + 2,), -1.0, dtype=torch.float64, device="cuda")
            stream = nat.stream_ptr(cuda)
            if fused:
                nat.call("eth_tied_grad_sum_stats", nat.ptr(table), len(entries), nat.ptr(root), nat.ptr(copy),
                         scale, nat.ptr(flag), nat.ptr(part), 2, stream)
            else:
                K.tied_grad_sum(root, copy) if misalign == 0 else _tied_sum_unaligned(root, copy)
                nat.call("eth_grad_stats", nat.ptr(table), len(entries), scale, nat.STATS_SCALED_OVERFLOW,
                         nat.ptr(flag), nat.ptr(part), 2, stream)
            torch.cuda.synchronize()
            results.append((root.clone(), copy.clone(), part.clone(), flag.item()))
        (ra, ca, pa, fa), (rb, cb, pb, fb) = results
        assert torch.equal(ra, rb) and torch.equal(ca, cb) and torch.equal(ra, ca)
        assert torch.equal(pa, pb) and pa[0].item() == pa[1].item() == -1.0
        assert fa == fb == (1.0 if overflow else 0.0)


def _tied_sum_unaligned(root, copy):
    """The tied sum of fp32 tensors that eth_tied_grad_sum (16-byte aligned
    only) does not take, in torch: the same one fp32 add per element."""
    s = root + copy
    root.copy_(s)
    copy.copy_(s)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["fused", "standalone", "overlapped"])
def test_shared_tied_storage_is_bit_identical_to_two_copies(cuda, dtype, mode):
    """The tied head copy sharing the root's weight, master and moments (one
    update for both) against two separately updated copies, as the
    reference keeps them: three steps give the same losses and norms, and
    every parameter, main grad, master and moment is bit-identical -- with
    the statistics fused into the sync, in one standalone pass (which also
    unscales the copy's main grad in place), and with the update overlapped
    with the next forward."""
    announce(f"shared tied storage {dtype} {mode}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=17)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=0.05, initial_loss_scale=1024.0,
              overlap_optimizer=mode == "overlapped")
    two = FirstLastStageTrainer(cfg, share_tied_storage=False, **kw)
    one = FirstLastStageTrainer(cfg, **kw)
    root, copy = one.embedding.word_embeddings.weight, one.post.word_embeddings.weight
    assert copy.data_ptr() == root.data_ptr() and copy.main_grad.data_ptr() != root.main_grad.data_ptr()
    assert one.optimizer.optimizer_parameter_for_model_parameter(copy) is \
        one.optimizer.optimizer_parameter_for_model_parameter(root)
    if mode == "standalone":
        one.optimizer.unbind_gradient_sync()
        two.optimizer.unbind_gradient_sync()
    gen = torch.Generator(device="cuda").manual_seed(5)
    for step in range(3):
        labels = torch.randint(0, 50257, (2, 128), generator=gen, device="cuda")
        l2, _, ok2, n2 = two.train_step([3 + step, 8 + step], labels)
        l1, _, ok1, n1 = one.train_step([3 + step, 8 + step], labels)
        assert ok1 and ok2 and n1 == n2, (step, n1, n2)
        assert torch.equal(l1, l2), step
    one.optimizer.join_overlapped_update()
    two.optimizer.join_overlapped_update()
    torch.cuda.synchronize()
    for (name, p1), (_, p2) in zip(one.model.named_parameters(), two.model.named_parameters()):
        assert torch.equal(p1, p2), name
        assert torch.equal(p1.main_grad, p2.main_grad), name
        m1 = one.optimizer.optimizer_parameter_for_model_parameter(p1)
        m2 = two.optimizer.optimizer_parameter_for_model_parameter(p2)
        assert torch.equal(m1, m2), name
        s1, s2 = one.optimizer.state_for_model_parameter(p1), two.optimizer.state_for_model_parameter(p2)
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(s1[k], s2[k]), (name, k)
        assert float(s1["step"]) == float(s2["step"]) == 3.0, name


@pytest.mark.parametrize("case", ["microbatches", "fp16_main_grads"])
def test_shared_tied_storage_in_microbatches_and_fp16_main_grads(cuda, tmp_path, case):
    """The shared tied storage against two updated copies where the step
    takes other paths: two microbatches per step (the loss weights of both
    forwards read from their pinned copies and summed on the host), and fp16
    main grads (the reference's fp16 contract: 16-bit tied sum, the widening
    statistics pass).  Losses, norms, parameters, masters and moments are
    bit-identical over two steps, and so are the post_step evidence
    snapshots of every parameter."""
    from eth_amd.grad_sync.evidence import load_rank_snapshot

    announce(f"shared tied storage: {case}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=torch.float16, device="cuda", seed=23)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=0.05, initial_loss_scale=1024.0,
              accumulate_allreduce_grads_in_fp32=case != "fp16_main_grads")
    two = FirstLastStageTrainer(cfg, share_tied_storage=False, **kw)
    one = FirstLastStageTrainer(cfg, **kw)
    assert one.post.word_embeddings.weight.data_ptr() == one.embedding.word_embeddings.weight.data_ptr()
    gen = torch.Generator(device="cuda").manual_seed(29)
    for step in range(2):
        if case == "microbatches":
            ids = [[3 + step, 8 + step], [11 + step, 2 + step]]
            labels = [torch.randint(0, 50257, (2, 128), generator=gen, device="cuda") for _ in ids]
            l2, (n2_, w2), ok2, norm2 = two.train_step_microbatches(ids, labels)
            l1, (n1_, w1), ok1, norm1 = one.train_step_microbatches(ids, labels)
            assert torch.equal(n1_, n2_) and torch.equal(w1, w2)
            assert all(torch.equal(a, b) for a, b in zip(l1, l2))
        else:
            labels = torch.randint(0, 50257, (2, 128), generator=gen, device="cuda")
            l2, _, ok2, norm2 = two.train_step([3 + step, 8 + step], labels)
            l1, _, ok1, norm1 = one.train_step([3 + step, 8 + step], labels)
            assert torch.equal(l1, l2)
        assert ok1 and ok2 and norm1 == norm2, (step, norm1, norm2)
    paths = [tr.record_evidence(tmp_path / name, "post_step", 2) for tr, name in ((one, "one"), (two, "two"))]
    torch.cuda.synchronize()
    snaps = [load_rank_snapshot(p_) for p_ in paths]
    assert len(snaps[0]["records"]) == len(snaps[1]["records"]) == len(one.bindings)
    for r1, r2 in zip(*(s_["records"] for s_ in snaps)):
        name = r1["descriptor"]["logical_param_id"]
        assert name == r2["descriptor"]["logical_param_id"]
        for key in ("parameter", "main_grad", "optimizer_parameter"):
            assert torch.equal(r1[key], r2[key]), (name, key)
        for key in ("exp_avg", "exp_avg_sq", "step"):
            assert torch.equal(r1["optimizer_state"][key], r2["optimizer_state"][key]), (name, key)
        assert r1["optimizer_hyperparameters"] == r2["optimizer_hyperparameters"], name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_first_last_fused_statistics_match_the_standalone_pass(cuda, dtype):
    """The first+last stage unscales in the sync's unpack and takes the tied
    root's norm share after the tied sum: the step's norm, outcome and
    updated parameters equal those of one standalone statistics pass over
    every gradient, and an overflow that appears in the root after the sync
    is still caught under fp16 loss scaling (the step is skipped)."""
    announce(f"first+last fused statistics {dtype}")
    cfg = GPTConfig(hidden_size=256, num_attention_heads=4, ffn_hidden_size=1024, num_layers=2, seq_length=128,
                    micro_batch_size=2, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=11)
    kw = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=0.05, initial_loss_scale=1024.0)
    fused, plain = FirstLastStageTrainer(cfg, **kw), FirstLastStageTrainer(cfg, **kw)
    assert fused.optimizer.grads_unscaled_by_sync
    plain.optimizer.unbind_gradient_sync()
    for (n1, p1), (n2, p2) in zip(fused.model.named_parameters(), plain.model.named_parameters()):
        assert n1 == n2 and torch.equal(p1, p2)
    for step in range(2):
        _, _, ok_f, norm_f = fused.train_step([3, 8])
        _, _, ok_p, norm_p = plain.train_step([3, 8])
        assert ok_f and ok_p
        # the sums of squares are formed in other chunks (fp32 within a
        # chunk), so the norms agree to the 1e-6 bar of the canonical clip
        assert abs(norm_f - norm_p) <= 1e-6 * norm_p, (step, norm_f, norm_p)
        for (n1, p1), (_, p2) in zip(fused.model.named_parameters(), plain.model.named_parameters()):
            # unscaling each tied addend before the sum (power-of-two scale)
            # leaves the same bits as unscaling the sum
            assert torch.equal(p1.main_grad, p2.main_grad), n1
            m1 = fused.optimizer.optimizer_parameter_for_model_parameter(p1)
            m2 = plain.optimizer.optimizer_parameter_for_model_parameter(p2)
            assert torch.allclose(m1, m2, rtol=1e-6, atol=1e-9), n1
    if dtype != torch.float16:
        return  # bf16 trains without a loss scaler, hence without an overflow check
    # overflow in the tied root after the sync
    tr = fused
    tr.ddp.zero_grad_buffer()
    _, lo = tr.forward_backward([5, 9])
    from eth_amd.loss import global_normalization_scale

    tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
    # (the tied sum takes the root's post-sync statistics in the same pass)
    tr.embedding.word_embeddings.weight.main_grad[7, 3] = float("inf")
    tr.tie_gradients()
    before = tr.embedding.word_embeddings.weight.detach().clone()
    ok, norm, _ = tr.optimizer.step()
    torch.cuda.synchronize()
    assert not ok and norm is None
    assert torch.equal(tr.embedding.word_embeddings.weight, before)
    assert tr.optimizer.get_loss_scale().item() == 1024.0  # hysteresis 2: one overflow does not back off
    # a tied sum that is finite once unscaled but whose loss-scaled value
    # overflows fp32: the reference sums the scaled addends (inf) and skips
    # the step, and so does the fused path; the second overflow backs off
    tr.ddp.zero_grad_buffer()
    _, lo = tr.forward_backward([5, 9])
    tr.grad_sync.execute(global_normalization_scale(tr.nominal, lo.local_loss_weight))
    tr.embedding.word_embeddings.weight.main_grad[7, 3] = 1e36  # the sum x 1024 > fp32 max
    tr.post.word_embeddings.weight.main_grad[7, 3] = 0.0
    tr.tie_gradients()
    ok, norm, _ = tr.optimizer.step()
    torch.cuda.synchronize()
    assert not ok and norm is None
    assert torch.equal(tr.embedding.word_embeddings.weight, before)
    assert tr.optimizer.get_loss_scale().item() == 512.0
