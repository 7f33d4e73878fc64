"""torch-CPU restatement of the GPT layer ops and one pipeline stage (test
oracle).  Computes in fp32 (or fp64) from the same 16-bit inputs the GPU
path sees.

Follows eth/runtime/megatron/model/flex_ops.py:
  * LayerNorm: MixedFusedLayerNorm, eps 1e-5 (model/fused_layer_norm.py:62-89)
  * QKV: F.linear + bias, view [s, b, np, 3*hn], split q | k | v per head
    (flex_ops.py:1069-1103, mpu/utils.py:33-52)
  * attention: F.scaled_dot_product_attention(is_causal=True) on
    [b, np, s, hn], output [s, b, np*hn] (flex_ops.py:66-96)
  * proj / fc2: F.linear without bias (skip_bias_add), bias added in
    bias-dropout-add: residual + dropout(x + b) (flex_ops.py:104-134)
  * fc1 + GELU: F.gelu(x + b, approximate="tanh") (flex_ops.py:60-63,1897)
  * LM head + cross entropy: logits = h @ E^T, max-subtracted
    loss = log sum exp(z - max) - (z[label] - max)
    (model/language_model.py:24-38, mpu/cross_entropy.py:36-92)
"""

import math

import torch
import torch.nn.functional as F


def layer_norm(x, gamma, beta, eps=1e-5):
    return F.layer_norm(x, (x.shape[-1],), gamma, beta, eps)


def bias_gelu(x, bias):
    return F.gelu(x + bias, approximate="tanh")


def bias_dropout_add(x, bias, residual):
    """p = 0 (the parity setting): residual + (x + bias)."""
    return residual + (x + bias)


def causal_attention(q, k, v):
    """q, k, v: [s, b, np, hn] -> [s, b, np*hn] (SDPA semantics)."""
    s, b, n, d = q.shape
    out = F.scaled_dot_product_attention(
        q.permute(1, 2, 0, 3), k.permute(1, 2, 0, 3), v.permute(1, 2, 0, 3), is_causal=True
    )
    return out.permute(2, 0, 1, 3).reshape(s, b, n * d)


def causal_attention_explicit(q, k, v):
    """Brute-force softmax(QK^T/sqrt(d) + causal -inf) V for tiny shapes."""
    s, b, n, d = q.shape
    qh, kh, vh = (t.permute(1, 2, 0, 3) for t in (q, k, v))
    scores = qh @ kh.transpose(-1, -2) / math.sqrt(d)
    mask = torch.triu(torch.ones(s, s, dtype=torch.bool), diagonal=1)
    scores = scores.masked_fill(mask, float("-inf"))
    out = torch.softmax(scores, dim=-1) @ vh
    return out.permute(2, 0, 1, 3).reshape(s, b, n * d)


def transformer_layer(x, p, heads):
    """One ParallelTransformerLayer (10 ops) on x [s, b, h]; p holds the
    layer's parameters (fp32 or fp64 CPU tensors)."""
    s, b, h = x.shape
    hn = h // heads
    ln1 = layer_norm(x, p["ln1_w"], p["ln1_b"])
    qkv = F.linear(ln1, p["qkv_w"], p["qkv_b"]).view(s, b, heads, 3 * hn)
    q, k, v = torch.split(qkv, hn, dim=-1)
    ctx = causal_attention(q, k, v)
    proj = F.linear(ctx, p["proj_w"])
    h1 = bias_dropout_add(proj, p["proj_b"], x)
    ln2 = layer_norm(h1, p["ln2_w"], p["ln2_b"])
    fc1 = F.linear(ln2, p["fc1_w"])
    act = bias_gelu(fc1, p["fc1_b"])
    fc2 = F.linear(act, p["fc2_w"])
    return bias_dropout_add(fc2, p["fc2_b"], h1)


LAYER_PARAM_NAMES = ("ln1_w", "ln1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "ln2_w", "ln2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")


def middle_stage_fwd_bwd(x, layers, heads, dy, dtype=torch.float32):
    """Forward + backward of a middle pipeline stage: returns the output,
    the input gradient and per-parameter gradients (lists of dicts)."""
    x = x.to(dtype).detach().requires_grad_(True)
    params = [{k: v.to(dtype).detach().requires_grad_(True) for k, v in p.items()} for p in layers]
    h = x
    for p in params:
        h = transformer_layer(h, p, heads)
    h.backward(dy.to(dtype))
    return h.detach(), x.grad.detach(), [{k: v.grad.detach() for k, v in p.items()} for p in params]


def vocab_cross_entropy(logits, labels):
    """Per-token loss of _VocabParallelCrossEntropy at TP = 1
    (mpu/cross_entropy.py:36-92): subtract the row maximum, then
    loss = log(sum(exp(z - max))) - (z[label] - max).  The maximum is a
    constant of the backward, as in the reference's autograd Function.

    Computes in the dtype it is given (fp32 for the reference's
    `output.float()`, flex_ops.py:1976-1981; fp64 in the fp64 oracle); 16-bit
    logits are widened to fp32 first."""
    z = logits if logits.dtype in (torch.float32, torch.float64) else logits.float()
    shifted = z - z.detach().amax(dim=-1, keepdim=True)
    target = shifted.gather(-1, labels.unsqueeze(-1)).squeeze(-1)
    return torch.log(torch.exp(shifted).sum(dim=-1)) - target


EMBEDDING_CHUNK_ROWS = 32768


def embedding_grad_ordered(tokens, positions, dout, word_grad, pos_grad, chunk_rows=EMBEDDING_CHUNK_ROWS):
    """F.embedding's backward into fp32 main grads, restated with a fixed
    summation order (numpy fp32): every table row receives the fp32 sum of
    its dout rows taken in ascending dout-row order (row = s * b_size + b
    of dout [s, b, h]), added once to its previous value.  Inputs of more
    than `chunk_rows` rows are taken in consecutive chunks of whole sequence
    positions (floor(chunk_rows / b_size) positions each), each chunk adding
    its own ordered sums in turn.  Ids outside the table are clamped, as the
    kernels do.  `word_grad` / `pos_grad` are numpy fp32 tables updated in
    place (either may be None).
    (flex_ops.py:450-485 forward; the backward is autograd's
    embedding_dense_backward plus the main_grad hook of
    model/distributed.py:116-123.)"""
    import numpy as np

    s, b, h = dout.shape
    rows = np.ascontiguousarray(dout, dtype=np.float32).reshape(s * b, h)
    step = max(1, chunk_rows // b) * b
    for table, ids in ((word_grad, tokens), (pos_grad, positions)):
        if table is None:
            continue
        ids = np.clip(np.asarray(ids, dtype=np.int64), 0, table.shape[0] - 1)
        by_row = ids.T.reshape(-1)  # dout row s*b_size + b holds ids[b, s]
        for r0 in range(0, s * b, step):
            sums = {}
            for r in range(r0, min(r0 + step, s * b)):
                t = int(by_row[r])
                sums[t] = sums.get(t, np.zeros(h, dtype=np.float32)) + rows[r]
            for t, acc in sums.items():
                table[t] += acc
    return word_grad, pos_grad


def full_model_fwd_bwd(tokens, positions, loss_mask, params, heads, labels=None, dtype=torch.float64):
    """Whole GPT on one stage (embedding -> layers -> final LN -> tied LM
    head -> cross entropy -> masked mean), the way the first+last stage runs
    it (flex_ops.py:450-485,547-575,1952-1985; grad_sync/loss.py:16-39).

    Returns (per-token loss [b, s], mean masked loss, gradients of the mean
    masked loss by parameter name, with the word embedding's gradient being
    the tied sum of its embedding and LM-head uses)."""
    p = {k: (v.to(dtype).detach().requires_grad_(True) if torch.is_tensor(v) else v) for k, v in params.items()}
    layers = [{k: v.to(dtype).detach().requires_grad_(True) for k, v in lp.items()} for lp in params["layers"]]
    head = p["word"].detach().clone().requires_grad_(True)
    x = (p["word"][tokens] + p["pos"][positions]).transpose(0, 1)  # [s, b, h]
    for lp in layers:
        x = transformer_layer(x, lp, heads)
    hidden = layer_norm(x.transpose(0, 1), p["lnf_w"], p["lnf_b"])  # [b, s, h]
    logits = hidden @ head.t()
    if labels is None:
        labels = torch.zeros(tokens.shape, dtype=torch.long)
    losses = vocab_cross_entropy(logits, labels).to(dtype)
    mask = loss_mask.to(dtype)
    mean = (losses * mask).sum() / mask.sum()
    mean.backward()
    grads = {"word": p["word"].grad + head.grad, "pos": p["pos"].grad, "lnf_w": p["lnf_w"].grad, "lnf_b": p["lnf_b"].grad}
    grads["layers"] = [{k: v.grad for k, v in lp.items()} for lp in layers]
    return losses.detach(), mean.detach(), grads
