"""CPU pins of the layer oracle (oracle/layer.py).

Every function of the oracle is checked here against something other than
its own formula: the library routine the reference itself calls, a closed
form that a wiring mistake would break, or finite differences of the
oracle's own forward (for the gradients autograd derives from it).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import layer as ol

H, HEADS, FFN = 8, 2, 16


def _layer_params(gen, h=H, f=FFN, dtype=torch.float64, zero_weights=False):
    def w(*shape):
        return torch.zeros(*shape, dtype=dtype) if zero_weights else torch.randn(*shape, generator=gen, dtype=dtype) * 0.3

    return {
        "ln1_w": 1.0 + 0.1 * torch.randn(h, generator=gen, dtype=dtype),
        "ln1_b": 0.1 * torch.randn(h, generator=gen, dtype=dtype),
        "qkv_w": w(3 * h, h),
        "qkv_b": 0.1 * torch.randn(3 * h, generator=gen, dtype=dtype),
        "proj_w": w(h, h),
        "proj_b": 0.1 * torch.randn(h, generator=gen, dtype=dtype),
        "ln2_w": 1.0 + 0.1 * torch.randn(h, generator=gen, dtype=dtype),
        "ln2_b": 0.1 * torch.randn(h, generator=gen, dtype=dtype),
        "fc1_w": w(f, h),
        "fc1_b": 0.1 * torch.randn(f, generator=gen, dtype=dtype),
        "fc2_w": w(h, f),
        "fc2_b": 0.1 * torch.randn(h, generator=gen, dtype=dtype),
    }


# ------------------------------------------------------------ cross entropy --
def _reference_ce_case():
    """mpu/tests/test_cross_entropy.py:58-89: 13 x 17 rows of 11 logits
    scaled by 1000, seed 1234, targets uniform (CPU generator here)."""
    gen = torch.Generator().manual_seed(1234)
    logits = 1000.0 * torch.randn(13, 17, 11, generator=gen)
    target = torch.randint(0, 11, (13, 17), generator=gen)
    return logits, target


def _torch_ce(z, t):
    return F.cross_entropy(z.view(-1, z.shape[-1]), t.view(-1), reduction="none").view_as(t)


def _losses_and_grad(fn, logits, target):
    """Per-token losses and the gradient of their mean (the reference test
    compares the mean and its gradient; per-token losses are stricter)."""
    z = logits.clone().requires_grad_(True)
    losses = fn(z, target)
    losses.mean().backward()
    return losses.detach(), z.grad


def test_cross_entropy_meets_the_reference_bar_at_logit_scale_1000():
    logits, target = _reference_ce_case()
    lt, gt = _losses_and_grad(_torch_ce, logits, target)
    lo, go = _losses_and_grad(ol.vocab_cross_entropy, logits, target)
    assert (lt - lo).abs().max().item() < 1e-6
    assert (lt.mean() - lo.mean()).abs().item() < 1e-6
    assert (gt - go).abs().max().item() < 1e-6


def test_cross_entropy_pin_rejects_the_unshifted_form():
    """A planted mistake -- logsumexp(z) - z[t] in fp32, which adds the
    maximum back before subtracting the target logit and so loses its low
    bits at logits ~1e3 -- fails the same bar: the pin has teeth."""
    logits, target = _reference_ce_case()

    def unshifted(z, t):
        return torch.logsumexp(z, dim=-1) - z.gather(-1, t.unsqueeze(-1)).squeeze(-1)

    lt, _ = _losses_and_grad(_torch_ce, logits, target)
    lo, _ = _losses_and_grad(unshifted, logits, target)
    assert (lt - lo).abs().max().item() >= 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cross_entropy_matches_torch_and_keeps_its_dtype(dtype):
    gen = torch.Generator().manual_seed(5)
    z = (torch.randn(37, 501, generator=gen) * 4).to(dtype)
    t = torch.randint(0, 501, (37,), generator=gen)
    out = ol.vocab_cross_entropy(z, t)
    assert out.dtype == dtype
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert torch.allclose(out, F.cross_entropy(z, t, reduction="none"), rtol=tol, atol=tol)
    # 16-bit logits are computed in fp32, as the reference's logits.float()
    assert ol.vocab_cross_entropy(z.to(torch.bfloat16), t).dtype == torch.float32


def test_cross_entropy_of_uniform_logits_is_log_vocab():
    z = torch.full((3, 50304), 7.25, dtype=torch.float64)
    t = torch.tensor([0, 17, 50303])
    assert torch.allclose(ol.vocab_cross_entropy(z, t), torch.full((3,), math.log(50304), dtype=torch.float64))


# ------------------------------------------------------------- layer pieces --
def test_layer_norm_uses_eps_1e5():
    x = torch.tensor([[1.0, -1.0, 1.0, -1.0]], dtype=torch.float64)
    y = ol.layer_norm(x, torch.ones(4, dtype=torch.float64), torch.zeros(4, dtype=torch.float64))
    assert torch.allclose(y, x / math.sqrt(1.0 + 1e-5), rtol=0, atol=1e-15)


def test_bias_gelu_is_the_tanh_approximation():
    # fast_gelu (flex_ops.py:60-63) at 1 and -1: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
    x = torch.tensor([0.5, -1.5], dtype=torch.float64)
    b = torch.tensor([0.5, 0.5], dtype=torch.float64)
    y = ol.bias_gelu(x, b)
    assert torch.allclose(y, torch.tensor([0.8411919906082768, -0.15880800939172324], dtype=torch.float64),
                          rtol=0, atol=1e-15)


def test_explicit_attention_equals_sdpa():
    gen = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(9, 2, 3, 4, generator=gen, dtype=torch.float64) for _ in range(3))
    assert torch.allclose(ol.causal_attention(q, k, v), ol.causal_attention_explicit(q, k, v), atol=1e-13)


# ------------------------------------------------- transformer layer wiring --
def test_zero_weight_layer_is_residual_plus_both_biases():
    """Zero QKV/proj/fc1/fc2 weights: the attention and MLP branches reduce
    to their output biases, so layer(x) = x + proj_b + fc2_b exactly."""
    gen = torch.Generator().manual_seed(3)
    p = _layer_params(gen, zero_weights=True)
    x = torch.randn(5, 2, H, generator=gen, dtype=torch.float64)
    out = ol.transformer_layer(x, p, HEADS)
    assert torch.allclose(out, x + p["proj_b"] + p["fc2_b"], rtol=0, atol=1e-14)


def test_qkv_is_split_per_head_q_k_v():
    """Head i owns rows [3 hn i, 3 hn (i+1)) of the QKV output, as q | k | v
    (flex_ops.py:1091-1103).  With zero QKV weights every key scores the
    same, attention averages identical values, so the context of head i is
    exactly the v slice of head i's bias; an identity projection then adds
    it to the residual."""
    gen = torch.Generator().manual_seed(4)
    p = _layer_params(gen, zero_weights=True)
    p["proj_w"] = torch.eye(H, dtype=torch.float64)
    x = torch.randn(6, 3, H, generator=gen, dtype=torch.float64)
    hn = H // HEADS
    v_bias = torch.cat([p["qkv_b"][3 * hn * i + 2 * hn : 3 * hn * (i + 1)] for i in range(HEADS)])
    out = ol.transformer_layer(x, p, HEADS)
    assert torch.allclose(out, x + v_bias + p["proj_b"] + p["fc2_b"], rtol=0, atol=1e-13)
    # the global [q | k | v] split would give a different context
    assert not torch.allclose(v_bias, p["qkv_b"][2 * H :])


def test_attention_is_causal_over_the_sequence_axis():
    """Zero query/key rows: scores are all equal, so each query averages
    the values of keys 0..t of its own sequence and batch entry.  The v
    rows copy LayerNorm's output, proj is the identity: the residual gains
    the running mean of ln1(x) along the sequence axis."""
    gen = torch.Generator().manual_seed(6)
    s, b = 7, 2
    p = _layer_params(gen, zero_weights=True)
    hn = H // HEADS
    qkv_w = torch.zeros(3 * H, H, dtype=torch.float64)
    for i in range(HEADS):
        qkv_w[3 * hn * i + 2 * hn : 3 * hn * (i + 1), hn * i : hn * (i + 1)] = torch.eye(hn, dtype=torch.float64)
    p["qkv_w"] = qkv_w
    p["qkv_b"] = torch.zeros(3 * H, dtype=torch.float64)
    p["proj_w"] = torch.eye(H, dtype=torch.float64)
    x = torch.randn(s, b, H, generator=gen, dtype=torch.float64)
    ln1 = F.layer_norm(x, (H,), p["ln1_w"], p["ln1_b"], 1e-5)
    running = ln1.cumsum(0) / torch.arange(1, s + 1, dtype=torch.float64).view(s, 1, 1)
    out = ol.transformer_layer(x, p, HEADS)
    assert torch.allclose(out, x + running + p["proj_b"] + p["fc2_b"], rtol=0, atol=1e-12)


def test_mlp_branch_is_fc2_of_gelu_of_the_fc1_bias():
    gen = torch.Generator().manual_seed(7)
    p = _layer_params(gen, zero_weights=True)
    p["fc2_w"] = torch.randn(H, FFN, generator=gen, dtype=torch.float64)
    x = torch.randn(3, 2, H, generator=gen, dtype=torch.float64)
    c = math.sqrt(2.0 / math.pi)
    fb = p["fc1_b"]
    gelu = 0.5 * fb * (1.0 + torch.tanh(c * (fb + 0.044715 * fb**3)))
    out = ol.transformer_layer(x, p, HEADS)
    assert torch.allclose(out, x + p["proj_b"] + p["fc2_w"] @ gelu + p["fc2_b"], rtol=0, atol=1e-12)


def test_layer_gradients_match_finite_differences():
    gen = torch.Generator().manual_seed(8)
    p = _layer_params(gen)
    x = torch.randn(4, 2, H, generator=gen, dtype=torch.float64)
    names = list(p)

    def fn(x, *vals):
        return ol.transformer_layer(x, dict(zip(names, vals)), HEADS)

    inputs = (x.requires_grad_(True), *(p[n].clone().requires_grad_(True) for n in names))
    assert torch.autograd.gradcheck(fn, inputs, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_middle_stage_gradients_are_the_directional_derivatives():
    """middle_stage_fwd_bwd contracts the upstream gradient dy with the
    stage's Jacobian: <dx, d> and <dW, D> equal the central differences of
    <stage(x), dy> along random directions d, D."""
    gen = torch.Generator().manual_seed(9)
    layers = [_layer_params(gen), _layer_params(gen)]
    x = torch.randn(4, 2, H, generator=gen, dtype=torch.float64)
    dy = torch.randn(4, 2, H, generator=gen, dtype=torch.float64)
    out, dx, grads = ol.middle_stage_fwd_bwd(x, layers, HEADS, dy, dtype=torch.float64)
    eps = 1e-6

    def objective(xv, ls):
        h = xv
        for lp in ls:
            h = ol.transformer_layer(h, lp, HEADS)
        return (h * dy).sum().item()

    d = torch.randn(x.shape, generator=gen, dtype=torch.float64)
    fd = (objective(x + eps * d, layers) - objective(x - eps * d, layers)) / (2 * eps)
    assert fd == pytest.approx((dx * d).sum().item(), rel=1e-6)
    for name in ("qkv_w", "fc2_b", "ln2_w"):
        D = torch.randn(layers[1][name].shape, generator=gen, dtype=torch.float64)
        plus = [layers[0], {**layers[1], name: layers[1][name] + eps * D}]
        minus = [layers[0], {**layers[1], name: layers[1][name] - eps * D}]
        fd = (objective(x, plus) - objective(x, minus)) / (2 * eps)
        assert fd == pytest.approx((grads[1][name] * D).sum().item(), rel=1e-6)


# -------------------------------------------------------- whole-model oracle --
def _model_params(gen, V, s, zero_word=False):
    word = torch.zeros(V, H, dtype=torch.float64) if zero_word else 0.5 * torch.randn(V, H, generator=gen, dtype=torch.float64)
    return {
        "word": word,
        "pos": torch.randn(s, H, generator=gen, dtype=torch.float64),
        "lnf_w": 1.0 + 0.1 * torch.randn(H, generator=gen, dtype=torch.float64),
        "lnf_b": 0.1 * torch.randn(H, generator=gen, dtype=torch.float64),
        "layers": [_layer_params(gen, zero_weights=zero_word)],
    }


def test_zero_tied_embedding_gives_log_vocab_and_the_closed_form_gradient():
    """A zero word embedding is a zero tied LM head: every logit is 0, each
    token's loss is ln V, and with labels = 0 (flex_ops.py:1962) the tied
    gradient is (1/V - [v = 0]) times the mask-weighted mean of the final
    hidden states; the embedding side contributes nothing (the head is
    zero), and neither does the position table."""
    gen = torch.Generator().manual_seed(10)
    V, s, b = 13, 6, 2
    params = _model_params(gen, V, s, zero_word=True)
    tokens = torch.randint(0, V, (b, s), generator=gen)
    positions = torch.arange(s).expand(b, s)
    mask = torch.tensor([[1, 0, 1, 1, 0, 1], [0, 1, 1, 1, 1, 0]], dtype=torch.float64)
    losses, mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, HEADS)
    assert torch.allclose(losses, torch.full((b, s), math.log(V), dtype=torch.float64), rtol=0, atol=1e-13)
    assert mean.item() == pytest.approx(math.log(V), rel=1e-14)
    # zero layer weights: the stack adds its output biases to pos[t]
    lp = params["layers"][0]
    x = params["pos"][positions] + lp["proj_b"] + lp["fc2_b"]  # [b, s, h]
    hidden = F.layer_norm(x, (H,), params["lnf_w"], params["lnf_b"], 1e-5)
    hbar = (hidden * mask.unsqueeze(-1)).sum((0, 1)) / mask.sum()
    coef = torch.full((V,), 1.0 / V, dtype=torch.float64)
    coef[0] -= 1.0
    assert torch.allclose(grads["word"], coef.unsqueeze(1) * hbar.unsqueeze(0), rtol=0, atol=1e-13)
    assert grads["pos"].abs().max().item() < 1e-14


def test_whole_model_gradients_are_the_directional_derivatives():
    """The masked mean loss against central differences: along the word
    table (moving the embedding and the tied head together, so the tied
    sum is what is checked), the position table and a layer weight."""
    gen = torch.Generator().manual_seed(11)
    V, s, b = 11, 5, 2
    params = _model_params(gen, V, s)
    tokens = torch.randint(0, V, (b, s), generator=gen)
    tokens[1, 2] = tokens[0, 1]  # a repeated token
    positions = torch.arange(s).expand(b, s)
    mask = (torch.rand(b, s, generator=gen) > 0.3).double()
    labels = torch.randint(0, V, (b, s), generator=gen)
    _, mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, HEADS, labels=labels)
    eps = 1e-6

    def mean_at(p):
        return ol.full_model_fwd_bwd(tokens, positions, mask, p, HEADS, labels=labels)[1].item()

    for name in ("word", "pos", "lnf_w"):
        D = torch.randn(params[name].shape, generator=gen, dtype=torch.float64)
        fd = (mean_at({**params, name: params[name] + eps * D}) - mean_at({**params, name: params[name] - eps * D})) / (2 * eps)
        assert fd == pytest.approx((grads[name] * D).sum().item(), rel=1e-6, abs=1e-12)
    lp = params["layers"][0]
    D = torch.randn(lp["fc1_w"].shape, generator=gen, dtype=torch.float64)
    plus = {**params, "layers": [{**lp, "fc1_w": lp["fc1_w"] + eps * D}]}
    minus = {**params, "layers": [{**lp, "fc1_w": lp["fc1_w"] - eps * D}]}
    fd = (mean_at(plus) - mean_at(minus)) / (2 * eps)
    assert fd == pytest.approx((grads["layers"][0]["fc1_w"] * D).sum().item(), rel=1e-6, abs=1e-12)


# --------------------------------------------------------- embedding backward --
def test_ordered_embedding_grad_equals_index_add():
    """Against torch's index_add in fp64 (the scatter-add the embedding
    backward is): exactly for small-integer gradients, to fp32 rounding
    otherwise; ids past the table are clamped; accumulates into the table."""
    import numpy as np

    gen = torch.Generator().manual_seed(12)
    s, b, h, V = 9, 3, 16, 7
    tok = torch.randint(0, V, (b, s), generator=gen)
    tok[0, 0] = V + 3  # clamped to V - 1
    pos = torch.arange(s).expand(b, s).contiguous()
    for dout in (torch.randint(-8, 9, (s, b, h), generator=gen).float(), torch.randn(s, b, h, generator=gen)):
        start = torch.randn(V, h, generator=gen)
        word = start.numpy().copy()
        posg = np.zeros((s, h), dtype=np.float32)
        ol.embedding_grad_ordered(tok.numpy(), pos.numpy(), dout.numpy(), word, posg)
        flat = dout.transpose(0, 1).reshape(-1, h).double()
        ref_w = start.double().index_add(0, tok.clamp(0, V - 1).reshape(-1), flat)
        ref_p = torch.zeros(s, h, dtype=torch.float64).index_add(0, pos.reshape(-1), flat)
        exact = dout.abs().max() <= 8 and float(dout.round().sub(dout).abs().max()) == 0.0
        tol = 0 if exact else 1e-5
        assert torch.allclose(torch.from_numpy(posg).double(), ref_p, rtol=0, atol=tol)
        if exact:
            # integers: the ordered fp32 sum is exact, so only the add into
            # the random start rounds
            assert torch.allclose(torch.from_numpy(word).double(), ref_w, rtol=2**-23, atol=0)
        else:
            assert torch.allclose(torch.from_numpy(word).double(), ref_w, rtol=0, atol=1e-5)


def test_chunked_ordered_embedding_grad_sums_every_chunk():
    """The chunked order (consecutive chunks of whole sequence positions):
    with small-integer gradients and zero tables every partial sum is
    exact, so any chunk size gives index_add exactly (a dropped or repeated
    chunk fails); a chunk covering the whole input is the unchunked order."""
    import numpy as np

    gen = torch.Generator().manual_seed(13)
    s, b, h, V = 11, 3, 8, 5
    tok = torch.randint(0, V, (b, s), generator=gen)
    pos = torch.arange(s).expand(b, s).contiguous()
    dout = torch.randint(-8, 9, (s, b, h), generator=gen).float()
    flat = dout.transpose(0, 1).reshape(-1, h).double()
    ref_w = torch.zeros(V, h, dtype=torch.float64).index_add(0, tok.reshape(-1), flat)
    ref_p = torch.zeros(s, h, dtype=torch.float64).index_add(0, pos.reshape(-1), flat)
    for chunk in (1, 3, 7, 12, 33, 1 << 20):
        word, posg = np.zeros((V, h), dtype=np.float32), np.zeros((s, h), dtype=np.float32)
        ol.embedding_grad_ordered(tok.numpy(), pos.numpy(), dout.numpy(), word, posg, chunk_rows=chunk)
        assert torch.equal(torch.from_numpy(word).double(), ref_w), chunk
        assert torch.equal(torch.from_numpy(posg).double(), ref_p), chunk
    # random gradients into a random table: one chunk over everything is the
    # default order bit for bit
    dout = torch.randn(s, b, h, generator=gen)
    start = torch.randn(V, h, generator=gen).numpy()
    a, c = start.copy(), start.copy()
    ol.embedding_grad_ordered(tok.numpy(), pos.numpy(), dout.numpy(), a, None)
    ol.embedding_grad_ordered(tok.numpy(), pos.numpy(), dout.numpy(), c, None, chunk_rows=s * b)
    assert np.array_equal(a, c)
