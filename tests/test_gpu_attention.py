"""GPU parity of causal flash attention against F.scaled_dot_product_attention
(is_causal=True) computed in fp32 on the CPU from the same 16-bit inputs,
and of the SDPA oracle against an explicit softmax on tiny shapes.

Tolerance: the kernel rounds P and dS to the input dtype before the second
matrix product (as every flash-attention kernel does), so outputs are held
to 2^-7 (bf16) / 2^-9 (fp16) of the output's max magnitude and gradients to
2^-6 / 2^-8."""

import pytest
import torch

from eth_amd import kernels as K
from oracle import layer as ol
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _err(out, ref):
    out = out.float().cpu()
    ref = ref.float().cpu()
    return (out - ref).abs().max().item() / (ref.abs().max().item() + 1e-12)


def test_sdpa_oracle_matches_explicit_softmax():
    gen = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(16, 2, 2, 8, generator=gen, dtype=torch.float64) for _ in range(3))
    a = ol.causal_attention(q, k, v)
    b = ol.causal_attention_explicit(q, k, v)
    assert torch.allclose(a, b, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("s,b,n,d", [(128, 2, 2, 64), (256, 1, 3, 128), (384, 2, 1, 128), (512, 2, 2, 64),
                                     (768, 1, 2, 128),
                                     # ragged sequences and head dims on the padded kernels
                                     (200, 2, 2, 80), (77, 1, 3, 64), (130, 1, 2, 128), (96, 2, 1, 96),
                                     (300, 1, 2, 40), (64, 1, 1, 120)])
def test_attention_fwd_bwd_interleaved_qkv(cuda, dtype, s, b, n, d):
    announce(f"attention {dtype} s={s} b={b} n={n} d={d}")
    gen = torch.Generator().manual_seed(s + n + d)
    qkv = torch.randn(s, b, n, 3 * d, generator=gen).to(dtype)
    dout = torch.randn(s, b, n * d, generator=gen).to(dtype)
    qkv_d = qkv.to(cuda)
    q, k, v = torch.split(qkv_d, d, dim=-1)
    out, lse = K.attention_fwd(q, k, v)
    # reference in fp32 on CPU
    qr, kr, vr = (t.float().requires_grad_(True) for t in torch.split(qkv, d, dim=-1))
    ref = ol.causal_attention(qr, kr, vr)
    e = _err(out, ref)
    assert e < (2**-7 if dtype == torch.bfloat16 else 2**-9), f"fwd rel err {e}"
    ref.backward(dout.float())
    dqkv = torch.empty_like(qkv_d)
    dq, dk, dv = torch.split(dqkv, d, dim=-1)
    K.attention_bwd(q, k, v, out, dout.to(cuda), lse, dq, dk, dv)
    tol = 2**-6 if dtype == torch.bfloat16 else 2**-8
    for name, g, r in (("dq", dq, qr.grad), ("dk", dk, kr.grad), ("dv", dv, vr.grad)):
        e = _err(g, r)
        assert e < tol, f"{name} rel err {e}"


def test_attention_rejects_unsupported_shapes(cuda):
    x = torch.zeros(100, 1, 1, 100, dtype=torch.bfloat16, device=cuda)  # head_dim not a multiple of 8
    with pytest.raises(ValueError):
        K.attention_fwd(x, x, x)
    y = torch.zeros(128, 1, 1, 136, dtype=torch.bfloat16, device=cuda)  # head_dim above 128
    with pytest.raises(ValueError):
        K.attention_fwd(y, y, y)
