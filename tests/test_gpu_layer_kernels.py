"""GPU parity of the layer kernels against the torch-CPU fp32 oracle on the
same 16-bit inputs.  Tolerances: outputs are rounded to bf16/fp16, so the
bar is a few units of the output dtype's rounding (2^-8 relative for bf16,
2^-11 for fp16) on top of fp32 accumulation-order noise."""

import pytest
import torch
import torch.nn.functional as F

from eth_amd import kernels as K
from oracle import layer as ol
from tests.conftest import announce

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


def _tol(dtype):
    return 2.0**-7 if dtype == torch.bfloat16 else 2.0**-10


def _close(out, ref, dtype, what, scale=None):
    out = out.float().cpu()
    ref = ref.float().cpu()
    scale = scale if scale is not None else ref.abs().max().item() + 1e-12
    err = (out - ref).abs().max().item()
    assert err <= _tol(dtype) * scale, f"{what}: max err {err:.3e} vs scale {scale:.3e}"


def _rand(shape, dtype, gen, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,Kd", [(256, 384, 128), (8, 16, 8), (200, 136, 72), (512, 512, 1024)])
def test_gemm_three_layouts(cuda, dtype, M, N, Kd):
    announce(f"gemm {dtype} {M}x{N}x{Kd}")
    gen = torch.Generator().manual_seed(M * 7 + N)
    x = _rand((M, Kd), dtype, gen)
    w = _rand((N, Kd), dtype, gen, 0.05)
    bias = _rand((N,), dtype, gen)
    dy = _rand((M, N), dtype, gen)
    xd, wd, bd, dyd = (t.to(cuda) for t in (x, w, bias, dy))
    # forward (A K-contiguous, B K-contiguous) with bias
    y = K.linear(xd, wd, bias=bd)
    ref = x.float() @ w.float().t() + bias.float()
    _close(y, ref, dtype, "fwd")
    # dgrad (B N-contiguous)
    dx = K.gemm(dyd, wd)
    _close(dx, dy.float() @ w.float(), dtype, "dgrad")
    # wgrad accumulate into fp32 (A M-contiguous, B N-contiguous)
    acc = torch.full((N, Kd), 0.5, dtype=torch.float32, device=cuda)
    K.gemm(dyd.t(), xd, out=acc, accumulate=True)
    ref = 0.5 + dy.float().t() @ x.float()
    err = (acc.cpu() - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item() + 1e-5, f"wgrad fp32 err {err}"
    # M-contiguous A with K-contiguous B
    z = K.gemm(xd.t().contiguous().t(), wd.t())
    _close(z, x.float() @ w.float().t(), dtype, "A col-major")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("a_k,b_k", [(True, True), (True, False), (False, False), (False, True)])
def test_gemm_pipelined_kernel_layouts(cuda, dtype, a_k, b_k):
    """Shapes that take the 256x256 pipelined kernel (>= 128 tiles of 256,
    K % 128 == 0) with ragged M and N: every operand layout, 16-bit output
    with bias, fp32 output, and fp32 accumulation with alpha."""
    M, N, Kd = 4000, 2056, 384  # 16 x 9 tiles, last row and column tiles partial
    announce(f"gemm256 {dtype} a_k={a_k} b_k={b_k} {M}x{N}x{Kd}")
    gen = torch.Generator().manual_seed(17 + 2 * a_k + b_k)
    a = _rand((M, Kd), dtype, gen)
    b = _rand((Kd, N), dtype, gen, 0.05)
    bias = _rand((N,), dtype, gen)
    ad = a.to(cuda) if a_k else a.t().contiguous().to(cuda).t()
    bd = b.t().contiguous().to(cuda).t() if b_k else b.to(cuda)
    ref = a.float() @ b.float()
    y = K.gemm(ad, bd, bias=bias.to(cuda))
    _close(y, ref + bias.float(), dtype, "16-bit out + bias")
    y32 = K.gemm(ad, bd, out_dtype=torch.float32)
    err = (y32.cpu() - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item(), f"fp32 out err {err}"
    acc = torch.full((M, N), 0.25, dtype=torch.float32, device=cuda)
    K.gemm(ad, bd, out=acc, accumulate=True, alpha=0.5)
    ref2 = 0.25 + 0.5 * ref
    err = (acc.cpu() - ref2).abs().max().item()
    assert err <= 1e-4 * ref2.abs().max().item(), f"accumulate err {err}"


@pytest.mark.parametrize("a_k,b_k", [(True, True), (True, False), (False, False), (False, True)])
def test_gemm_splitk_accumulate(cuda, a_k, b_k):
    """Small-grid fp32 accumulation (20 tiles of 256, K 4096) takes the
    split-K path: 4 k-splits into a workspace, added in order.  Matches the
    fp32 reference and is bit-identical run to run."""
    from eth_amd import _native as nat

    M, N, Kd = 1024, 1032, 4096
    assert K._splitk_splits(M, N, Kd, torch.empty(M, N, device=cuda)) == 4
    announce(f"gemm split-K a_k={a_k} b_k={b_k} {M}x{N}x{Kd}")
    gen = torch.Generator().manual_seed(23 + 2 * a_k + b_k)
    a = _rand((M, Kd), torch.bfloat16, gen)
    b = _rand((Kd, N), torch.bfloat16, gen, 0.05)
    ad = a.to(cuda) if a_k else a.t().contiguous().to(cuda).t()
    bd = b.t().contiguous().to(cuda).t() if b_k else b.to(cuda)
    ref = 0.25 + a.float() @ b.float()
    outs = []
    for _ in range(2):
        acc = torch.full((M, N), 0.25, dtype=torch.float32, device=cuda)
        K.gemm(ad, bd, out=acc, accumulate=True)
        outs.append(acc.cpu())
    err = (outs[0] - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item(), f"split-K err {err}"
    assert torch.equal(outs[0], outs[1])
    # store form (C = A B): the same partial sums, written over garbage
    st = torch.full((M, N), 9.0, dtype=torch.float32, device=cuda)
    K.gemm(ad, bd, out=st, accumulate=False)
    assert torch.equal(st.cpu() + 0.25, outs[0])  # one fp32 add of the same sum, either order
    # the single-pass kernel agrees to fp32 summation-order noise
    one = torch.full((M, N), 0.25, dtype=torch.float32, device=cuda)
    lda = ad.stride(0) if a_k else ad.stride(1)
    ldb = bd.stride(1) if b_k else bd.stride(0)
    nat.call("eth_gemm", nat.ptr(ad), lda, int(a_k), nat.ptr(bd), ldb, int(b_k), nat.ptr(one), N, nat.ETH_F32,
             None, M, N, Kd, nat.dtype_code(torch.bfloat16), nat.GEMM_ACCUMULATE, 1.0, nat.stream_ptr(cuda))
    assert (one.cpu() - outs[0]).abs().max().item() <= 1e-5 * ref.abs().max().item()


def test_gemm_rejects_bad_shapes(cuda):
    a = torch.zeros(16, 12, dtype=torch.bfloat16, device=cuda)
    b = torch.zeros(12, 16, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError):
        K.gemm(a, b)  # K = 12 is not a multiple of 8
    with pytest.raises(ValueError):
        K.gemm(a.float(), b.float())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(300, 256), (64, 2048), (33, 4096), (5, 8), (40, 1536), (17, 6144), (9, 8192)])
def test_layer_norm_fwd_bwd(cuda, dtype, rows, cols):
    announce(f"layernorm {dtype} {rows}x{cols}")
    gen = torch.Generator().manual_seed(rows + cols)
    x = _rand((rows, cols), dtype, gen, 2.0) + 0.5
    g = (1 + _rand((cols,), torch.float32, gen, 0.1)).to(dtype)
    b = _rand((cols,), dtype, gen, 0.1)
    dy = _rand((rows, cols), dtype, gen)
    y, mean, rstd = K.layer_norm_fwd(x.to(cuda), g.to(cuda), b.to(cuda))
    xr = x.float().requires_grad_(True)
    gr = g.float().requires_grad_(True)
    br = b.float().requires_grad_(True)
    ref = ol.layer_norm(xr, gr, br)
    _close(y, ref, dtype, "ln fwd")
    assert torch.allclose(mean.cpu(), x.float().mean(-1), atol=1e-4, rtol=1e-4)
    ref.backward(dy.float())
    dg = torch.full((cols,), 1.0, device=cuda)
    db = torch.zeros(cols, device=cuda)
    dx = K.layer_norm_bwd(dy.to(cuda), x.to(cuda), mean, rstd, g.to(cuda), dg, db, accumulate=True)
    _close(dx, xr.grad, dtype, "ln dx")
    assert torch.allclose(dg.cpu() - 1.0, gr.grad, rtol=1e-3, atol=1e-3 * gr.grad.abs().max().item())
    assert torch.allclose(db.cpu(), br.grad, rtol=1e-3, atol=1e-3 * br.grad.abs().max().item())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("seq,batch,cols", [(2048, 2, 4096), (37, 3, 1032), (64, 4, 2048), (5, 1, 8), (1, 7, 256)])
def test_transposed_layer_norm_equals_the_copy_then_layer_norm(cuda, dtype, seq, batch, cols):
    """The final LayerNorm with its [s, b, h] -> [b, s, h] transpose folded
    into the kernels (eth_ln_fwd_sb / eth_ln_bwd_sb) against
    .transpose(0, 1).contiguous() + eth_ln_fwd / eth_ln_bwd: y, mean, rstd,
    dx (transposed back) and the accumulated dgamma / dbeta bit for bit, and
    y against the fp32 oracle."""
    announce(f"transposed layernorm {dtype} s{seq} b{batch} h{cols}")
    gen = torch.Generator().manual_seed(seq * 7 + batch * 3 + cols)
    x = (_rand((seq, batch, cols), dtype, gen, 2.0) + 0.5).to(cuda)
    g = (1 + _rand((cols,), torch.float32, gen, 0.1)).to(dtype).to(cuda)
    b = _rand((cols,), dtype, gen, 0.1).to(cuda)
    dy = _rand((batch, seq, cols), dtype, gen).to(cuda)
    y1, m1, r1 = K.layer_norm_fwd_sb(x, g, b)
    xt = x.transpose(0, 1).contiguous()
    y2, m2, r2 = K.layer_norm_fwd(xt.view(-1, cols), g, b)
    assert torch.equal(y1.view(-1, cols), y2) and torch.equal(m1, m2) and torch.equal(r1, r2)
    _close(y1.cpu().view(-1, cols), ol.layer_norm(xt.float().cpu().view(-1, cols), g.float().cpu(), b.float().cpu()),
           dtype, "transposed ln fwd")
    outs = []
    for sb in (True, False):
        dg = torch.full((cols,), 0.5, device=cuda)
        db = torch.full((cols,), -0.25, device=cuda)
        if sb:
            dx = K.layer_norm_bwd_sb(dy, x, m1, r1, g, dg, db, accumulate=True)
        else:
            dx = K.layer_norm_bwd(dy.view(-1, cols), xt.view(-1, cols), m2, r2, g, dg, db, accumulate=True)
            dx = dx.view(batch, seq, cols).transpose(0, 1).contiguous()
        outs.append((dx, dg, db))
    for a, c in zip(*outs):
        assert torch.equal(a, c)
    with pytest.raises(ValueError):  # dy in the input's [s, b] order
        K.layer_norm_bwd_sb(dy.transpose(0, 1).contiguous(), x, m1, r1, g, dg, db, accumulate=False)
    with pytest.raises(ValueError):  # not a 3-D [s, b, h] input
        K.layer_norm_fwd_sb(x.view(-1, cols), g, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(300, 256), (1000, 2048), (2100, 1032), (33, 4096), (5, 8), (40, 1536), (17, 8192)])
def test_layer_norm_bwd_residual_colsum(cuda, dtype, rows, cols):
    """LayerNorm backward fused with the residual gradient: dx equals the
    plain backward's dx plus dresid, rounded as two 16-bit tensors and a
    16-bit add (bit-exact); dgamma/dbeta equal the plain path's to fp32
    summation-order noise; the column-sum partials fold to the fp32 column
    sums of the returned dx."""
    announce(f"layernorm residual {dtype} {rows}x{cols}")
    gen = torch.Generator().manual_seed(rows * 3 + cols)
    x = (_rand((rows, cols), dtype, gen, 2.0) + 0.5).to(cuda)
    g = (1 + _rand((cols,), torch.float32, gen, 0.1)).to(dtype).to(cuda)
    b = _rand((cols,), dtype, gen, 0.1).to(cuda)
    dy = _rand((rows, cols), dtype, gen).to(cuda)
    dres = _rand((rows, cols), dtype, gen).to(cuda)
    _, mean, rstd = K.layer_norm_fwd(x, g, b)
    dg0, db0 = torch.zeros(cols, device=cuda), torch.zeros(cols, device=cuda)
    dx0 = K.layer_norm_bwd(dy, x, mean, rstd, g, dg0, db0, accumulate=False)
    dg, db = torch.full((cols,), 2.0, device=cuda), torch.full((cols,), -1.0, device=cuda)
    dx, part = K.layer_norm_bwd(dy, x, mean, rstd, g, dg, db, accumulate=True, dresid=dres, colsum=True)
    assert torch.equal(dx.cpu(), (dx0 + dres).cpu())  # torch's 16-bit add: fp32 sum, one rounding
    scale = dg0.abs().max().item() + db0.abs().max().item()
    assert (dg - 2.0 - dg0).abs().max().item() <= 1e-5 * scale
    assert (db + 1.0 - db0).abs().max().item() <= 1e-5 * scale
    cs = torch.full((cols,), 0.5, device=cuda)
    K.reduce_partials(part, cs, accumulate=True)
    ref = 0.5 + dx.cpu().double().sum(0)
    assert (cs.cpu().double() - ref).abs().max().item() <= 1e-5 * (ref.abs().max().item() + rows)
    dx2 = K.layer_norm_bwd(dy, x, mean, rstd, g, dg0, db0, accumulate=False, dresid=dres)
    assert torch.equal(dx2.cpu(), dx.cpu())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(96, 1024), (1000, 8192), (37, 520), (3, 8)])
def test_bias_gelu_bwd_fused_dbias(cuda, dtype, rows, cols):
    """The fused bias gradient: dx bit-identical to the plain kernel, dbias
    the fp32 column sums of that dx (stored, then accumulated)."""
    announce(f"bias-gelu dbias {dtype} {rows}x{cols}")
    gen = torch.Generator().manual_seed(rows + 5 * cols)
    x = _rand((rows, cols), dtype, gen, 2.0).to(cuda)
    b = _rand((cols,), dtype, gen).to(cuda)
    dy = _rand((rows, cols), dtype, gen).to(cuda)
    dx0 = K.bias_gelu_bwd(dy, x, b)
    dbias = torch.full((cols,), 7.0, device=cuda)
    dx = K.bias_gelu_bwd(dy, x, b, dbias=dbias, accumulate=False)
    assert torch.equal(dx.cpu(), dx0.cpu())
    ref = dx0.cpu().double().sum(0)
    tol = 1e-5 * (ref.abs().max().item() + rows)
    assert (dbias.cpu().double() - ref).abs().max().item() <= tol
    K.bias_gelu_bwd(dy, x, b, dbias=dbias, accumulate=True)
    assert (dbias.cpu().double() - 2 * ref).abs().max().item() <= 2 * tol


@pytest.mark.parametrize("dtype", DTYPES)
def test_bias_gelu_fwd_bwd(cuda, dtype):
    announce(f"bias-gelu {dtype}")
    gen = torch.Generator().manual_seed(3)
    x = _rand((96, 1024), dtype, gen, 2.0)
    b = _rand((1024,), dtype, gen)
    dy = _rand((96, 1024), dtype, gen)
    y = K.bias_gelu_fwd(x.to(cuda), b.to(cuda))
    # reference rounds x + b to the activation dtype first (separate torch add)
    t = (x + b).float().requires_grad_(True)
    ref = F.gelu(t, approximate="tanh")
    _close(y, ref, dtype, "gelu fwd")
    ref.backward(dy.float())
    dx = K.bias_gelu_bwd(dy.to(cuda), x.to(cuda), b.to(cuda))
    _close(dx, t.grad, dtype, "gelu bwd")


@pytest.mark.parametrize("dtype", DTYPES)
def test_bias_dropout_add_and_col_sum(cuda, dtype):
    announce(f"bias-dropout-add {dtype}")
    gen = torch.Generator().manual_seed(4)
    x = _rand((130, 512), dtype, gen)
    b = _rand((512,), dtype, gen)
    r = _rand((130, 512), dtype, gen)
    out = K.bias_dropout_add_fwd(x.to(cuda), b.to(cuda), r.to(cuda), p=0.0)
    ref = (r + (x + b)).float()  # torch bf16 semantics: two rounded adds
    assert torch.equal(out.cpu().float(), ref)
    acc = torch.ones(512, device=cuda)
    K.col_sum(x.to(cuda), acc, accumulate=True)
    ref = 1.0 + x.float().sum(0)
    assert torch.allclose(acc.cpu(), ref, rtol=1e-5, atol=1e-4)
    # wide and ragged column sums (several 512-column strips, row groups)
    for rows, cols in ((8192, 6144), (4099, 1032), (7, 16)):
        xw = _rand((rows, cols), dtype, gen).to(cuda)
        out = torch.full((cols,), 3.0, device=cuda)
        K.col_sum(xw, out, accumulate=False)
        ref = xw.cpu().double().sum(0)
        assert (out.cpu().double() - ref).abs().max().item() <= 1e-5 * (ref.abs().max().item() + rows), (rows, cols)
    # dropout p=0.25: kept fraction, scaling, and backward uses the same mask
    outp = K.bias_dropout_add_fwd(x.to(cuda), b.to(cuda), torch.zeros_like(r).to(cuda), p=0.25, seed=123)
    kept = (outp.cpu().float() != 0)
    frac = kept.float().mean().item()
    assert 0.70 < frac < 0.80
    xb = (x + b).float()
    assert torch.allclose(outp.cpu().float()[kept], (xb * (1 / 0.75)).to(dtype).float()[kept], rtol=1e-2, atol=1e-2)
    dxp = K.dropout_bwd(torch.ones_like(x).to(cuda), 0.25, 123)
    keep_bwd = dxp.cpu().float() != 0
    assert torch.all(keep_bwd[kept])  # every element kept forward is kept backward
    assert 0.70 < keep_bwd.float().mean().item() < 0.80


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols,p", [(4099, 2048, 0.0), (300, 1032, 0.1), (33, 8192, 0.0), (5, 8, 0.3),
                                         (257, 4096, 0.1)])
def test_bias_dropout_add_layer_norm_matches_the_two_kernels(cuda, dtype, rows, cols, p):
    """eth_bda_ln_fwd against eth_bias_dropout_add_fwd followed by eth_ln_fwd
    on the same inputs: h, y, mean and rstd bit for bit (same dropout mask,
    same LayerNorm arithmetic on the stored h)."""
    announce(f"bias-dropout-add + LayerNorm fused, {dtype} {rows}x{cols} p={p}")
    gen = torch.Generator().manual_seed(rows + cols)
    x = _rand((rows, cols), dtype, gen).to(cuda)
    b = _rand((cols,), dtype, gen).to(cuda)
    r = _rand((rows, cols), dtype, gen).to(cuda)
    g = (1.0 + 0.1 * torch.randn(cols, generator=gen)).to(dtype).to(cuda)
    be = (0.1 * torch.randn(cols, generator=gen)).to(dtype).to(cuda)
    h, y, mean, rstd = K.bias_dropout_add_layer_norm_fwd(x, b, r, g, be, p=p, seed=77, eps=1e-5)
    h_ref = K.bias_dropout_add_fwd(x, b, r, p=p, seed=77)
    y_ref, mean_ref, rstd_ref = K.layer_norm_fwd(h_ref, g, be, 1e-5)
    assert torch.equal(h.view(torch.int16), h_ref.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(mean, mean_ref) and torch.equal(rstd, rstd_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 2047, 2049, 4096 * 3 + 7, (1 << 20) + 5])
def test_tied_grad_sum_ragged_lengths(cuda, dtype, n):
    """Both copies become root + copy, bit for bit against torch's sum (one
    rounding to the dtype), at lengths that leave a scalar tail, fill part of
    a workgroup or fit in one vector."""
    announce(f"tied grad sum n={n} {dtype}")
    g = torch.Generator(device=cuda).manual_seed(n)
    root = torch.randn(n, device=cuda, generator=g).to(dtype)
    copy = torch.randn(n, device=cuda, generator=g).to(dtype)
    want = (root.float() + copy.float()).to(dtype)
    K.tied_grad_sum(root, copy)
    assert torch.equal(root, want) and torch.equal(copy, want)
