"""Tensor-level wrappers over the C-ABI (include/eth_amd.h).

Each wrapper checks, on the host, that shapes, strides, dtypes and devices
match what the kernel and its launch grid assume, then enqueues the kernel on
the current stream.  There is no CPU fallback: CPU tensors raise.
"""

import ctypes

import numpy as np

import torch

from . import _native as nat

_HALF = (torch.bfloat16, torch.float16)


def _check_half(*ts):
    dt = ts[0].dtype
    if dt not in _HALF:
        raise ValueError(f"expected bf16/fp16 tensors, got {dt}")
    for t in ts:
        if t.dtype != dt:
            raise ValueError(f"dtype mismatch {t.dtype} vs {dt}")
        if not t.is_cuda:
            raise ValueError("eth_amd kernels run on the GPU only (no CPU fallback)")
    return nat.dtype_code(dt)


def _rows_cols(x):
    if not x.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    cols = x.shape[-1]
    return x.numel() // cols if cols else 0, cols


# --------------------------------------------------------------------- GEMM --
def _matrix_layout(t):
    """(ld, kcontig-ready) of a 2-D view: returns (ld, row_major) where
    row_major means t[i, j] = base[i*ld + j]; column-major views (t.T of a
    row-major matrix) give row_major False."""
    if t.dim() != 2:
        raise ValueError("expected a 2-D operand")
    s0, s1 = t.stride()
    if s1 == 1 and s0 >= t.shape[1]:
        return s0, True
    if s0 == 1 and s1 >= t.shape[0]:
        return s1, False
    raise ValueError(f"operand with strides {t.stride()} is neither row- nor column-major")


_observer = None


def set_kernel_observer(fn):
    """fn(kind, phase, flops) is called right before ("begin") and after
    ("end") every GEMM ("gemm") and attention ("attn_fwd", "attn_bwd")
    launch, on the thread that launches it, with the launch's algorithmic
    FLOPs (the benchmark records HIP events on the launch stream with it);
    None disables it."""
    global _observer
    _observer = fn


def _observe(kind, phase, flops):
    obs = _observer
    if obs is not None:
        obs(kind, phase, flops)


def _splitk_splits(M, N, K, out):
    """Split-K factor for an fp32 product whose 256x256 tile grid is too
    small to fill the chip (fewer than 128 tiles): enough k-splits for about
    one workgroup per CU, each split a multiple of 128 deep."""
    tiles = -(-M // 256) * -(-N // 256)
    if tiles >= 128 or N % 4 or out.stride(0) % 4 or out.data_ptr() % 16:
        return 1
    splits = 1
    while splits < 16 and tiles * splits * 2 <= 256 and K % (128 * splits * 2) == 0 and K // (splits * 2) >= 1024:
        splits *= 2
    return splits


_scratch = {}


def _scratch_f32(numel, device):
    """An fp32 workspace per (device, stream), reused across calls and grown
    on demand: launches on one stream are ordered, so they may share it."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    buf = _scratch.get(key)
    if buf is None or buf.numel() < numel:
        buf = torch.empty(numel, dtype=torch.float32, device=device)
        _scratch[key] = buf
    return buf[:numel]


_side = {}


def side_stream(device):
    """The stream the weight-gradient GEMMs run on when overlapped with the
    data-gradient chain (default priority, one per device)."""
    st = _side.get(device)
    if st is None:
        st = torch.cuda.Stream(device=device)
        _side[device] = st
    return st


def join_side_streams():
    """Make the current stream wait for all side-stream work (before main
    grads are read)."""
    for dev, st in _side.items():
        torch.cuda.current_stream(dev).wait_stream(st)


def gemm(a, b, out=None, bias=None, accumulate=False, out_dtype=None, alpha=1.0):
    """out (+)= alpha * a @ b (+ bias), a: [M, K], b: [K, N] (any row/column-
    major 2-D views), out: [M, N] row-major.  fp32 `out` with accumulate=True
    adds into it."""
    code = _check_half(a, b)
    M, K = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {a.shape} @ {b.shape}")
    lda, a_row = _matrix_layout(a)
    ldb, b_row = _matrix_layout(b)
    # A(m,k) K-contiguous <=> a row-major; B(k,n) K-contiguous <=> b column-major
    a_kcontig = 1 if a_row else 0
    b_kcontig = 0 if b_row else 1
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype or a.dtype, device=a.device)
    if out.dim() != 2 or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a row-major [M, N] matrix")
    if accumulate and out.dtype != torch.float32:
        raise ValueError("accumulate needs an fp32 output")
    flags = 0
    if accumulate:
        flags |= nat.GEMM_ACCUMULATE
    if bias is not None:
        if bias.dtype != a.dtype or bias.numel() != N or not bias.is_contiguous():
            raise ValueError("bias must be a contiguous [N] tensor of the input dtype")
        flags |= nat.GEMM_BIAS
    _observe("gemm", "begin", 2.0 * M * N * K)
    fp32_product = out.dtype == torch.float32 and alpha == 1.0 and bias is None
    splits = _splitk_splits(M, N, K, out) if fp32_product else 1
    if splits > 1:
        ws = _scratch_f32(nat.value("eth_gemm_splitk_workspace", M, N, splits) // 4, a.device)
        nat.call(
            "eth_gemm_splitk",
            nat.ptr(a), lda, a_kcontig,
            nat.ptr(b), ldb, b_kcontig,
            nat.ptr(out), out.stride(0), M, N, K, code, splits, 1 if accumulate else 0, nat.ptr(ws),
            nat.stream_ptr(a.device),
        )
        _observe("gemm", "end", 2.0 * M * N * K)
        return out
    nat.call(
        "eth_gemm",
        nat.ptr(a), lda, a_kcontig,
        nat.ptr(b), ldb, b_kcontig,
        nat.ptr(out), out.stride(0), nat.dtype_code(out.dtype),
        nat.ptr(bias), M, N, K, code, flags, float(alpha),
        nat.stream_ptr(a.device),
    )
    _observe("gemm", "end", 2.0 * M * N * K)
    return out


def linear(x2d, weight, bias=None):
    """F.linear: x2d [T, K] @ weight[N, K]^T (+ bias)."""
    return gemm(x2d, weight.t(), bias=bias)


# ---------------------------------------------------------------- LayerNorm --
def layer_norm_fwd(x, gamma, beta, eps=1e-5):
    code = _check_half(x, gamma, beta)
    rows, cols = _rows_cols(x)
    if gamma.numel() != cols or beta.numel() != cols:
        raise ValueError("gamma/beta must match the normalized size")
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    nat.call("eth_ln_fwd", nat.ptr(x), nat.ptr(gamma), nat.ptr(beta), nat.ptr(y), nat.ptr(mean), nat.ptr(rstd),
             rows, cols, float(eps), code, nat.stream_ptr(x.device))
    return y, mean, rstd


def layer_norm_fwd_sb(x, gamma, beta, eps=1e-5):
    """LayerNorm of a contiguous [s, b, h] x returned as [b, s, h] (the
    final LayerNorm after .transpose(0, 1).contiguous(), without the copy);
    mean / rstd in the output's row order."""
    code = _check_half(x, gamma, beta)
    if x.dim() != 3 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [s, b, h] tensor")
    s, b, h = x.shape
    if gamma.numel() != h or beta.numel() != h:
        raise ValueError("gamma/beta must match the normalized size")
    y = torch.empty(b, s, h, dtype=x.dtype, device=x.device)
    mean = torch.empty(b * s, dtype=torch.float32, device=x.device)
    rstd = torch.empty(b * s, dtype=torch.float32, device=x.device)
    nat.call("eth_ln_fwd_sb", nat.ptr(x), nat.ptr(gamma), nat.ptr(beta), nat.ptr(y), nat.ptr(mean), nat.ptr(rstd),
             s, b, h, float(eps), code, nat.stream_ptr(x.device))
    return y, mean, rstd


def layer_norm_bwd_sb(dy, x, mean, rstd, gamma, dgamma, dbeta, accumulate):
    """Backward of layer_norm_fwd_sb: dy [b, s, h], x [s, b, h] -> dx [s, b, h];
    dgamma/dbeta fp32 stored or accumulated in place."""
    code = _check_half(dy, x, gamma)
    if x.dim() != 3 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [s, b, h] tensor")
    s, b, h = x.shape
    if tuple(dy.shape) != (b, s, h) or not dy.is_contiguous():
        raise ValueError("dy must be a contiguous [b, s, h] tensor")
    for t in (dgamma, dbeta):
        if t.dtype != torch.float32 or t.numel() != h or not t.is_contiguous():
            raise ValueError("dgamma/dbeta must be contiguous fp32 [cols]")
    ws = torch.empty(nat.value("eth_ln_bwd_workspace", s * b, h), dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    nat.call("eth_ln_bwd_sb", nat.ptr(dy), nat.ptr(x), nat.ptr(mean), nat.ptr(rstd), nat.ptr(gamma), nat.ptr(dx),
             nat.ptr(dgamma), nat.ptr(dbeta), nat.ptr(ws), s, b, h, 1 if accumulate else 0, code,
             nat.stream_ptr(x.device))
    return dx


def layer_norm_bwd(dy, x, mean, rstd, gamma, dgamma, dbeta, accumulate, dresid=None, colsum=False):
    """dx (returned); dgamma/dbeta fp32 stored or accumulated in place.

    With `dresid` (the gradient of the residual branch that read the same x)
    the returned dx is bf16(bf16(dx_ln) + dresid).  With `colsum` as well,
    returns (dx, part): fp32 [groups, cols] column-sum partials of dx, folded
    by `reduce_partials` into a bias gradient."""
    code = _check_half(dy, x, gamma)
    rows, cols = _rows_cols(x)
    if dy.shape != x.shape or not dy.is_contiguous():
        raise ValueError("dy must match x")
    for t in (dgamma, dbeta):
        if t.dtype != torch.float32 or t.numel() != cols or not t.is_contiguous():
            raise ValueError("dgamma/dbeta must be contiguous fp32 [cols]")
    if dresid is not None:
        _check_half(dresid)
        if dresid.dtype != x.dtype or dresid.shape != x.shape or not dresid.is_contiguous():
            raise ValueError("dresid must be a contiguous tensor like x")
    elif colsum:
        raise ValueError("colsum needs dresid")
    ws = torch.empty(nat.value("eth_ln_bwd_workspace", rows, cols), dtype=torch.float32, device=x.device)
    part = None
    if colsum:
        part = torch.empty(nat.value("eth_ln_bwd_groups", rows, cols), cols, dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    nat.call("eth_ln_bwd_residual", nat.ptr(dy), nat.ptr(x), nat.ptr(mean), nat.ptr(rstd), nat.ptr(gamma),
             nat.ptr(dresid), nat.ptr(dx), nat.ptr(dgamma), nat.ptr(dbeta),
             nat.ptr(part), nat.ptr(ws), rows, cols, 1 if accumulate else 0, code,
             nat.stream_ptr(x.device))
    return (dx, part) if colsum else dx


def reduce_partials(part, out, accumulate):
    """out[c] (+)= sum_g part[g, c] (fp32), fixed summation order."""
    if part.dtype != torch.float32 or part.dim() != 2 or not part.is_contiguous():
        raise ValueError("part must be contiguous fp32 [groups, cols]")
    groups, cols = part.shape
    if out.dtype != torch.float32 or out.numel() != cols or not out.is_contiguous():
        raise ValueError("out must be contiguous fp32 [cols]")
    nat.call("eth_reduce_partials", nat.ptr(part), groups, cols, cols, nat.ptr(out), 1 if accumulate else 0,
             nat.stream_ptr(part.device))
    return out


# -------------------------------------------------------------- elementwise --
def bias_gelu_fwd(x, bias):
    code = _check_half(x, bias)
    rows, cols = _rows_cols(x)
    if bias.numel() != cols:
        raise ValueError("bias size mismatch")
    y = torch.empty_like(x)
    nat.call("eth_bias_gelu_fwd", nat.ptr(x), nat.ptr(bias), nat.ptr(y), rows, cols, code, nat.stream_ptr(x.device))
    return y


def bias_gelu_bwd(dy, x, bias, dbias=None, accumulate=False):
    """dx = dy * gelu_tanh'(x + b); with `dbias` (fp32 [cols]) the column
    sums of dx are stored or added into it in the same pass."""
    code = _check_half(dy, x, bias)
    rows, cols = _rows_cols(x)
    if dy.shape != x.shape or not dy.is_contiguous() or bias.numel() != cols:
        raise ValueError("shape mismatch")
    dx = torch.empty_like(x)
    if dbias is None:
        nat.call("eth_bias_gelu_bwd", nat.ptr(dy), nat.ptr(x), nat.ptr(bias), nat.ptr(dx), rows, cols, code,
                 nat.stream_ptr(x.device))
        return dx
    if dbias.dtype != torch.float32 or dbias.numel() != cols or not dbias.is_contiguous():
        raise ValueError("dbias must be contiguous fp32 [cols]")
    ws = torch.empty(nat.value("eth_bias_gelu_bwd_workspace", rows, cols), dtype=torch.float32, device=x.device)
    nat.call("eth_bias_gelu_bwd_dbias", nat.ptr(dy), nat.ptr(x), nat.ptr(bias), nat.ptr(dx), nat.ptr(dbias),
             nat.ptr(ws), rows, cols, 1 if accumulate else 0, code, nat.stream_ptr(x.device))
    return dx


def bias_dropout_add_fwd(x, bias, residual, p=0.0, seed=0):
    code = _check_half(x, bias, residual)
    rows, cols = _rows_cols(x)
    if residual.shape != x.shape or not residual.is_contiguous() or bias.numel() != cols:
        raise ValueError("shape mismatch")
    out = torch.empty_like(x)
    nat.call("eth_bias_dropout_add_fwd", nat.ptr(x), nat.ptr(bias), nat.ptr(residual), nat.ptr(out), rows, cols,
             float(p), int(seed) & (2**64 - 1), code, nat.stream_ptr(x.device))
    return out


def bias_dropout_add_layer_norm_fwd(x, bias, residual, gamma, beta, p=0.0, seed=0, eps=1e-5):
    """(h, y, mean, rstd): h = bias_dropout_add_fwd(x, bias, residual, p,
    seed) and (y, mean, rstd) = layer_norm_fwd(h, gamma, beta, eps), bit for
    bit, from one kernel that does not read h back."""
    code = _check_half(x, bias, residual, gamma, beta)
    rows, cols = _rows_cols(x)
    if residual.shape != x.shape or not residual.is_contiguous() or bias.numel() != cols:
        raise ValueError("shape mismatch")
    if gamma.numel() != cols or beta.numel() != cols:
        raise ValueError("gamma/beta must match the normalized size")
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    nat.call("eth_bda_ln_fwd", nat.ptr(x), nat.ptr(bias), nat.ptr(residual), nat.ptr(h), nat.ptr(gamma),
             nat.ptr(beta), nat.ptr(y), nat.ptr(mean), nat.ptr(rstd), rows, cols, float(p),
             int(seed) & (2**64 - 1), float(eps), code, nat.stream_ptr(x.device))
    return h, y, mean, rstd


def dropout_bwd(dy, p, seed):
    code = _check_half(dy)
    rows, cols = _rows_cols(dy)
    dx = torch.empty_like(dy)
    nat.call("eth_dropout_bwd", nat.ptr(dy), nat.ptr(dx), rows, cols, float(p), int(seed) & (2**64 - 1), code,
             nat.stream_ptr(dy.device))
    return dx


def col_sum(x, out, accumulate):
    """out[c] (+)= sum over rows of x[..., c] (fp32 out)."""
    code = _check_half(x)
    rows, cols = _rows_cols(x)
    if out.dtype != torch.float32 or out.numel() != cols or not out.is_contiguous():
        raise ValueError("out must be contiguous fp32 [cols]")
    ws = torch.empty(nat.value("eth_col_sum_workspace", rows, cols), dtype=torch.float32, device=x.device)
    nat.call("eth_col_sum", nat.ptr(x), cols, rows, cols, nat.ptr(out), nat.ptr(ws), 1 if accumulate else 0, code,
             nat.stream_ptr(x.device))
    return out


# ---------------------------------------------------------------- attention --
def _sbhd_strides(t):
    """(seq, batch, head) strides of a [s, b, np, hn] view with hn contiguous."""
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError("attention operands must be [s, b, np, hn] views with hn contiguous")
    return (t.stride(0), t.stride(1), t.stride(2))


def _attn_desc(q, dtype_code):
    s, b, n, d = q.shape
    desc = nat.AttnDesc()
    desc.batch, desc.heads, desc.seq, desc.head_dim, desc.dtype = b, n, s, d, dtype_code
    return desc


def attention_fwd(q, k, v, out=None):
    """Causal attention on [s, b, np, hn] views (any seq/batch/head strides).
    Returns (out [s, b, np, hn] view of a contiguous [s, b, np*hn], lse)."""
    code = _check_half(q, k, v)
    if not (q.shape == k.shape == v.shape):
        raise ValueError("q, k, v shapes differ")
    s, b, n, d = q.shape
    if d % 8 or not 8 <= d <= 128 or s < 1:
        raise ValueError(f"attention needs head_dim a multiple of 8 in [8, 128] and seq >= 1 (got {d}, {s})")
    if out is None:
        out = torch.empty(s, b, n * d, dtype=q.dtype, device=q.device)
    o4 = out.view(s, b, n, d)
    lse = torch.empty(b * n, s, dtype=torch.float32, device=q.device)
    desc = _attn_desc(q, code)
    desc.q_strides[:] = _sbhd_strides(q)
    desc.k_strides[:] = _sbhd_strides(k)
    desc.v_strides[:] = _sbhd_strides(v)
    desc.o_strides[:] = _sbhd_strides(o4)
    flops = 2.0 * b * n * s * s * d  # QK^T and PV over the causal half
    _observe("attn_fwd", "begin", flops)
    nat.call("eth_attn_fwd", ctypes.byref(desc), nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(o4), nat.ptr(lse),
             nat.stream_ptr(q.device))
    _observe("attn_fwd", "end", flops)
    return out, lse


def attention_bwd(q, k, v, out, dout, lse, dq, dk, dv):
    """Gradients of causal attention into dq/dk/dv ([s, b, np, hn] views, e.g.
    of one [s, b, np, 3*hn] buffer).  out/dout are [s, b, np*hn]."""
    code = _check_half(q, k, v, out, dout, dq, dk, dv)
    s, b, n, d = q.shape
    o4 = out.view(s, b, n, d)
    do4 = dout.reshape(s, b, n, d) if dout.is_contiguous() else None
    if do4 is None:
        raise ValueError("dout must be contiguous [s, b, np*hn]")
    if lse.shape != (b * n, s):
        raise ValueError("lse shape mismatch")
    delta = torch.empty(b * n, s, dtype=torch.float32, device=q.device)
    desc = _attn_desc(q, code)
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o4), ("do", do4), ("dq", dq), ("dk", dk), ("dv", dv)):
        if t.shape != q.shape:
            raise ValueError(f"{name} shape mismatch")
        getattr(desc, f"{name}_strides")[:] = _sbhd_strides(t)
    flops = 2.5 * 2.0 * b * n * s * s * d  # dS = dP, dQ, dK, dV: 2.5x the forward's products
    _observe("attn_bwd", "begin", flops)
    nat.call("eth_attn_bwd", ctypes.byref(desc), nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(o4), nat.ptr(do4),
             nat.ptr(lse), nat.ptr(delta), nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.stream_ptr(q.device))
    _observe("attn_bwd", "end", flops)


# --------------------------------------------------------------- vocabulary --
def _check_ids(t, shape=None):
    if t.dtype != torch.int64 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError("token / position ids must be contiguous int64 GPU tensors")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"ids shape {tuple(t.shape)} != {tuple(shape)}")


def embedding_fwd(tokens, positions, word, pos, bad_flag):
    """[b, s] ids -> [s, b, h] = word[tokens] + pos[positions] (16-bit)."""
    code = _check_half(word, pos)
    b, s = tokens.shape
    _check_ids(tokens)
    _check_ids(positions, (b, s))
    V, h = word.shape
    P, h2 = pos.shape
    if h != h2 or not word.is_contiguous() or not pos.is_contiguous():
        raise ValueError("embedding tables must be contiguous [rows, hidden] with equal hidden")
    out = torch.empty(s, b, h, dtype=word.dtype, device=word.device)
    nat.call("eth_embedding_fwd", nat.ptr(tokens), nat.ptr(positions), nat.ptr(word), nat.ptr(pos), nat.ptr(out),
             b, s, h, V, P, nat.ptr(bad_flag), code, nat.stream_ptr(word.device))
    return out


def embedding_bwd(tokens, positions, dout, dword, dpos):
    """fp32 dword[tokens] += dout and dpos[positions] += dout (dout [s, b, h]),
    bitwise deterministic (sorted ids, one owner per table row)."""
    code = _check_half(dout)
    b, s = tokens.shape
    _check_ids(tokens)
    _check_ids(positions, (b, s))
    if dout.shape[:2] != (s, b) or not dout.is_contiguous():
        raise ValueError("dout must be contiguous [s, b, h]")
    h = dout.shape[2]
    for t in (dword, dpos):
        if t is not None and (t.dtype != torch.float32 or t.shape[1] != h or not t.is_contiguous()):
            raise ValueError("embedding gradients must be contiguous fp32 [rows, hidden]")
    V = dword.shape[0] if dword is not None else 1
    P = dpos.shape[0] if dpos is not None else 1
    ws = _scratch_f32(-(-nat.value("eth_embedding_bwd_workspace", b, s) // 4), dout.device)
    nat.call("eth_embedding_bwd", nat.ptr(tokens), nat.ptr(positions), nat.ptr(dout), nat.ptr(dword), nat.ptr(dpos),
             nat.ptr(ws), b, s, h, V, P, code, nat.stream_ptr(dout.device))


def xent_fwd(logits2d, labels, bad_flag):
    """Per-row loss and lse (fp32) of 16-bit logits [rows, V]."""
    code = _check_half(logits2d)
    rows, V = logits2d.shape
    if logits2d.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    _check_ids(labels, (rows,))
    loss = torch.empty(rows, dtype=torch.float32, device=logits2d.device)
    lse = torch.empty(rows, dtype=torch.float32, device=logits2d.device)
    nat.call("eth_xent_fwd", nat.ptr(logits2d), logits2d.stride(0), nat.ptr(labels), nat.ptr(loss), nat.ptr(lse),
             rows, V, nat.ptr(bad_flag), code, nat.stream_ptr(logits2d.device))
    return loss, lse


def xent_bwd(logits2d, labels, lse, dloss):
    code = _check_half(logits2d)
    rows, V = logits2d.shape
    if dloss.dtype != torch.float32 or dloss.numel() != rows or not dloss.is_contiguous():
        raise ValueError("dloss must be contiguous fp32 [rows]")
    dz = torch.empty(rows, V, dtype=logits2d.dtype, device=logits2d.device)
    nat.call("eth_xent_bwd", nat.ptr(logits2d), logits2d.stride(0), nat.ptr(labels), nat.ptr(lse), nat.ptr(dloss),
             nat.ptr(dz), V, rows, V, code, nat.stream_ptr(logits2d.device))
    return dz


def synthetic_batch(sample_ids, seq, vocab, device):
    """tokens [b, s] int64, loss_mask [b, s] fp32, position_ids [b, s] int64
    of the deterministic synthetic batch, computed on the device in one
    launch per 64 samples (the ids cross as a host array)."""
    if isinstance(sample_ids, torch.Tensor):
        sample_ids = sample_ids.detach().cpu()  # the ids travel to the kernel by value
    ids = np.ascontiguousarray(np.asarray(sample_ids, dtype=np.int64).reshape(-1))
    b = ids.size
    if seq <= 0 or vocab <= 0:
        raise ValueError("sequence length and vocabulary size must be positive")
    tokens = torch.empty(b, seq, dtype=torch.int64, device=device)
    mask = torch.empty(b, seq, dtype=torch.float32, device=device)
    positions = torch.empty(b, seq, dtype=torch.int64, device=device)
    nat.require_cuda(tokens)
    nat.call("eth_synthetic_batch", ids.ctypes.data_as(ctypes.c_void_p), b, seq, vocab, nat.ptr(tokens),
             nat.ptr(mask), nat.ptr(positions), nat.stream_ptr(tokens.device))
    return tokens, mask, positions


def tied_grad_sum(root, copy):
    """root = copy = root + copy (main grads of a tied weight: fp32, or 16-bit
    with the sum rounded once to their dtype)."""
    if root.dtype != copy.dtype or root.shape != copy.shape:
        raise ValueError("tied gradients must be tensors of one dtype and shape")
    if not (root.is_contiguous() and copy.is_contiguous()):
        raise ValueError("tied gradients must be contiguous")
    if root.dtype == torch.float32:
        nat.call("eth_tied_grad_sum", nat.ptr(root), nat.ptr(copy), root.numel(), nat.stream_ptr(root.device))
    else:
        code = _check_half(root, copy)
        nat.call("eth_tied_grad_sum_half", nat.ptr(root), nat.ptr(copy), root.numel(), code,
                 nat.stream_ptr(root.device))
