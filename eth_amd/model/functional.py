"""autograd Functions over the HIP kernels.

Weight and bias gradients follow the Megatron local-DDP contract
(eth/runtime/megatron/model/distributed.py:116-123): when a parameter has an
fp32 `main_grad` buffer, its gradient is accumulated straight into it by
the kernel (the wgrad GEMM adds into main_grad; bias / LayerNorm gradients
are reduced in fp32 and added), and the autograd gradient returned for the
parameter is None, so `param.grad` stays None.  Without `main_grad`, or with
a 16-bit one (fp16 training without fp32 accumulation, the reference's
default), the gradient is returned in the parameter's dtype -- rounded once
from its fp32 reduction -- and the DDP hook adds it into main_grad, a second
rounding, as the reference's `main_grad.add_(param.grad)` does.
"""

import torch

from .. import kernels as K
from .distributed import grad_written, main_grad_target, materialize_main_grad


_overlap = {"wgrad": False}


class overlapped_wgrad:
    """Within this context, LinearFn's weight-gradient GEMMs into main_grad
    run on a side stream, overlapped with the data-gradient chain; on exit
    the current stream waits for them, so main_grad is complete for
    whatever runs next."""

    def __enter__(self):
        self._prev = _overlap["wgrad"]
        _overlap["wgrad"] = True
        return self

    def __exit__(self, *exc):
        _overlap["wgrad"] = self._prev
        K.join_side_streams()
        return False



def _fp32_accum_target(param):
    """(main_grad, accumulate): the fp32 buffer the kernel writes param's
    gradient into, and whether it adds (False for the first contribution
    after a deferred zero_grad_buffer(), when it stores).  (None, False) when
    param has no fp32 main_grad: the gradient is then returned."""
    mg = getattr(param, "main_grad", None)
    if mg is None or mg.dtype != torch.float32:
        return None, False
    return main_grad_target(param)


def _pair_target(p1, p2):
    """(main_grad 1, main_grad 2, accumulate) for two gradients one kernel
    call writes under one accumulate flag (LayerNorm gamma and beta).  If
    only one of them is stale, that one is zeroed now and both accumulate;
    (None, None, False) unless both have a main_grad (stale flags are then
    left as they were)."""
    for p in (p1, p2):
        mg = getattr(p, "main_grad", None)
        if mg is None or mg.dtype != torch.float32:
            return None, None, False
    s1 = getattr(p1, "_eth_main_grad_stale", False)
    s2 = getattr(p2, "_eth_main_grad_stale", False)
    if s1 and s2:
        p1._eth_main_grad_stale = p2._eth_main_grad_stale = False
        return p1.main_grad, p2.main_grad, False
    return materialize_main_grad(p1), materialize_main_grad(p2), True


def _flat(x):
    return x.reshape(-1, x.shape[-1])


class LinearFn(torch.autograd.Function):
    """y = x @ W^T (+ b): ColumnParallelLinear / RowParallelLinear at TP=1."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        x2 = _flat(x.contiguous())
        y = K.gemm(x2, weight.t(), bias=bias)
        ctx.save_for_backward(x2, weight, bias)
        ctx.in_shape = x.shape
        return y.view(*x.shape[:-1], weight.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, weight, bias = ctx.saved_tensors
        dy2 = _flat(dy.contiguous())
        dx = K.gemm(dy2, weight).view(ctx.in_shape) if ctx.needs_input_grad[0] else None
        dw = db = None
        if ctx.needs_input_grad[1]:
            mg, accumulate = _fp32_accum_target(weight)
            if mg is not None and _overlap["wgrad"] and dy2.is_cuda:
                # the weight gradient only feeds main_grad: it runs on a side
                # stream, overlapped with the data-gradient chain, and is
                # joined before the gradient sync reads the buffer
                main = torch.cuda.current_stream(dy2.device)
                side = K.side_stream(dy2.device)
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    K.gemm(dy2.t(), x2, out=mg, accumulate=accumulate)
                dy2.record_stream(side)
                x2.record_stream(side)
                grad_written(weight)
            elif mg is not None:
                K.gemm(dy2.t(), x2, out=mg, accumulate=accumulate)
                grad_written(weight)
            else:
                # one rounding of the fp32 product to the parameter dtype
                dw = K.gemm(dy2.t(), x2, out_dtype=weight.dtype)
        if bias is not None and ctx.needs_input_grad[2]:
            mg, accumulate = _fp32_accum_target(bias)
            if mg is not None:
                K.col_sum(dy2, mg, accumulate=accumulate)
                grad_written(bias)
            else:
                acc = torch.empty(bias.shape, dtype=torch.float32, device=bias.device)
                K.col_sum(dy2, acc, accumulate=False)
                db = acc.to(bias.dtype)
        return dx, dw, db


class LayerNormFn(torch.autograd.Function):
    """MixedFusedLayerNorm (model/fused_layer_norm.py:30-89)."""

    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        xc = x.contiguous()
        y, mean, rstd = K.layer_norm_fwd(_flat(xc), gamma, beta, eps)
        ctx.save_for_backward(xc, gamma, beta, mean, rstd)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x, gamma, beta, mean, rstd = ctx.saved_tensors
        dg, db, acc = _pair_target(gamma, beta)
        own = dg is None
        if own:
            dg = torch.empty(gamma.shape, dtype=torch.float32, device=x.device)
            db = torch.empty(beta.shape, dtype=torch.float32, device=x.device)
        dx = K.layer_norm_bwd(_flat(dy.contiguous()), _flat(x), mean, rstd, gamma, dg, db, accumulate=acc)
        if not own:
            grad_written(gamma)
            grad_written(beta)
            return dx.view(x.shape), None, None, None
        return dx.view(x.shape), dg.to(gamma.dtype), db.to(beta.dtype), None


class TransposedLayerNormFn(torch.autograd.Function):
    """The final LayerNorm of the GPT stage, x.transpose(0, 1).contiguous()
    then MixedFusedLayerNorm (flex_ops.py final-layernorm, :552-553): [s, b, h]
    in, [b, s, h] out, with the row permutation done by the LayerNorm
    kernels' own reads and writes instead of two transposing copies."""

    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        xc = x.contiguous()
        y, mean, rstd = K.layer_norm_fwd_sb(xc, gamma, beta, eps)
        ctx.save_for_backward(xc, gamma, beta, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, gamma, beta, mean, rstd = ctx.saved_tensors
        dg, db, acc = _pair_target(gamma, beta)
        own = dg is None
        if own:
            dg = torch.empty(gamma.shape, dtype=torch.float32, device=x.device)
            db = torch.empty(beta.shape, dtype=torch.float32, device=x.device)
        dx = K.layer_norm_bwd_sb(dy.contiguous(), x, mean, rstd, gamma, dg, db, accumulate=acc)
        if not own:
            grad_written(gamma)
            grad_written(beta)
            return dx, None, None, None
        return dx, dg.to(gamma.dtype), db.to(beta.dtype), None


class LayerNormResidualFn(torch.autograd.Function):
    """MixedFusedLayerNorm whose input also feeds a later residual add:
    returns (LayerNorm(x), x).  The second output is what the op publishes
    as the residual (hidden_states_1/2, flex_ops.py:488-664), so both
    gradients of x arrive in one backward call and are added inside the
    LayerNorm backward kernel instead of by autograd's accumulation.  When x
    was produced by an op (not a leaf), the backward also leaves the
    column-sum partials of the returned gradient on it as
    `_eth_colsum_part`: BiasDropoutAddFn's backward folds them into its bias
    gradient instead of summing that gradient again."""

    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        ctx.set_materialize_grads(False)
        xc = x.contiguous()
        pre = getattr(x, "_eth_ln_fwd", None)
        if pre is not None:
            # the bias-dropout-add that made x already normalized it for this
            # LayerNorm (BiasDropoutAddLayerNormFn): taken once
            del x._eth_ln_fwd
        if pre is not None and pre[0] is gamma and pre[1] is beta and pre[2] == eps:
            y, mean, rstd = pre[3], pre[4], pre[5]
        else:
            y, mean, rstd = K.layer_norm_fwd(_flat(xc), gamma, beta, eps)
        ctx.save_for_backward(xc, gamma, beta, mean, rstd)
        ctx.colsum = x.grad_fn is not None
        return y.view(x.shape), x.view_as(x)

    @staticmethod
    def backward(ctx, dy, dres):
        x, gamma, beta, mean, rstd = ctx.saved_tensors
        if dy is None:
            return dres, None, None, None
        dg, db, acc = _pair_target(gamma, beta)
        own = dg is None
        if own:
            dg = torch.empty(gamma.shape, dtype=torch.float32, device=x.device)
            db = torch.empty(beta.shape, dtype=torch.float32, device=x.device)
        part = None
        if dres is None:
            dx = K.layer_norm_bwd(_flat(dy.contiguous()), _flat(x), mean, rstd, gamma, dg, db, accumulate=acc)
        else:
            out = K.layer_norm_bwd(_flat(dy.contiguous()), _flat(x), mean, rstd, gamma, dg, db, accumulate=acc,
                                   dresid=_flat(dres.contiguous()), colsum=ctx.colsum)
            dx, part = out if ctx.colsum else (out, None)
        dx = dx.view(x.shape)
        if part is not None:
            dx._eth_colsum_part = part
        if not own:
            grad_written(gamma)
            grad_written(beta)
            return dx, None, None, None
        return dx, dg.to(gamma.dtype), db.to(beta.dtype), None


class BiasGeluFn(torch.autograd.Function):
    """gelu_tanh(x + b) (flex_ops.py:1882-1906)."""

    @staticmethod
    def forward(ctx, x, bias):
        xc = x.contiguous()
        y = K.bias_gelu_fwd(_flat(xc), bias)
        ctx.save_for_backward(xc, bias)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x, bias = ctx.saved_tensors
        db = None
        if ctx.needs_input_grad[1]:
            # the bias gradient (column sums of dx) comes out of the same pass
            mg, accumulate = _fp32_accum_target(bias)
            target = mg if mg is not None else torch.empty(bias.shape, dtype=torch.float32, device=bias.device)
            dx = K.bias_gelu_bwd(_flat(dy.contiguous()), _flat(x), bias, dbias=target, accumulate=accumulate)
            if mg is None:
                db = target.to(bias.dtype)
            else:
                grad_written(bias)
        else:
            dx = K.bias_gelu_bwd(_flat(dy.contiguous()), _flat(x), bias)
        return dx.view(x.shape), db


class BiasDropoutAddFn(torch.autograd.Function):
    """residual + dropout(x + b, p) (flex_ops.py:104-134)."""

    @staticmethod
    def forward(ctx, x, bias, residual, p, seed):
        out = K.bias_dropout_add_fwd(_flat(x.contiguous()), bias, _flat(residual.contiguous()), p=p, seed=seed)
        ctx.p, ctx.seed = p, seed
        ctx.save_for_backward(bias)
        return out.view(x.shape)

    @staticmethod
    def backward(ctx, dout):
        return _bias_dropout_add_bwd(ctx, dout)


class BiasDropoutAddLayerNormFn(torch.autograd.Function):
    """BiasDropoutAddFn whose output the next op normalizes with `ln` (its
    LayerNorm module): one kernel also produces that LayerNorm's output,
    mean and rstd, returned as non-differentiable outputs for
    LayerNormResidualFn to take over, so the LayerNorm does not read h back.
    Gradients are BiasDropoutAddFn's; the LayerNorm keeps its own node."""

    @staticmethod
    def forward(ctx, x, bias, residual, p, seed, ln):
        # no zero tensors for the gradients of y, mean, rstd: they have none
        ctx.set_materialize_grads(False)
        h, y, mean, rstd = K.bias_dropout_add_layer_norm_fwd(
            _flat(x.contiguous()), bias, _flat(residual.contiguous()), ln.weight, ln.bias, p=p, seed=seed,
            eps=ln.eps)
        ctx.p, ctx.seed = p, seed
        ctx.save_for_backward(bias)
        ctx.mark_non_differentiable(y, mean, rstd)
        return h.view(x.shape), y.view(x.shape), mean, rstd

    @staticmethod
    def backward(ctx, dout, _dy, _dmean, _drstd):
        if dout is None:
            return None, None, None, None, None, None
        return (*_bias_dropout_add_bwd(ctx, dout), None)


def _bias_dropout_add_bwd(ctx, dout):
    """Gradients of residual + dropout(x + b) for (x, bias, residual, p, seed)."""
    (bias,) = ctx.saved_tensors
    part = getattr(dout, "_eth_colsum_part", None) if ctx.p == 0 else None
    dout = dout.contiguous()
    dx = K.dropout_bwd(_flat(dout), ctx.p, ctx.seed).view(dout.shape) if ctx.p > 0 else dout
    db = None
    if ctx.needs_input_grad[1]:
        mg, accumulate = _fp32_accum_target(bias)
        target = mg if mg is not None else torch.empty(bias.shape, dtype=torch.float32, device=bias.device)
        if part is not None:
            # column sums already produced by the LayerNorm backward that
            # made dout (p == 0: dx is dout)
            K.reduce_partials(part, target, accumulate=accumulate)
        else:
            K.col_sum(_flat(dx), target, accumulate=accumulate)
        if mg is None:
            db = target.to(bias.dtype)
        else:
            grad_written(bias)
    return dx, db, dout, None, None


class SplitQKVFn(torch.autograd.Function):
    """[s, b, np, 3*hn] -> q, k, v views (split_tensor_along_last_dim,
    mpu/utils.py:33-52) without copies.  When the incoming gradients are the
    three views of one [s, b, np, 3*hn] buffer (what attention's backward
    writes), that buffer is passed back as is."""

    @staticmethod
    def forward(ctx, mixed, hn):
        ctx.hn = hn
        ctx.shape = mixed.shape
        q, k, v = torch.split(mixed, hn, dim=-1)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        hn = ctx.hn
        base = getattr(dq, "_eth_qkv_base", None)
        if base is not None and dk is not None and dv is not None:
            return base, None
        out = torch.zeros(ctx.shape, dtype=(dq if dq is not None else dk).dtype, device=(dq if dq is not None else dk).device)
        for i, g in enumerate((dq, dk, dv)):
            if g is not None:
                out[..., i * hn : (i + 1) * hn].copy_(g)
        return out, None


class CausalAttentionFn(torch.autograd.Function):
    """softmax(QK^T/sqrt(hn) + causal) V on [s, b, np, hn] views -> [s, b, np*hn]."""

    @staticmethod
    def forward(ctx, q, k, v):
        out, lse = K.attention_fwd(q, k, v)
        ctx.save_for_backward(q, k, v, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        s, b, n, hn = q.shape
        dqkv = torch.empty(s, b, n, 3 * hn, dtype=q.dtype, device=q.device)
        dq, dk, dv = torch.split(dqkv, hn, dim=-1)
        K.attention_bwd(q, k, v, out, dout.contiguous(), lse, dq, dk, dv)
        dq._eth_qkv_base = dqkv
        return dq, dk, dv


class EmbeddingFn(torch.autograd.Function):
    """word[tokens] + pos[positions] -> [s, b, h] (Embedding_v1, dropout p = 0
    handled by the caller)."""

    @staticmethod
    def forward(ctx, word, pos, tokens, positions, bad_flag):
        out = K.embedding_fwd(tokens, positions, word, pos, bad_flag)
        ctx.save_for_backward(tokens, positions, word, pos)
        return out

    @staticmethod
    def backward(ctx, dout):
        tokens, positions, word, pos = ctx.saved_tensors
        # the scatter-add needs real values underneath: stale buffers are
        # zeroed first; 16-bit main grads receive the returned gradient
        # through the DDP hook
        def fp32_target(p):
            mg = getattr(p, "main_grad", None)
            return materialize_main_grad(p) if mg is not None and mg.dtype == torch.float32 else None

        mw, mp = fp32_target(word), fp32_target(pos)
        gw = mw if mw is not None else torch.zeros(word.shape, dtype=torch.float32, device=word.device)
        gp = mp if mp is not None else torch.zeros(pos.shape, dtype=torch.float32, device=pos.device)
        K.embedding_bwd(tokens, positions, dout.contiguous(), gw, gp)
        for p, m in ((word, mw), (pos, mp)):
            if m is not None:
                grad_written(p)
        return (None if mw is not None else gw.to(word.dtype), None if mp is not None else gp.to(pos.dtype), None,
                None, None)


class CrossEntropyFn(torch.autograd.Function):
    """Per-token loss of 16-bit logits [..., V] against int64 labels [...]
    (vocab_parallel_cross_entropy at TP = 1, computed in fp32)."""

    @staticmethod
    def forward(ctx, logits, labels, bad_flag):
        shape = logits.shape[:-1]
        z = logits.reshape(-1, logits.shape[-1])
        lab = labels.reshape(-1).contiguous()
        loss, lse = K.xent_fwd(z, lab, bad_flag)
        ctx.save_for_backward(z, lab, lse)
        ctx.shape = logits.shape
        return loss.view(shape)

    @staticmethod
    def backward(ctx, dloss):
        z, lab, lse = ctx.saved_tensors
        dz = K.xent_bwd(z, lab, lse, dloss.reshape(-1).float().contiguous())
        return dz.view(ctx.shape), None, None
