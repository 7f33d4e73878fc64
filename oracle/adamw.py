"""numpy restatement of torch.optim.AdamW's single-tensor step (test oracle).

The reference constructs apex FusedAdam and falls back to torch.optim.AdamW
(eth/runtime/megatron/optimizer/__init__.py:28-34,66-72); the closed form it
checks against is grad_sync/evidence.py:476-507.  The arithmetic below is
torch 2.x `_single_tensor_adam` with decoupled weight decay, with the
rounding of torch's CPU kernels (lerp and addcmul are fused multiply-adds,
addcdiv multiplies before dividing) and a correctly rounded sqrt (as CUDA's
and HIP's sqrtf are; torch's vectorized CPU sqrt is off by one ulp for
~0.6% of inputs, so parameters agree with torch CPU to ~1e-7 relative and
moments bit for bit).
"""

import math

import numpy as np


def fma(a, b, c):
    """Fused multiply-add, one rounding (exact product via float64 for fp32
    operands; plain arithmetic for fp64, where the difference is below the
    tests' tolerance)."""
    t = np.result_type(a, b, c)
    if t == np.float32:
        return (np.float64(a) * np.float64(b) + np.float64(c)).astype(np.float32)
    return a * b + c


def lerp(a, b, w):
    """torch CPU lerp: w < 0.5 ? fma(w, b-a, a) : fma(-(1-w), b-a, b)."""
    t = a.dtype.type
    d = b - a
    if w < 0.5:
        return fma(np.full_like(a, t(w)), d, a)
    return fma(np.full_like(a, -t(1.0 - w)), d, b)


def adamw_step(param, grad, exp_avg, exp_avg_sq, step, lr, beta1, beta2, eps, weight_decay, clip_coef=1.0):
    """One AdamW step; returns new (param, exp_avg, exp_avg_sq)."""
    t = param.dtype.type
    g = grad * t(clip_coef) if clip_coef < 1.0 else grad.copy()
    p = param * t(1.0 - lr * weight_decay) if weight_decay != 0 else param.copy()
    m = lerp(exp_avg, g, 1.0 - beta1)
    # exp_avg_sq.mul_(beta2).addcmul_(g, g, value=1-beta2): fma(value*g, g, v*beta2)
    v = fma(t(1.0 - beta2) * g, g, exp_avg_sq * t(beta2))
    bc1 = 1.0 - beta1**step
    bc2_sqrt = math.sqrt(1.0 - beta2**step)
    denom = np.sqrt(v) / t(bc2_sqrt) + t(eps)
    # param.addcdiv_(m, denom, value=-lr/bc1): p + (value*m)/denom
    p = p + (t(-lr / bc1) * m) / denom
    return p, m, v


def to_bf16(x):
    """fp32 -> bf16 (round to nearest even) returned as fp32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = r.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), r)
