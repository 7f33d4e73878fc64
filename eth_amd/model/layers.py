"""Tensor-parallel layer modules at TP = 1 on the HIP kernels.

Same modules, parameter shapes and TP attributes as
eth/runtime/megatron/mpu/layers.py (ColumnParallelLinear :282-370,
RowParallelLinear :373-470, attribute helpers :49-84) and
model/fused_layer_norm.py (MixedFusedLayerNorm :62-89); the grad-sync
metadata adapter reads `tensor_model_parallel`, `partition_dim` and
`partition_stride` from every parameter.
"""

import torch
from torch import nn

from .functional import LayerNormFn, LayerNormResidualFn, LinearFn

_TP_ATTRS = {"tensor_model_parallel": False, "partition_dim": -1, "partition_stride": 1}


def set_tensor_model_parallel_attributes(tensor, is_parallel, dim, stride):
    tensor.tensor_model_parallel = is_parallel
    tensor.partition_dim = dim
    tensor.partition_stride = stride


def set_defaults_if_not_set_tensor_model_parallel_attributes(tensor):
    for attr, value in _TP_ATTRS.items():
        if not hasattr(tensor, attr):
            setattr(tensor, attr, value)


def _param(shape, dtype, device, init=None, fill=None):
    t = torch.empty(shape, dtype=torch.float32, device="cpu")
    if init is not None:
        init(t)
    elif fill is not None:
        t.fill_(fill)
    return nn.Parameter(t.to(device=device, dtype=dtype))


class LayerNorm(nn.Module):
    """MixedFusedLayerNorm: weight 1, bias 0, eps 1e-5 by default."""

    def __init__(self, normalized_shape, eps=1e-5, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.normalized_shape = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
        self.eps = eps
        self.weight = _param(self.normalized_shape, dtype, device, fill=1.0)
        self.bias = _param(self.normalized_shape, dtype, device, fill=0.0)
        for p in (self.weight, self.bias):
            set_defaults_if_not_set_tensor_model_parallel_attributes(p)

    def forward(self, x):
        return LayerNormFn.apply(x, self.weight, self.bias, self.eps)

    def forward_with_residual(self, x):
        """(LayerNorm(x), x) where the second output is the residual-branch
        copy of x: its gradient is added to the LayerNorm input gradient by
        the backward kernel."""
        return LayerNormResidualFn.apply(x, self.weight, self.bias, self.eps)


class ColumnParallelLinear(nn.Module):
    """Y = X A^T + b with A split along dim 0 (no split at TP=1)."""

    def __init__(self, input_size, output_size, bias=True, gather_output=False, init_method=None,
                 stride=1, skip_bias_add=False, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.input_size, self.output_size = input_size, output_size
        self.skip_bias_add = skip_bias_add
        self.weight = _param((output_size, input_size), dtype, device, init=init_method or nn.init.xavier_normal_)
        set_tensor_model_parallel_attributes(self.weight, True, 0, stride)
        if bias:
            self.bias = _param((output_size,), dtype, device, fill=0.0)
            set_tensor_model_parallel_attributes(self.bias, True, 0, stride)
        else:
            self.register_parameter("bias", None)

    def forward(self, x):
        bias = self.bias if not self.skip_bias_add else None
        out = LinearFn.apply(x, self.weight, bias)
        return out, (self.bias if self.skip_bias_add else None)


class RowParallelLinear(nn.Module):
    """Y = X A^T + b with A split along dim 1; the bias is replicated."""

    def __init__(self, input_size, output_size, bias=True, input_is_parallel=True, init_method=None,
                 stride=1, skip_bias_add=False, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.input_size, self.output_size = input_size, output_size
        self.skip_bias_add = skip_bias_add
        self.weight = _param((output_size, input_size), dtype, device, init=init_method or nn.init.xavier_normal_)
        set_tensor_model_parallel_attributes(self.weight, True, 1, stride)
        if bias:
            self.bias = _param((output_size,), dtype, device, fill=0.0)
            set_defaults_if_not_set_tensor_model_parallel_attributes(self.bias)
        else:
            self.register_parameter("bias", None)

    def forward(self, x):
        bias = self.bias if not self.skip_bias_add else None
        out = LinearFn.apply(x, self.weight, bias)
        return out, (self.bias if self.skip_bias_add else None)


def init_method_normal(sigma, generator=None):
    """N(0, sigma) (model/utils.py:24-29)."""

    def init_(tensor):
        return nn.init.normal_(tensor, mean=0.0, std=sigma, generator=generator)

    return init_
