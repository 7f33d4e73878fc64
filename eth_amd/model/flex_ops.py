"""GPT stage operators with the reference's dict-in / dict-out contract.

Each op is `forward(input_tensors, input_extra_tensors, output_extra_tensors,
profiling=False) -> dict`, exactly as the ops of
eth/runtime/megatron/model/flex_ops.py (contract :328), with the same op
names, op indices (1 + 10*layer + k), side-channel keys (`hidden_states_1`,
`hidden_states_2`, `value_layer`, `output_bias`) and parameter paths
(`input_layernorm`, `query_key_value`, `dense`) that the grad-sync adapter
resolves.  The arithmetic runs in the HIP kernels through the autograd
Functions of eth_amd.model.functional; TP = 1, so the reference's
resharding branches have no counterpart.
"""

from dataclasses import dataclass

import torch
from torch import nn

from .functional import (BiasDropoutAddFn, BiasDropoutAddLayerNormFn, BiasGeluFn, CausalAttentionFn, SplitQKVFn,
                         TransposedLayerNormFn)
from .layers import ColumnParallelLinear, LayerNorm, RowParallelLinear, init_method_normal


@dataclass
class GPTConfig:
    hidden_size: int
    num_attention_heads: int
    ffn_hidden_size: int
    num_layers: int
    seq_length: int
    micro_batch_size: int
    padded_vocab_size: int = 50304
    hidden_dropout: float = 0.0
    layernorm_epsilon: float = 1e-5
    init_method_std: float = 0.02
    scaled_output_init: bool = False  # sigma/sqrt(2L) for dense/fc2 (model/utils.py:32-39)
    params_dtype: torch.dtype = torch.bfloat16
    device: str = "cuda"
    seed: int = 1234

    @property
    def kv_channels(self):
        return self.hidden_size // self.num_attention_heads


LAYER_SCHEMA = (
    "enc-1st-layernorm",
    "enc-attention-qkv",
    "enc-flash-attention",
    "enc-attention-dense",
    "enc-post-attention-dropout",
    "enc-2nd-layernorm",
    "enc-MLP-GEMM-1",
    "enc-MLP-gelu",
    "enc-MLP-GEMM-2",
    "enc-post-MLP-dropout",
)


class RopalaModule(nn.Module):
    """Base of every stage op: index, name and side-channel bookkeeping."""

    def __init__(self, op_index, name, prev_name=None):
        super().__init__()
        self.op_index = op_index
        self.name = name
        self.prev_name = prev_name
        self.output_extra_tensors_info = {}
        self.tp_size = 1
        self.dp_size = 1

    def _publish(self, key, value, input_extra_tensors, output_extra_tensors):
        info = self.output_extra_tensors_info[key]
        if info.get("cross_stage", False):
            output_extra_tensors[key] = value
        input_extra_tensors[key] = value


class ParallelLayerNormOp(RopalaModule):
    """enc-1st-layernorm / enc-2nd-layernorm / final-layernorm
    (flex_ops.py:488-664)."""

    _EXTRA = {"enc-1st-layernorm": ("hidden_states_1", 4), "enc-2nd-layernorm": ("hidden_states_2", 4)}

    def __init__(self, op_index, name, cfg, prev_name=None):
        super().__init__(op_index, name, prev_name)
        self.input_layernorm = LayerNorm(cfg.hidden_size, eps=cfg.layernorm_epsilon, dtype=cfg.params_dtype,
                                         device=cfg.device)
        if name in self._EXTRA:
            key, send_to = self._EXTRA[name]
            self.output_extra_tensors_info = {key: {"send_to": send_to, "cross_stage": False}}

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        hidden = input_tensors["hidden_states"]
        if self.name == "final-layernorm" and not self.output_extra_tensors_info:
            # hidden.transpose(0, 1).contiguous() and the LayerNorm, the
            # [s, b, h] -> [b, s, h] permutation inside the LayerNorm kernels
            ln = self.input_layernorm
            return {"hidden_states": TransposedLayerNormFn.apply(hidden, ln.weight, ln.bias, ln.eps)}
        if self.name == "final-layernorm":
            hidden = hidden.transpose(0, 1).contiguous()
        if not self.output_extra_tensors_info:
            return {"hidden_states": self.input_layernorm(hidden)}
        out, residual = self.input_layernorm.forward_with_residual(hidden)
        for key in sorted(self.output_extra_tensors_info):
            self._publish(key, residual, input_extra_tensors, output_extra_tensors)
        return {"hidden_states": out}


class ParallelQKVOp(RopalaModule):
    """enc-attention-qkv: [s,b,h] -> [s,b,np,3hn] -> q, k, v per head
    (flex_ops.py:905-1142, split :1091-1103)."""

    def __init__(self, op_index, cfg, init_method, name="enc-attention-qkv", prev_name=None):
        super().__init__(op_index, name, prev_name)
        self.num_attention_heads_per_partition = cfg.num_attention_heads
        self.hidden_size_per_attention_head = cfg.kv_channels
        self.query_key_value = ColumnParallelLinear(cfg.hidden_size, 3 * cfg.hidden_size, bias=True,
                                                    init_method=init_method, dtype=cfg.params_dtype,
                                                    device=cfg.device)
        self.output_extra_tensors_info = {"value_layer": {"send_to": 1, "cross_stage": False}}

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        hidden = input_tensors["hidden_states"]
        mixed, _ = self.query_key_value(hidden)
        hn = self.hidden_size_per_attention_head
        mixed = mixed.view(*mixed.shape[:-1], self.num_attention_heads_per_partition, 3 * hn)
        q, k, v = SplitQKVFn.apply(mixed, hn)
        for key in sorted(self.output_extra_tensors_info):
            self._publish(key, v, input_extra_tensors, output_extra_tensors)
        return {"query_layer": q, "key_layer": k}


class ParallelFlashAtten(RopalaModule):
    """enc-flash-attention: causal SDPA (flex_ops.py:66-96,1377-1426)."""

    def __init__(self, op_index, name="enc-flash-attention", prev_name=None):
        super().__init__(op_index, name, prev_name)

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        v = input_extra_tensors["value_layer"] if profiling else input_extra_tensors.pop("value_layer")
        out = CausalAttentionFn.apply(input_tensors["query_layer"], input_tensors["key_layer"], v)
        return {"hidden_states": out}


class ParallelGEMM(RopalaModule):
    """enc-attention-dense / enc-MLP-GEMM-1 / enc-MLP-GEMM-2 with the bias
    returned separately (skip_bias_add) (flex_ops.py:1526-1632)."""

    def __init__(self, op_index, name, cfg, init_method, dim1_size, dim2_size, algo=0, prev_name=None):
        super().__init__(op_index, name, prev_name)
        rowish = name in ("enc-attention-dense", "enc-MLP-GEMM-2")
        self.algo = ("row" if algo == 0 else "column") if rowish else ("column" if algo == 0 else "row")
        cls = RowParallelLinear if self.algo == "row" else ColumnParallelLinear
        self.dense = cls(dim1_size, dim2_size, bias=True, init_method=init_method, skip_bias_add=True,
                         dtype=cfg.params_dtype, device=cfg.device)
        self.output_extra_tensors_info = {"output_bias": {"send_to": 1, "cross_stage": False}}

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        out, bias = self.dense(input_tensors["hidden_states"])
        for key in sorted(self.output_extra_tensors_info):
            self._publish(key, bias, input_extra_tensors, output_extra_tensors)
        return {"output_tensor": out}


class ParallelDropoutOp(RopalaModule):
    """enc-post-attention-dropout / enc-post-MLP-dropout: residual +
    dropout(x + bias) (flex_ops.py:1634-1847)."""

    def __init__(self, op_index, name, cfg, prev_name=None):
        super().__init__(op_index, name, prev_name)
        self.hidden_dropout = cfg.hidden_dropout
        self.residual_key = "hidden_states_1" if name == "enc-post-attention-dropout" else "hidden_states_2"
        self._seed = (cfg.seed * 1000003 + op_index) & (2**63 - 1)
        self._calls = 0
        # the LayerNorm op that takes this op's output next in the same stage,
        # when the stage runs the two back to back (set by the stage model,
        # outside the module registry)
        object.__setattr__(self, "fused_layernorm_op", None)

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        residual = input_extra_tensors[self.residual_key]
        bias = input_extra_tensors["output_bias"]
        p = self.hidden_dropout if self.training else 0.0
        seed = self._seed + 7919 * self._calls
        self._calls += 1
        ln_op = self.fused_layernorm_op
        if ln_op is not None and not profiling:
            # one pass also normalizes the output for the next op's LayerNorm,
            # which takes the result from the tensor
            ln = ln_op.input_layernorm
            out, y, mean, rstd = BiasDropoutAddLayerNormFn.apply(input_tensors["output_tensor"], bias, residual, p,
                                                                 seed, ln)
            out._eth_ln_fwd = (ln.weight, ln.bias, ln.eps, y, mean, rstd)
        else:
            out = BiasDropoutAddFn.apply(input_tensors["output_tensor"], bias, residual, p, seed)
        if not profiling:
            input_extra_tensors.pop("output_bias")
            input_extra_tensors.pop(self.residual_key)
        return {"hidden_states": out}


class ParallelMlpGeLUOp(RopalaModule):
    """enc-MLP-gelu: gelu_tanh(x + bias) (flex_ops.py:1849-1906)."""

    def __init__(self, op_index, name="enc-MLP-gelu", prev_name=None):
        super().__init__(op_index, name, prev_name)

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        bias = input_extra_tensors["output_bias"] if profiling else input_extra_tensors.pop("output_bias")
        return {"hidden_states": BiasGeluFn.apply(input_tensors["output_tensor"], bias)}


def gen_op(name, op_index, cfg, layer_index=None):
    """Instantiate the op for a manifest entry (flex_ops.py:140-236)."""
    gen = torch.Generator().manual_seed(cfg.seed * 131 + op_index)
    init = init_method_normal(cfg.init_method_std, gen)
    out_std = cfg.init_method_std / (2.0 * cfg.num_layers) ** 0.5 if cfg.scaled_output_init else cfg.init_method_std
    out_init = init_method_normal(out_std, gen)
    h, f = cfg.hidden_size, cfg.ffn_hidden_size
    if name in ("enc-1st-layernorm", "enc-2nd-layernorm", "final-layernorm"):
        return ParallelLayerNormOp(op_index, name, cfg)
    if name == "enc-attention-qkv":
        return ParallelQKVOp(op_index, cfg, init)
    if name == "enc-flash-attention":
        return ParallelFlashAtten(op_index)
    if name == "enc-attention-dense":
        return ParallelGEMM(op_index, name, cfg, out_init, h, h)
    if name == "enc-MLP-GEMM-1":
        return ParallelGEMM(op_index, name, cfg, init, h, f)
    if name == "enc-MLP-GEMM-2":
        return ParallelGEMM(op_index, name, cfg, out_init, f, h)
    if name in ("enc-post-attention-dropout", "enc-post-MLP-dropout"):
        return ParallelDropoutOp(op_index, name, cfg)
    if name == "enc-MLP-gelu":
        return ParallelMlpGeLUOp(op_index)
    raise ValueError(f"unsupported GPT op {name!r}")


def build_gpt_op_list(num_layers):
    """(name, op_index, layer_index) of the full GPT manifest
    (model/flex_gpt.py:23-43): embedding, 10 ops per layer, final LN, head."""
    ops = [("encoder-embedding", 0, None)]
    for layer in range(num_layers):
        for k, name in enumerate(LAYER_SCHEMA):
            ops.append((name, 1 + 10 * layer + k, layer))
    ops.append(("final-layernorm", 1 + 10 * num_layers, None))
    ops.append(("gpt-post-process", 2 + 10 * num_layers, None))
    return ops
