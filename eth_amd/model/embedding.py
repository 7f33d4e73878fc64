"""First- and last-stage vocabulary ops with the reference's op contract.

* `Embedding_v1` (op 0): word + position embeddings, dropout, [s, b, h]
  output (eth/runtime/megatron/model/flex_ops.py:365-485).
* `GPTPostProcess` (last op): logits = h @ E_head^T and the per-token
  vocab cross entropy (flex_ops.py:1908-1985).  The head keeps its own copy
  of the word embedding (`shared = True`, initialised from the root and
  kept equal by the tied-gradient sum).  Labels: the reference builds
  `torch.rand(b, s).long() * V`, which is always 0 (flex_ops.py:1962); that
  is the default here too, and an explicit `labels` side-channel tensor
  overrides it.
"""

import torch
from torch import nn

from .functional import BiasDropoutAddFn, CrossEntropyFn, EmbeddingFn, LinearFn
from .flex_ops import RopalaModule
from .layers import _param, init_method_normal, set_defaults_if_not_set_tensor_model_parallel_attributes, set_tensor_model_parallel_attributes


class VocabParallelEmbedding(nn.Module):
    """[V, h] table split along the vocabulary (TP = 1: whole)."""

    def __init__(self, num_embeddings, embedding_dim, init_method=None, dtype=torch.bfloat16, device="cuda", zero=False):
        super().__init__()
        self.num_embeddings, self.embedding_dim = num_embeddings, embedding_dim
        self.weight = _param((num_embeddings, embedding_dim), dtype, device, init=None if zero else init_method,
                             fill=0.0 if zero else None)
        set_tensor_model_parallel_attributes(self.weight, True, 0, 1)


class PositionEmbedding(nn.Module):
    def __init__(self, num_embeddings, embedding_dim, init_method, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.weight = _param((num_embeddings, embedding_dim), dtype, device, init=init_method)
        set_defaults_if_not_set_tensor_model_parallel_attributes(self.weight)


class Embedding_v1(RopalaModule):
    def __init__(self, op_index, cfg, init_method, name="encoder-embedding"):
        super().__init__(op_index, name)
        self.hidden_size = cfg.hidden_size
        self.word_embeddings = VocabParallelEmbedding(cfg.padded_vocab_size, cfg.hidden_size, init_method,
                                                      cfg.params_dtype, cfg.device)
        self.position_embeddings = PositionEmbedding(cfg.seq_length, cfg.hidden_size, init_method, cfg.params_dtype,
                                                     cfg.device)
        self.tokentype_embeddings = None
        self.embedding_dropout = cfg.hidden_dropout
        self.shared_weights_info = {"word_embeddings": {"root": True, "sharing_with_ops": [10 * cfg.num_layers + 2]}}
        self._bad = torch.zeros(1, dtype=torch.int32, device=cfg.device)
        # dropout stream: a fresh mask per call, replayed by that call's
        # backward (the seed travels with the autograd node)
        self._seed = (cfg.seed * 1000003 + 0x5EED + op_index) & (2**63 - 1)
        self._calls = 0

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        ids = input_tensors["enc_input_ids"]
        pos = input_tensors["enc_position_ids"]
        out = EmbeddingFn.apply(self.word_embeddings.weight, self.position_embeddings.weight, ids, pos, self._bad)
        if self.training and self.embedding_dropout > 0:
            zero = torch.zeros(out.shape[-1], dtype=out.dtype, device=out.device)
            seed = self._seed + 7919 * self._calls
            self._calls += 1
            out = BiasDropoutAddFn.apply(out, zero, torch.zeros_like(out), self.embedding_dropout, seed)
        return {"hidden_states": out}

    def check_ids(self):
        """Raise if any token / position id was outside its table (syncs)."""
        if int(self._bad.item()):
            raise IndexError("embedding index out of range")


class GPTPostProcess(RopalaModule):
    def __init__(self, op_index, cfg, name="gpt-post-process"):
        super().__init__(op_index, name)
        self.word_embeddings = VocabParallelEmbedding(cfg.padded_vocab_size, cfg.hidden_size, None, cfg.params_dtype,
                                                      cfg.device, zero=True)
        self.word_embeddings.weight.shared = True
        self.shared_weights_info = {"word_embeddings": {"root": False, "sharing_with_ops": [0]}}
        self.padded_vocab_size = cfg.padded_vocab_size
        self._bad = torch.zeros(1, dtype=torch.int32, device=cfg.device)

    def forward(self, input_tensors, input_extra_tensors, output_extra_tensors, profiling=False):
        lm_output = input_tensors["hidden_states"]  # [b, s, h] after final-layernorm
        labels = input_extra_tensors.get("labels")
        if labels is None:
            labels = torch.zeros(lm_output.shape[:2], dtype=torch.int64, device=lm_output.device)
        logits = LinearFn.apply(lm_output, self.word_embeddings.weight, None)
        return {"output": CrossEntropyFn.apply(logits, labels, self._bad)}


def gen_embedding_op(name, op_index, cfg):
    gen = torch.Generator().manual_seed(cfg.seed * 131 + op_index)
    init = init_method_normal(cfg.init_method_std, gen)
    if name == "encoder-embedding":
        return Embedding_v1(op_index, cfg, init)
    if name == "gpt-post-process":
        return GPTPostProcess(op_index, cfg)
    raise ValueError(f"unsupported vocabulary op {name!r}")
