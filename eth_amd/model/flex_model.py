"""Pipeline-stage container: the ops [op_start, op_end) of the GPT manifest,
run in order with the dict contract of
eth/runtime/megatron/model/flex_model.py:554-600 (FlexPipeModel.forward) and
model/flex_gpt.py:45-102 (FlexGPTModel).  Activation recompute is off in
every tracked reference config and is not provided."""

import torch
from torch import nn

from .flex_ops import GPTConfig, build_gpt_op_list, gen_op


class FlexPipeModel(nn.Module):
    def __init__(self, ops, pre_process, post_process):
        super().__init__()
        self.ops = nn.ModuleList(ops)
        self.num_ops = len(ops)
        self.pre_process = pre_process
        self.post_process = post_process
        self.input_tensor = None
        self._mark_cross_stage()

    def _mark_cross_stage(self):
        """An extra tensor crosses the stage when its consumer op is not here
        (flex_model.py:195-209)."""
        indices = {op.op_index for op in self.ops}
        for op in self.ops:
            for key, info in op.output_extra_tensors_info.items():
                info["cross_stage"] = op.op_index + info.get("send_to", 1) not in indices

    def set_input_tensor(self, input_tensor):
        self.input_tensor = input_tensor

    def forward(self, inputs, input_extra_tensors):
        output_extra_tensors = {}
        hidden = inputs if self.pre_process else self.input_tensor
        for op in self.ops:
            hidden = op(hidden, input_extra_tensors, output_extra_tensors)
        if self.post_process:
            return hidden
        return hidden, output_extra_tensors


class FlexGPTModel(nn.Module):
    """The ops of one pipeline stage of a GPT model."""

    def __init__(self, cfg: GPTConfig, op_start, op_end, pre_process=None, post_process=None):
        super().__init__()
        full = build_gpt_op_list(cfg.num_layers)
        if not 0 <= op_start < op_end <= len(full):
            raise ValueError(f"bad op range [{op_start}, {op_end}) for {len(full)} ops")
        ops = []
        for name, index, layer in full[op_start:op_end]:
            if name in ("encoder-embedding", "gpt-post-process"):
                from .embedding import gen_embedding_op

                ops.append(gen_embedding_op(name, index, cfg))
            else:
                ops.append(gen_op(name, index, cfg, layer))
        self.cfg = cfg
        self.op_start, self.op_end = op_start, op_end
        pre = op_start == 0 if pre_process is None else pre_process
        post = op_end == len(full) if post_process is None else post_process
        self.language_model = FlexPipeModel(ops, pre, post)

    def set_input_tensor(self, input_tensor):
        self.language_model.set_input_tensor(input_tensor)

    def forward(self, input_tensors, input_extra_tensors):
        return self.language_model(input_tensors, input_extra_tensors)


def middle_stage(cfg: GPTConfig, first_layer=0, num_layers=None):
    """Ops of `num_layers` whole transformer layers starting at `first_layer`
    (a middle pipeline stage: no embedding, no head)."""
    num_layers = cfg.num_layers - first_layer if num_layers is None else num_layers
    start = 1 + 10 * first_layer
    return FlexGPTModel(cfg, start, start + 10 * num_layers, pre_process=False, post_process=False)
