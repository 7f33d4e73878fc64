"""Pipeline-stage container: the ops [op_start, op_end) of the GPT manifest,
run in order with the dict contract of
eth/runtime/megatron/model/flex_model.py:554-600 (FlexPipeModel.forward) and
model/flex_gpt.py:45-102 (FlexGPTModel), with the optional activation
recompute of flex_model.py:395-535,564-588.

Stage boundaries may fall inside a transformer layer.  An op's side-channel
tensor (residual, value layer, output bias) whose consumer lies in a later
stage is marked cross-stage and returned in the stage's output extra
tensors; a stage whose first ops consume side-channel tensors of an earlier
stage receives them as input extra tensors (flex_model.py:63-240).

Recompute: `recompute_ops[i] == 1` puts op i into a checkpointed segment.
Consecutive flagged ops form one segment, cut before every
`enc-1st-layernorm` (the reference's breaking point, :575-580).  A segment's
forward runs without autograd and keeps only its inputs; its backward runs
the segment again with autograd and backpropagates through it.  Dropout ops
draw their masks from a per-op call counter, which the recompute rewinds, so
the recomputed forward is bit-identical to the first one.  Unlike the
reference, the side-channel tensors a segment leaves behind for later ops
(or later stages) are outputs of the checkpoint too, so their gradients
reach the segment.
"""

import torch
from torch import nn

from .flex_ops import GPTConfig, ParallelDropoutOp, ParallelLayerNormOp, build_gpt_op_list, gen_op

_SEGMENT_BREAK = "enc-1st-layernorm"


# a pending overlapped update of the parameters of op i + _UPDATE_LEAD is
# issued when op i is about to run: a layer's update then starts as the layer
# before it reaches its MLP products and overlaps GEMMs, not attention
_UPDATE_LEAD = 5


def launch_updates(op):
    """Issue the not yet launched parts of an overlapped update that write
    op's parameters (an optimizer step leaves `_eth_update_launch` on them)."""
    for p in op.parameters():
        launch = getattr(p, "_eth_update_launch", None)
        if launch is not None:
            launch()


def await_parameters(op):
    """Make the current stream wait for the pending update of op's
    parameters (an optimizer step overlapped with this forward leaves its
    events on them), once per update part: the wait clears the event from
    every parameter of the part, so later ops on the same stream (the
    forward's) do not queue it again (each queued wait costs the stream a
    few microseconds).  A part not launched yet is launched first, since a
    wait on an event not yet recorded waits for nothing."""
    for p in op.parameters():
        launch = getattr(p, "_eth_update_launch", None)
        if launch is not None:
            launch()
        ev = getattr(p, "_eth_ready_event", None)
        if ev is not None:
            torch.cuda.current_stream(p.device).wait_event(ev)
            for q in getattr(p, "_eth_ready_part", (p,)):
                q._eth_ready_event = None
            p._eth_ready_event = None


def _await_op(op):
    """await_parameters for op, and for the LayerNorm op whose forward it runs
    (a bias-dropout-add paired with the next LayerNorm reads its weights)."""
    await_parameters(op)
    ln_op = getattr(op, "fused_layernorm_op", None)
    if ln_op is not None:
        await_parameters(ln_op)


def _launch_op_updates(op):
    launch_updates(op)
    ln_op = getattr(op, "fused_layernorm_op", None)
    if ln_op is not None:
        launch_updates(ln_op)


def _rng_state(ops):
    return {id(op): op._calls for op in ops if hasattr(op, "_calls")}


def _set_rng_state(ops, state):
    for op in ops:
        if id(op) in state:
            op._calls = state[id(op)]


class _Segment:
    """Runs ops[start:end] of a stage on flattened tensors and returns every
    tensor the rest of the step can read: the hidden-state dict, the
    side-channel tensors left for later ops, and new cross-stage outputs."""

    def __init__(self, ops, hidden_keys, extra_keys):
        self.ops = ops
        self.hidden_keys = hidden_keys
        self.extra_keys = extra_keys
        self.out_layout = None  # (hidden keys, remaining extra keys, cross-stage keys)
        self.rng_before = None
        self.passthrough = {}

    def run(self, tensors):
        nh = len(self.hidden_keys)
        hidden = dict(zip(self.hidden_keys, tensors[:nh]))
        extras = dict(zip(self.extra_keys, tensors[nh:]))
        cross = {}
        for op in self.ops:
            await_parameters(op)
            hidden = op(hidden, extras, cross)
        layout = (tuple(sorted(hidden)), tuple(sorted(extras)), tuple(sorted(cross)))
        if self.out_layout is None:
            self.out_layout = layout
        elif layout != self.out_layout:
            raise RuntimeError("recomputed segment produced different tensors than its forward")
        return [hidden[k] for k in layout[0]] + [extras[k] for k in layout[1]] + [cross[k] for k in layout[2]]


class _Checkpoint(torch.autograd.Function):
    """Outputs are the segment's computed tensors only: tensors that leave
    the segment unchanged (an input passed on, or a parameter such as a
    linear's returned bias) are handed on as themselves by the caller, so
    their gradients keep their usual path (e.g. the fp32 main grad)."""

    @staticmethod
    def forward(ctx, segment, *tensors):
        segment.rng_before = _rng_state(segment.ops)
        with torch.no_grad():
            outs = segment.run(list(tensors))
        ctx.segment = segment
        ctx.needs = [t.requires_grad for t in tensors]
        ctx.save_for_backward(*tensors)
        # under no_grad only pre-existing tensors can require grad
        segment.passthrough = {i: o for i, o in enumerate(outs) if o.requires_grad or any(o is t for t in tensors)}
        stores = {t.untyped_storage().data_ptr() for t in tensors}
        computed = []
        for i, o in enumerate(outs):
            if i in segment.passthrough:
                continue
            # a view of an input (a published residual) must be its own
            # tensor for autograd
            computed.append(o.clone() if o.untyped_storage().data_ptr() in stores else o)
        return tuple(computed)

    @staticmethod
    def backward(ctx, *grads):
        seg = ctx.segment
        inputs = [t.detach().requires_grad_(need) for t, need in zip(ctx.saved_tensors, ctx.needs)]
        after = _rng_state(seg.ops)
        _set_rng_state(seg.ops, seg.rng_before)
        with torch.enable_grad():
            outs = seg.run(list(inputs))
        _set_rng_state(seg.ops, after)
        computed = [o for i, o in enumerate(outs) if i not in seg.passthrough]
        pairs = [(o, g) for o, g in zip(computed, grads) if g is not None and o.requires_grad]
        if pairs:
            torch.autograd.backward([o for o, _ in pairs], [g for _, g in pairs])
        return (None, *[t.grad if need else None for t, need in zip(inputs, ctx.needs)])


class FlexPipeModel(nn.Module):
    def __init__(self, ops, pre_process, post_process, recompute_ops=None):
        super().__init__()
        self.ops = nn.ModuleList(ops)
        self.num_ops = len(ops)
        self.pre_process = pre_process
        self.post_process = post_process
        self.input_tensor = None
        flags = list(recompute_ops) if recompute_ops is not None else [0] * self.num_ops
        if len(flags) != self.num_ops or any(f not in (0, 1) for f in flags):
            raise ValueError(f"recompute_ops must hold one 0/1 flag per op ({self.num_ops}), got {flags}")
        self.recompute_ops = flags
        self._mark_cross_stage()
        self._pair_dropout_layernorm()

    def _pair_dropout_layernorm(self):
        """A bias-dropout-add followed in this stage by a residual-publishing
        LayerNorm, neither in a checkpointed segment, runs as one kernel with
        it (BiasDropoutAddLayerNormFn); the LayerNorm op then takes the
        precomputed result.  Same values, bit for bit."""
        for i, op in enumerate(self.ops):
            if isinstance(op, ParallelDropoutOp):
                nxt = self.ops[i + 1] if i + 1 < self.num_ops else None
                fuse = (isinstance(nxt, ParallelLayerNormOp) and bool(nxt.output_extra_tensors_info)
                        and not self.recompute_ops[i] and not self.recompute_ops[i + 1])
                # a plain attribute, not a registered submodule: the LayerNorm's
                # parameters keep their one name in the module tree
                object.__setattr__(op, "fused_layernorm_op", nxt if fuse else None)

    def _mark_cross_stage(self):
        """An extra tensor crosses the stage when its consumer op is not here
        (flex_model.py:195-209)."""
        indices = {op.op_index for op in self.ops}
        for op in self.ops:
            for key, info in op.output_extra_tensors_info.items():
                info["cross_stage"] = op.op_index + info.get("send_to", 1) not in indices

    def set_input_tensor(self, input_tensor):
        self.input_tensor = input_tensor

    def segments(self):
        """[(start, end, checkpointed)] covering the ops in order."""
        out, i = [], 0
        while i < self.num_ops:
            if not self.recompute_ops[i]:
                out.append((i, i + 1, False))
                i += 1
                continue
            j = i + 1
            while j < self.num_ops and self.recompute_ops[j] and self.ops[j].name != _SEGMENT_BREAK:
                j += 1
            out.append((i, j, True))
            i = j
        return out

    def _checkpointed(self, start, end, hidden, input_extra_tensors, output_extra_tensors):
        hk, ek = tuple(sorted(hidden)), tuple(sorted(input_extra_tensors))
        seg = _Segment(list(self.ops[start:end]), hk, ek)
        flat = [hidden[k] for k in hk] + [input_extra_tensors[k] for k in ek]
        computed = iter(_Checkpoint.apply(seg, *flat))
        h_keys, e_keys, c_keys = seg.out_layout
        n_out = len(h_keys) + len(e_keys) + len(c_keys)
        outs = [seg.passthrough[i] if i in seg.passthrough else next(computed) for i in range(n_out)]
        n_h, n_e = len(h_keys), len(e_keys)
        input_extra_tensors.clear()
        input_extra_tensors.update(zip(e_keys, outs[n_h : n_h + n_e]))
        output_extra_tensors.update(zip(c_keys, outs[n_h + n_e :]))
        return dict(zip(h_keys, outs[:n_h]))

    def forward(self, inputs, input_extra_tensors):
        output_extra_tensors = {}
        hidden = inputs if self.pre_process else self.input_tensor
        ops = self.ops
        if not any(self.recompute_ops):
            for i, op in enumerate(ops):
                if i + _UPDATE_LEAD < len(ops):
                    _launch_op_updates(ops[i + _UPDATE_LEAD])
                _await_op(op)
                hidden = op(hidden, input_extra_tensors, output_extra_tensors)
        else:
            for start, end, ckpt in self.segments():
                if start + _UPDATE_LEAD < len(ops):
                    _launch_op_updates(ops[start + _UPDATE_LEAD])
                if ckpt:
                    hidden = self._checkpointed(start, end, hidden, input_extra_tensors, output_extra_tensors)
                else:
                    _await_op(self.ops[start])
                    hidden = self.ops[start](hidden, input_extra_tensors, output_extra_tensors)
        if self.post_process:
            return hidden
        return hidden, output_extra_tensors


class FlexGPTModel(nn.Module):
    """The ops of one pipeline stage of a GPT model."""

    def __init__(self, cfg: GPTConfig, op_start, op_end, pre_process=None, post_process=None, recompute_ops=None):
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
        self.language_model = FlexPipeModel(ops, pre, post, recompute_ops)

    def set_input_tensor(self, input_tensor):
        self.language_model.set_input_tensor(input_tensor)

    def forward(self, input_tensors, input_extra_tensors):
        return self.language_model(input_tensors, input_extra_tensors)


def middle_stage(cfg: GPTConfig, first_layer=0, num_layers=None, recompute_ops=None):
    """Ops of `num_layers` whole transformer layers starting at `first_layer`
    (a middle pipeline stage: no embedding, no head)."""
    num_layers = cfg.num_layers - first_layer if num_layers is None else num_layers
    start = 1 + 10 * first_layer
    return FlexGPTModel(cfg, start, start + 10 * num_layers, pre_process=False, post_process=False,
                        recompute_ops=recompute_ops)


def op_range_stage(cfg: GPTConfig, op_start, op_end, recompute_ops=None):
    """A middle stage holding manifest ops [op_start, op_end), which may
    begin or end inside a transformer layer."""
    return FlexGPTModel(cfg, op_start, op_end, pre_process=False, post_process=False, recompute_ops=recompute_ops)
