"""One ETH pipeline stage's training step on one GPU.

Wires the pieces the way eth/runtime/megatron/training.py:904-1068
(train_step) drives them for a stage that owns whole transformer layers:

    zero_grad_buffer()                       distributed.py:125
    forward over the stage's ops             flex_model.py:554-600
    backward from the upstream gradient      schedules.py:196-227
    GradientSyncManager.execute(scale)       grad_sync/manager.py:31-32
    optimizer.step() -> (ok, norm, zeros)    optimizer/optimizer.py:493-531

with the local-DDP main-grad buffer, the grad-sync plan built from the
stage's ops, and the fused unscale / flag / L2 statistics of the grad-sync
unpack bound to the optimizer.
"""

import dataclasses
import functools
import math

import torch

from .grad_sync.gpt_adapter import collect_stage_metadata
from .loss import global_normalization_scale, gpt_loss_output, sum_loss_outputs, synthetic_gpt_batch
from .grad_sync.executor import local_all_reduce_sum
from .grad_sync.manager import initialize_gradient_sync
from .grad_sync.streamed import StreamedGradSync
from .model.distributed import DistributedDataParallel
from .grad_sync.evidence import save_rank_snapshot
from .model.flex_model import FlexGPTModel, middle_stage, op_range_stage
from .model.functional import overlapped_wgrad
from .model.flex_ops import GPTConfig
from .optimizer.optimizer import get_megatron_optimizer


def save_stage_snapshot(trainer, output_dir, phase, iteration, metrics=None, clock=None, run_metadata=None):
    """Snapshot of a trainer's parameters, main grads and optimizer state
    with the reference's record layout (training.py:720-808 gathers the same
    three optimizer maps through the optimizer's model-parameter accessors)."""
    opt = trainer.optimizer
    # an overlapped update still pending is issued and waited for first
    opt.join_overlapped_update()
    loss_scale = float(opt.get_loss_scale().item())
    bindings = list(trainer.bindings)
    if phase == "post_sync" and opt.grads_unscaled_by_sync and loss_scale != 1.0:
        # The reference records post_sync before optimizer.step(), with the
        # main grads still loss-scaled (training.py:1005-1020); here the
        # sync's unpack has already unscaled them in place.  The scale is a
        # power of two, so multiplying back restores the scaled values
        # exactly (short of an fp32 overflow, which the step then flags).
        if loss_scale != 2.0 ** round(math.log2(loss_scale)):
            raise ValueError(f"post_sync evidence needs a power-of-two loss scale, got {loss_scale}")
        bindings = [dataclasses.replace(b, main_grad=b.main_grad * loss_scale) for b in bindings]
    state, master, hyper = {}, {}, {}
    for b in trainer.bindings:
        st = opt.state_for_model_parameter(b.parameter)
        state[b.logical_param_id] = {k: st[k] for k in ("step", "exp_avg", "exp_avg_sq") if k in st}
        master[b.logical_param_id] = opt.optimizer_parameter_for_model_parameter(b.parameter)
        hyper[b.logical_param_id] = opt.hyperparameters_for_model_parameter(b.parameter)
    base_clock = {"learning_rate": opt.param_groups[0]["lr"], "loss_scale": loss_scale}
    return save_rank_snapshot(
        output_dir,
        phase=phase,
        iteration=iteration,
        global_rank=getattr(trainer, "global_rank", 0),
        descriptors=trainer.descriptors,
        runtime_bindings=bindings,
        optimizer_state_by_logical=state,
        optimizer_parameter_by_logical=master,
        optimizer_hyperparameters_by_logical=hyper,
        clock={**base_clock, **(clock or {})},
        metrics=metrics,
        run_metadata=run_metadata,
    )


def _weight_to_host(weight):
    """Queue a copy of a loss weight (device scalar) into pinned host memory
    on the current stream; returns (host tensor [1], event after the copy)."""
    host = torch.empty(1, dtype=weight.dtype, pin_memory=True)
    host.copy_(weight.detach().reshape(1), non_blocking=True)
    ev = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(weight.device))
    return host, ev


def _fp32_main_grads(cfg, requested):
    """Whether main grads accumulate (and buckets travel) in fp32: always
    for bf16, as the reference forces (arguments.py:267-276); for fp16 as
    requested.  The trainers default to True for fp16 too -- the weight-
    gradient GEMM then adds straight into fp32, more accurate than the
    reference's default fp16 main grads -- and False gives the reference's
    default fp16 contract: fp16 main grads and bucket payloads, widened to
    fp32 by the optimizer before unscaling (optimizer.py:388-404)."""
    return True if cfg.params_dtype == torch.bfloat16 else bool(requested)


class MiddleStageTrainer:
    """A middle pipeline stage (no embedding, no head): whole layers
    `[first_layer, first_layer + num_layers)`, or any manifest op range
    `op_range = (op_start, op_end)` that may cut a layer.  `model` (a
    FlexGPTModel) replaces both; `resynced` names parameters whose main
    grads change after the sync (a tied word embedding)."""

    def __init__(
        self,
        cfg: GPTConfig,
        first_layer=0,
        num_layers=None,
        lr=1e-4,
        betas=(0.9, 0.95),
        eps=1e-8,
        weight_decay=0.1,
        clip_grad=1.0,
        sync_mode="block",
        bucket_cap_bytes=32 * 1024 * 1024,
        all_reduce_sum=None,
        op_range=None,
        recompute_ops=None,
        runtime_evidence_dir=None,
        overlap_optimizer=False,
        accumulate_allreduce_grads_in_fp32=True,
        model=None,
        initial_loss_scale=2.0**32,
        resynced=(),
        global_rank=0,
        defer_grad_sync=False,
    ):
        if cfg.params_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the stage trains in bf16 or fp16")
        fp32_grads = _fp32_main_grads(cfg, accumulate_allreduce_grads_in_fp32)
        self.cfg = cfg
        self.global_rank = global_rank
        if model is not None:
            self.model = model
        elif op_range is not None:
            self.model = op_range_stage(cfg, *op_range, recompute_ops=recompute_ops)
        else:
            self.model = middle_stage(cfg, first_layer, num_layers, recompute_ops=recompute_ops)
        self.ddp = DistributedDataParallel(self.model, accumulate_allreduce_grads_in_fp32=fp32_grads)
        lm = self.model.language_model
        self.descriptors, self.bindings = collect_stage_metadata(lm.ops, self.model.op_start, self.model.op_end,
                                                                 global_rank=global_rank)
        self._setup = dict(sync_mode=sync_mode, bucket_cap_bytes=bucket_cap_bytes, all_reduce_sum=all_reduce_sum,
                           runtime_evidence_dir=runtime_evidence_dir, lr=lr, weight_decay=weight_decay, betas=betas,
                           eps=eps, clip_grad=clip_grad, initial_loss_scale=initial_loss_scale, fp32_grads=fp32_grads,
                           resynced=list(resynced), overlap_optimizer=overlap_optimizer)
        if not defer_grad_sync:
            self.finish_setup()

    def finish_setup(self, all_gather_object=None):
        """The gradient-sync plan and the optimizer.  The plan covers the
        descriptors `all_gather_object(own descriptors)` returns -- those of
        every stage of a pipeline built in one process (a stage built alone
        plans from its own) -- and this stage runs its rank's share of it."""
        o = self._setup
        cfg = self.cfg
        gather = {} if all_gather_object is None else {"all_gather_object": all_gather_object}
        self.grad_sync = initialize_gradient_sync(
            self.descriptors,
            self.bindings,
            global_rank=self.global_rank,
            expected_pipeline_ids=(0,),
            sync_mode=o["sync_mode"],
            bucket_cap_bytes=o["bucket_cap_bytes"],
            all_reduce_sum=o["all_reduce_sum"] or local_all_reduce_sum,
            runtime_evidence_dir=o["runtime_evidence_dir"],
            **gather,
        )
        self.optimizer = get_megatron_optimizer(
            [self.model],
            lr=o["lr"],
            weight_decay=o["weight_decay"],
            betas=o["betas"],
            eps=o["eps"],
            clip_grad=o["clip_grad"],
            bf16=cfg.params_dtype == torch.bfloat16,
            fp16=cfg.params_dtype == torch.float16,
            initial_loss_scale=o["initial_loss_scale"],
        )
        # (16-bit main grads are widened and unscaled by the optimizer; a
        # re-synced tied gradient is unscaled addend by addend by the sync,
        # exact only for a power-of-two loss scale)
        if o["fp32_grads"] and (not o["resynced"] or math.frexp(o["initial_loss_scale"])[0] == 0.5):
            self.optimizer.bind_gradient_sync(self.grad_sync.executor, resynced=o["resynced"])
        if o["overlap_optimizer"]:
            self.optimizer.overlap_with_next_forward(update_parts(self.model.language_model.ops))
        # buckets synced during the backward, as soon as their gradients
        # exist (train_step(streamed_sync=True))
        self._streamed = None
        dev = next(self.model.parameters()).device
        if dev.type == "cuda":
            self._streamed = StreamedGradSync(self.grad_sync.executor, dev)

    # ------------------------------------------------ stage dict contract --
    def forward_step(self, input_tensors, input_extra_tensors=None):
        """Forward of one microbatch with the stage's dict I/O
        (schedules.py:62-111, flex_model.py:554-600): `input_tensors` as the
        previous stage sends them ({"hidden_states": [s, b, h]}) and the
        side-channel tensors of ops in earlier stages this stage consumes.
        Returns (outputs, output_extra_tensors, leaves); `leaves` are this
        stage's own copies of the inputs, which collect the input gradients."""
        ins = {k: v.detach().requires_grad_(True) for k, v in input_tensors.items()}
        extras = {
            k: v.detach().requires_grad_(v.is_floating_point()) for k, v in (input_extra_tensors or {}).items()
        }
        self.model.set_input_tensor(ins)
        out, out_extra = self.model(None, dict(extras))
        return out, out_extra, (ins, extras)

    def backward_step(self, outputs, output_grads, output_extra_tensors=None, output_extra_grads=None, leaves=None):
        """Backward of one microbatch (schedules.py:196-227): the upstream
        gradients of the outputs and of the cross-stage side-channel outputs
        enter one autograd pass (weight gradients into the fp32 main grads);
        returns the gradients of the inputs and of the input side-channel
        tensors, zeros where nothing flowed (schedules.py:151-172).

        The reference assigns the side-channel gradients to `.grad` of its
        outputs (schedules.py:113-117), which autograd does not read for a
        tensor that is not a leaf; here they are backpropagated, so a stage
        cut inside a layer gives the gradients of the uncut model."""
        tensors, grads = [], []
        for key in sorted(outputs):
            tensors.append(outputs[key])
            grads.append(output_grads[key])
        for key in sorted(output_extra_tensors or {}):
            g = (output_extra_grads or {}).get(key)
            t = output_extra_tensors[key]
            if g is not None and t.requires_grad:
                tensors.append(t)
                grads.append(g)
        with overlapped_wgrad():
            torch.autograd.backward(tensors, grads)
        ins, extras = leaves if leaves is not None else ({}, {})
        zero = lambda t: t.grad if t.grad is not None else torch.zeros_like(t)  # noqa: E731
        return {k: zero(t) for k, t in ins.items()}, {k: zero(t) for k, t in extras.items() if t.is_floating_point()}

    def train_step_microbatches(self, microbatches, normalization_scale=1.0):
        """forward_backward_no_pipelining (schedules.py:236-281) and the rest
        of train_step for this stage: every microbatch's forward and
        backward, main grads accumulating across them (the first
        contribution after the deferred zeroing stores, the rest add), then
        one gradient sync and one optimizer step.

        Each microbatch is a dict with `input_tensors`, `output_grads` and
        optionally `input_extra_tensors` / `output_extra_grads`.  Returns
        ([(outputs, output_extra_tensors, input_grads, input_extra_grads)],
        update_successful, grad_norm)."""
        if hasattr(normalization_scale, "item"):
            normalization_scale = float(normalization_scale.item())
        self.ddp.zero_grad_buffer(defer=True)
        results = []
        # (the forwards below wait for an overlapped update layer by layer)
        for mb in microbatches:
            out, out_extra, leaves = self.forward_step(mb["input_tensors"], mb.get("input_extra_tensors"))
            in_g, extra_g = self.backward_step(out, mb["output_grads"], out_extra, mb.get("output_extra_grads"),
                                               leaves)
            results.append(({k: v.detach() for k, v in out.items()}, {k: v.detach() for k, v in out_extra.items()},
                            in_g, extra_g))
        self.optimizer.join_overlapped_update()
        self.ddp.settle_grad_buffer()
        self.grad_sync.execute(normalization_scale)
        ok, norm, _zeros = self.optimizer.step()
        return results, ok, norm

    # --------------------------------------------- single-microbatch path --
    def forward_backward(self, x, dy):
        """Forward the stage on activations x [s, b, h] and backpropagate the
        upstream gradient dy; returns (output, input gradient)."""
        x = x.detach().requires_grad_(True)
        self.model.set_input_tensor({"hidden_states": x})
        out, _extra = self.model(None, {})
        hidden = out["hidden_states"]
        with overlapped_wgrad():
            torch.autograd.backward(hidden, dy)
        return hidden.detach(), x.grad

    def train_step(self, x, dy, normalization_scale=1.0, streamed_sync=False):
        """One step over one microbatch.  With streamed_sync each gradient
        bucket is packed / all-reduced / unpacked as soon as the backward has
        written it, overlapped with the rest of the backward; otherwise (the
        default) the whole sync runs after it, as in the reference.  Both
        give identical results.  On one GPU the all-reduce seam moves no
        data, and the overlapped pack/unpack slows the backward's GEMMs by
        about as much as it hides (measured 413 K vs 417-420 K tokens/s), so
        the overlap is for deployments whose seam does real communication."""
        if hasattr(normalization_scale, "item"):
            normalization_scale = float(normalization_scale.item())
        # deferred: the first gradient written into each main_grad stores
        self.ddp.zero_grad_buffer(defer=True)
        streamed = streamed_sync and self._streamed is not None
        if streamed:
            # the sync resets the statistics the previous update reads
            self.optimizer.join_overlapped_update()
            self._streamed.start(normalization_scale)
            try:
                out, dx = self.forward_backward(x, dy)
            finally:
                self._streamed.finish()
            self.ddp.settle_grad_buffer()
        else:
            out, dx = self.forward_backward(x, dy)
            self.optimizer.join_overlapped_update()
            self.ddp.settle_grad_buffer()
            self.grad_sync.execute(normalization_scale)
        ok, norm, zeros = self.optimizer.step()
        return out, dx, ok, norm

    # ---------------------------------------------------------- evidence --
    def record_evidence(self, output_dir, phase, iteration, metrics=None, clock=None, run_metadata=None):
        """Write this rank's numerical snapshot (grad_sync/evidence.py layout,
        training.py:720-808) for `phase` in init / pre_sync / post_sync /
        post_step."""
        return save_stage_snapshot(self, output_dir, phase, iteration, metrics, clock, run_metadata)

    def layer_parameters(self):
        """[{oracle name: parameter}] per layer, in layer order."""
        names = {
            "enc-1st-layernorm": (("input_layernorm.weight", "ln1_w"), ("input_layernorm.bias", "ln1_b")),
            "enc-attention-qkv": (("query_key_value.weight", "qkv_w"), ("query_key_value.bias", "qkv_b")),
            "enc-attention-dense": (("dense.weight", "proj_w"), ("dense.bias", "proj_b")),
            "enc-2nd-layernorm": (("input_layernorm.weight", "ln2_w"), ("input_layernorm.bias", "ln2_b")),
            "enc-MLP-GEMM-1": (("dense.weight", "fc1_w"), ("dense.bias", "fc1_b")),
            "enc-MLP-GEMM-2": (("dense.weight", "fc2_w"), ("dense.bias", "fc2_b")),
        }
        layers = {}
        for op in self.model.language_model.ops:
            if op.name not in names:
                continue
            layer = layers.setdefault((op.op_index - 1) // 10, {})
            for path, key in names[op.name]:
                obj = op
                for part in path.split("."):
                    obj = getattr(obj, part)
                layer[key] = obj
        return [layers[k] for k in sorted(layers)]


def update_parts(ops):
    """Parameters of a stage's ops in the parts an overlapped AdamW update
    launches, in the order the next forward reads them: one part per
    transformer layer (ops before the first layer, such as the embedding,
    form one part; ops after the last, such as the final LayerNorm and the
    LM head, belong to the last layer's index and form the last part).  A
    LayerNorm whose forward runs inside the preceding bias-dropout-add (the
    next layer's first LayerNorm) updates with that op's layer, so the fused
    kernel waits for no later part.  The first transformer layer updates in
    two parts, its attention half (ops 1-6 of the layer) and its MLP half,
    so that only the first precedes its forward and the second runs under
    its attention."""
    runs_in = {}
    for op in ops:
        ln_op = getattr(op, "fused_layernorm_op", None)
        if ln_op is not None:
            runs_in[id(ln_op)] = op
    layers = [(op.op_index - 1) // 10 for op in ops]
    first_layer = max(0, min(layers))
    parts = {}
    for op in ops:
        owner = runs_in.get(id(op), op)
        layer = (owner.op_index - 1) // 10
        mlp_half = layer == first_layer and (owner.op_index - 1) % 10 >= 6
        parts.setdefault((layer, mlp_half), []).extend(op.parameters())
    return [parts[k] for k in sorted(parts) if parts[k]]


class FirstLastStageTrainer:
    """A stage holding the whole GPT model (embedding, layers, final LN, LM
    head + cross entropy) on one rank: BASELINE configs[0] (fp32 plumbing
    shape) and configs[4] (GPT-6.7B first+last, fp16)."""

    def __init__(self, cfg: GPTConfig, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                 sync_mode="block", bucket_cap_bytes=1024 * 1024, initial_loss_scale=2.0**16, unpadded_vocab=50257,
                 recompute_ops=None, runtime_evidence_dir=None, accumulate_allreduce_grads_in_fp32=True,
                 overlap_optimizer=False, share_tied_storage=True):
        self.cfg = cfg
        self.unpadded_vocab = unpadded_vocab
        n_ops = 10 * cfg.num_layers + 3
        self.model = FlexGPTModel(cfg, 0, n_ops, recompute_ops=recompute_ops)
        ops = self.model.language_model.ops
        self.embedding, self.post = ops[0], ops[-1]
        with torch.no_grad():  # the head copy starts from the root (training.py:349-470)
            self.post.word_embeddings.weight.copy_(self.embedding.word_embeddings.weight)
        self.ddp = DistributedDataParallel(
            self.model, accumulate_allreduce_grads_in_fp32=_fp32_main_grads(cfg, accumulate_allreduce_grads_in_fp32))
        self.descriptors, self.bindings = collect_stage_metadata(ops, 0, n_ops)
        self.grad_sync = initialize_gradient_sync(self.descriptors, self.bindings, global_rank=0,
                                                  expected_pipeline_ids=(0,), sync_mode=sync_mode,
                                                  bucket_cap_bytes=bucket_cap_bytes,
                                                  runtime_evidence_dir=runtime_evidence_dir)
        self.optimizer = get_megatron_optimizer(
            [self.model], lr=lr, weight_decay=weight_decay, betas=betas, eps=eps, clip_grad=clip_grad,
            bf16=cfg.params_dtype == torch.bfloat16, fp16=cfg.params_dtype == torch.float16,
            initial_loss_scale=initial_loss_scale,
        )
        if share_tied_storage:
            # both tied copies live on this GPU: one weight, one master, one
            # set of moments, updated once for both (bit-identical to two
            # updates of equal inputs); the main grads stay separate
            self.optimizer.share_tied_copy(self.embedding.word_embeddings.weight, self.post.word_embeddings.weight)
        if self.ddp.accumulate_allreduce_grads_in_fp32 and math.frexp(initial_loss_scale)[0] == 0.5:
            # unscale and inf/nan flag fused into the sync's unpack; the tied
            # word embedding, summed after the sync, gets its norm share and
            # overflow check in the pass of the tied sum (exact because a
            # power-of-two loss scale -- which the dynamic scaler keeps --
            # unscales each addend without rounding, short of subnormal
            # results)
            self.optimizer.bind_gradient_sync(
                self.grad_sync.executor,
                resynced=[self.embedding.word_embeddings.weight, self.post.word_embeddings.weight])
        if overlap_optimizer:
            # the update of each part overlaps the next step's forward up to
            # that part's first op; a tied head copy of its own (without
            # shared storage), read last, updates under the whole forward,
            # a shared one with the embedding's part
            self.optimizer.overlap_with_next_forward(update_parts(ops))
        self.nominal = float(cfg.micro_batch_size * cfg.seq_length)
        self._host_weights = []

    def forward_backward(self, sample_ids, labels=None, nominal=None):
        """One microbatch: forward, loss contract, backward of
        numerator / nominal times the loss scale (schedules.py:97-104,214-217).
        Returns (per-token loss [b, s], LossOutput)."""
        # the causal attention kernels imply the boolean attention mask
        tokens, mask, positions, _ = synthetic_gpt_batch(sample_ids, self.cfg.seq_length, self.unpadded_vocab,
                                                         self.embedding.word_embeddings.weight.device,
                                                         attention_mask=False)
        extra = {} if labels is None else {"labels": labels}
        out = self.model({"enc_input_ids": tokens, "enc_position_ids": positions}, extra)
        losses = out["output"]
        lo = gpt_loss_output(losses, mask, self.nominal if nominal is None else nominal)
        self._host_weights.append(_weight_to_host(lo.local_loss_weight))
        output_tensor = lo.local_loss_sum / lo.nominal_global_loss_scale
        with overlapped_wgrad():
            torch.autograd.backward(self.optimizer.scale_loss(output_tensor))
        return losses.detach(), lo

    def _host_weight(self):
        """The step's summed loss weight as a host tensor, from the pinned
        copies queued right after each forward's loss: reading it waits for
        those forwards only, not for the backward queued behind them, so the
        sync's launches follow the backward without the GPU idling."""
        weights, self._host_weights = self._host_weights, []
        for _, ev in weights:
            ev.synchronize()
        return functools.reduce(lambda a, b: a + b, [w[0] for w, _ in weights])

    def tie_gradients(self):
        # the sum, with the root's post-sync statistics in the same pass when
        # the sync's statistics are bound
        self.optimizer.sum_tied_gradients(self.embedding.word_embeddings.weight, self.post.word_embeddings.weight)

    def train_step(self, sample_ids, labels=None):
        self.ddp.zero_grad_buffer(defer=True)
        self._host_weights = []
        losses, lo = self.forward_backward(sample_ids, labels)
        self.optimizer.join_overlapped_update()
        self.ddp.settle_grad_buffer()
        self.grad_sync.execute(global_normalization_scale(self.nominal, self._host_weight()))
        self.tie_gradients()
        ok, norm, zeros = self.optimizer.step()
        return losses, lo, ok, norm

    def train_step_microbatches(self, sample_id_batches, labels=None):
        """train_step over several microbatches (schedules.py:236-281): the
        nominal loss scale is the global token count of the step
        (config_normalization.py:535-541), every microbatch backpropagates
        its numerator / nominal, main grads accumulate, and the sync
        normalizes by nominal / (sum of the masks) -- the gradient of the
        masked mean over all microbatches.  Returns (per-microbatch losses,
        summed LossOutput pair, update_successful, grad_norm)."""
        nominal = float(len(sample_id_batches) * self.cfg.micro_batch_size * self.cfg.seq_length)
        self.ddp.zero_grad_buffer(defer=True)
        self._host_weights = []
        losses, outs = [], []
        for i, ids in enumerate(sample_id_batches):
            lab = None if labels is None else labels[i]
            l, lo = self.forward_backward(ids, lab, nominal=nominal)
            losses.append(l)
            outs.append(lo)
        self.optimizer.join_overlapped_update()
        self.ddp.settle_grad_buffer()
        numerator, weight = sum_loss_outputs(outs)
        self.grad_sync.execute(global_normalization_scale(nominal, self._host_weight()))
        self.tie_gradients()
        ok, norm, _zeros = self.optimizer.step()
        return losses, (numerator, weight), ok, norm

    def record_evidence(self, output_dir, phase, iteration, metrics=None, clock=None, run_metadata=None):
        return save_stage_snapshot(self, output_dir, phase, iteration, metrics, clock, run_metadata)


class PipelineStageTrainer(MiddleStageTrainer):
    """One stage of a GPT pipeline: manifest ops [op_start, op_end) of the
    whole model.  The first stage holds the embedding and builds its input
    from the microbatch's sample ids; the last one holds the final
    LayerNorm, the tied LM head and the loss contract, and backpropagates
    numerator / nominal times the loss scale (forward_step and backward_step,
    schedules.py:62-111,196-227; grad_sync/loss.py:16-39).  Both read the
    microbatch, as get_batch does on the first and last stages; the pipeline
    driver (eth_amd.schedules) hands it to every forward.  The defaults are
    the first+last stage's (AdamW betas 0.9 / 0.999, weight decay 0.01,
    loss scale 2^16)."""

    takes_microbatch = True

    def __init__(self, cfg: GPTConfig, op_range, unpadded_vocab=50257, lr=1e-4, betas=(0.9, 0.999), eps=1e-8,
                 weight_decay=0.01, clip_grad=1.0, initial_loss_scale=2.0**16, sync_mode="block",
                 bucket_cap_bytes=1024 * 1024, recompute_ops=None, runtime_evidence_dir=None,
                 overlap_optimizer=False, accumulate_allreduce_grads_in_fp32=True, global_rank=0,
                 defer_grad_sync=False):
        lo, hi = op_range
        n_ops = 10 * cfg.num_layers + 3
        model = FlexGPTModel(cfg, lo, hi, recompute_ops=recompute_ops)
        ops = model.language_model.ops
        self.is_first, self.is_last = lo == 0, hi == n_ops
        # the tied word embedding: the root in the embedding op, the copy in
        # the LM head's op
        self.tied_root = ops[0].word_embeddings.weight if self.is_first else None
        self.tied_copy = ops[-1].word_embeddings.weight if self.is_last else None
        if self.is_first and self.is_last:
            with torch.no_grad():  # the head copy starts from the root (training.py:349-470)
                self.tied_copy.copy_(self.tied_root)
        self.unpadded_vocab = unpadded_vocab
        self.nominal = float(cfg.micro_batch_size * cfg.seq_length)
        self._host_weights = []
        self.loss_outputs = []
        super().__init__(cfg, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, clip_grad=clip_grad,
                         sync_mode=sync_mode, bucket_cap_bytes=bucket_cap_bytes, recompute_ops=recompute_ops,
                         runtime_evidence_dir=runtime_evidence_dir, overlap_optimizer=overlap_optimizer,
                         accumulate_allreduce_grads_in_fp32=accumulate_allreduce_grads_in_fp32, model=model,
                         initial_loss_scale=initial_loss_scale,
                         resynced=[p for p in (self.tied_root, self.tied_copy) if p is not None],
                         global_rank=global_rank, defer_grad_sync=defer_grad_sync)

    def begin_step(self, nominal):
        """Start a step whose nominal loss scale (the step's global token
        count, config_normalization.py:535-541) is `nominal`."""
        self.nominal = float(nominal)
        self._host_weights = []
        self.loss_outputs = []

    def _batch(self, microbatch):
        if microbatch is None or "sample_ids" not in microbatch:
            raise ValueError("a first or last stage needs the microbatch's sample ids")
        dev = next(self.model.parameters()).device
        tokens, mask, positions, _ = synthetic_gpt_batch(microbatch["sample_ids"], self.cfg.seq_length,
                                                         self.unpadded_vocab, dev, attention_mask=False)
        return tokens, mask, positions

    def forward_step(self, input_tensors, input_extra_tensors=None, microbatch=None):
        """The stage's forward of one microbatch.  A last stage returns
        ({"loss": numerator / nominal, "losses": per-token loss [b, s]}, {},
        leaves) and keeps the microbatch's LossOutput."""
        if not (self.is_first or self.is_last):
            return super().forward_step(input_tensors, input_extra_tensors)
        tokens, mask, positions = self._batch(microbatch)
        extras = {k: v.detach().requires_grad_(v.is_floating_point())
                  for k, v in (input_extra_tensors or {}).items()}
        if self.is_first:
            ins, inputs = {}, {"enc_input_ids": tokens, "enc_position_ids": positions}
        else:
            ins = {k: v.detach().requires_grad_(True) for k, v in input_tensors.items()}
            self.model.set_input_tensor(ins)
            inputs = None
        run_extras = dict(extras)
        if self.is_last and microbatch.get("labels") is not None:
            run_extras["labels"] = microbatch["labels"]
        result = self.model(inputs, run_extras)
        if not self.is_last:
            out, out_extra = result
            return out, out_extra, (ins, extras)
        losses = result["output"]
        lo = gpt_loss_output(losses, mask, self.nominal)
        self._host_weights.append(_weight_to_host(lo.local_loss_weight))
        self.loss_outputs.append(lo)
        return {"loss": lo.local_loss_sum / lo.nominal_global_loss_scale, "losses": losses}, {}, (ins, extras)

    def backward_step(self, outputs, output_grads, output_extra_tensors=None, output_extra_grads=None, leaves=None):
        """A last stage backpropagates its loss times the loss scale
        (schedules.py:214-217); the others take the next stage's gradients."""
        if not self.is_last:
            return super().backward_step(outputs, output_grads, output_extra_tensors, output_extra_grads, leaves)
        with overlapped_wgrad():
            torch.autograd.backward(self.optimizer.scale_loss(outputs["loss"]))
        ins, extras = leaves if leaves is not None else ({}, {})
        zero = lambda t: t.grad if t.grad is not None else torch.zeros_like(t)  # noqa: E731
        return {k: zero(t) for k, t in ins.items()}, {k: zero(t) for k, t in extras.items() if t.is_floating_point()}

    def step_loss_weight(self):
        """The step's summed loss weight as a host tensor (the pinned copies
        queued after each forward's loss; waits for those forwards only)."""
        weights, self._host_weights = self._host_weights, []
        for _, ev in weights:
            ev.synchronize()
        return functools.reduce(lambda a, b: a + b, [w[0] for w, _ in weights])
