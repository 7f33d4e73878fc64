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

import torch

from . import kernels as K
from .grad_sync.gpt_adapter import collect_stage_metadata
from .loss import global_normalization_scale, gpt_loss_output, synthetic_gpt_batch
from .grad_sync.manager import initialize_gradient_sync
from .grad_sync.streamed import StreamedGradSync
from .model.distributed import DistributedDataParallel
from .model.flex_model import FlexGPTModel, middle_stage
from .model.functional import overlapped_wgrad
from .model.flex_ops import GPTConfig
from .optimizer.optimizer import get_megatron_optimizer


class MiddleStageTrainer:
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
    ):
        if cfg.params_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the stage trains in bf16 or fp16")
        self.cfg = cfg
        self.model = middle_stage(cfg, first_layer, num_layers)
        # main grads accumulate in fp32 for bf16 (as the reference forces) and
        # for fp16 too: the wgrad GEMM adds into fp32, which is strictly more
        # accurate than the reference's fp16 main_grad + later fp32 copy
        self.ddp = DistributedDataParallel(self.model, accumulate_allreduce_grads_in_fp32=True)
        lm = self.model.language_model
        descriptors, bindings = collect_stage_metadata(lm.ops, self.model.op_start, self.model.op_end)
        self.grad_sync = initialize_gradient_sync(
            descriptors,
            bindings,
            global_rank=0,
            expected_pipeline_ids=(0,),
            sync_mode=sync_mode,
            bucket_cap_bytes=bucket_cap_bytes,
            all_reduce_sum=all_reduce_sum or (lambda payload, handle: None),
        )
        self.optimizer = get_megatron_optimizer(
            [self.model],
            lr=lr,
            weight_decay=weight_decay,
            betas=betas,
            eps=eps,
            clip_grad=clip_grad,
            bf16=cfg.params_dtype == torch.bfloat16,
            fp16=cfg.params_dtype == torch.float16,
        )
        self.optimizer.bind_gradient_sync(self.grad_sync.executor)
        # buckets synced during the backward, as soon as their gradients
        # exist (train_step(streamed_sync=True))
        self._streamed = None
        dev = next(self.model.parameters()).device
        if dev.type == "cuda":
            self._streamed = StreamedGradSync(self.grad_sync.executor, dev)

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
        """One step.  With streamed_sync each gradient bucket is packed /
        all-reduced / unpacked as soon as the backward has written it,
        overlapped with the rest of the backward; otherwise (the default) the
        whole sync runs after it, as in the reference.  Both give identical
        results.  On one GPU the all-reduce seam moves no data, and the
        overlapped pack/unpack slows the backward's GEMMs by about as much as
        it hides (measured 413 K vs 417-420 K tokens/s), so the overlap is
        for deployments whose seam does real communication."""
        if hasattr(normalization_scale, "item"):
            normalization_scale = float(normalization_scale.item())
        # deferred: the first gradient written into each main_grad stores
        self.ddp.zero_grad_buffer(defer=True)
        streamed = streamed_sync and self._streamed is not None
        if streamed:
            self._streamed.start(normalization_scale)
            try:
                out, dx = self.forward_backward(x, dy)
            finally:
                self._streamed.finish()
            self.ddp.settle_grad_buffer()
        else:
            out, dx = self.forward_backward(x, dy)
            self.ddp.settle_grad_buffer()
            self.grad_sync.execute(normalization_scale)
        ok, norm, zeros = self.optimizer.step()
        return out, dx, ok, norm

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


class FirstLastStageTrainer:
    """A stage holding the whole GPT model (embedding, layers, final LN, LM
    head + cross entropy) on one rank: BASELINE configs[0] (fp32 plumbing
    shape) and configs[4] (GPT-6.7B first+last, fp16)."""

    def __init__(self, cfg: GPTConfig, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, clip_grad=1.0,
                 sync_mode="block", bucket_cap_bytes=1024 * 1024, initial_loss_scale=2.0**16, unpadded_vocab=50257):
        self.cfg = cfg
        self.unpadded_vocab = unpadded_vocab
        n_ops = 10 * cfg.num_layers + 3
        self.model = FlexGPTModel(cfg, 0, n_ops)
        ops = self.model.language_model.ops
        self.embedding, self.post = ops[0], ops[-1]
        with torch.no_grad():  # the head copy starts from the root (training.py:349-470)
            self.post.word_embeddings.weight.copy_(self.embedding.word_embeddings.weight)
        self.ddp = DistributedDataParallel(self.model, accumulate_allreduce_grads_in_fp32=True)
        descriptors, bindings = collect_stage_metadata(ops, 0, n_ops)
        self.grad_sync = initialize_gradient_sync(descriptors, bindings, global_rank=0, expected_pipeline_ids=(0,),
                                                  sync_mode=sync_mode, bucket_cap_bytes=bucket_cap_bytes)
        self.optimizer = get_megatron_optimizer(
            [self.model], lr=lr, weight_decay=weight_decay, betas=betas, eps=eps, clip_grad=clip_grad,
            bf16=cfg.params_dtype == torch.bfloat16, fp16=cfg.params_dtype == torch.float16,
            initial_loss_scale=initial_loss_scale,
        )
        # tied weights: the norm / unscale run after the tied-gradient sum,
        # so the optimizer computes its statistics itself (no fused binding)
        self.nominal = float(cfg.micro_batch_size * cfg.seq_length)

    def forward_backward(self, sample_ids, labels=None):
        """Returns (per-token loss [b, s], LossOutput)."""
        tokens, mask, positions, _ = synthetic_gpt_batch(sample_ids, self.cfg.seq_length, self.unpadded_vocab,
                                                         self.embedding.word_embeddings.weight.device)
        extra = {} if labels is None else {"labels": labels}
        out = self.model({"enc_input_ids": tokens, "enc_position_ids": positions}, extra)
        losses = out["output"]
        lo = gpt_loss_output(losses, mask, self.nominal)
        output_tensor = lo.local_loss_sum / lo.nominal_global_loss_scale
        with overlapped_wgrad():
            torch.autograd.backward(self.optimizer.scale_loss(output_tensor))
        return losses.detach(), lo

    def tie_gradients(self):
        K.tied_grad_sum(self.embedding.word_embeddings.weight.main_grad, self.post.word_embeddings.weight.main_grad)

    def train_step(self, sample_ids, labels=None):
        self.ddp.zero_grad_buffer(defer=True)
        losses, lo = self.forward_backward(sample_ids, labels)
        self.ddp.settle_grad_buffer()
        self.grad_sync.execute(global_normalization_scale(self.nominal, lo.local_loss_weight))
        self.tie_gradients()
        ok, norm, zeros = self.optimizer.step()
        return losses, lo, ok, norm
