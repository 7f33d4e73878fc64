"""Loss contract, synthetic batch and training clock of the last stage.

Restates eth/runtime/megatron/grad_sync/loss.py:
  * gpt_loss_output (:16-30): local_loss_sum = sum(loss * mask),
    local_loss_weight = sum(mask);
  * global_normalization_scale (:33-39): nominal / global weight, applied to
    the gradients by GradientSyncManager.execute;
  * synthetic_gpt_batch (:100-119): tokens (id*1103515245 + pos*12345) mod
    vocab, mask (id + pos) % 4 != 0, positions arange(s);
  * TrainingClock (:123-137).
The backward runs on local_loss_sum / nominal_global_loss_scale
(schedules.py:97-104), times the loss scale (schedules.py:215).
These are [b, s]-sized host-orchestrated tensors, not a hot path.
"""

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class LossOutput:
    local_loss_sum: object
    local_loss_weight: object
    nominal_global_loss_scale: float
    metrics: dict


def gpt_loss_output(losses, loss_mask, nominal_global_loss_scale, metrics=None):
    if nominal_global_loss_scale <= 0:
        raise ValueError("nominal_global_loss_scale must be positive")
    flat_losses = losses.float().reshape(-1)
    flat_mask = loss_mask.float().reshape(-1)
    if flat_losses.numel() != flat_mask.numel():
        raise ValueError("GPT loss and loss_mask must have the same numel")
    return LossOutput(
        local_loss_sum=torch.sum(flat_losses * flat_mask),
        local_loss_weight=torch.sum(flat_mask),
        nominal_global_loss_scale=float(nominal_global_loss_scale),
        metrics={} if metrics is None else metrics,
    )


def global_normalization_scale(nominal_global_loss_scale, global_loss_weight):
    if nominal_global_loss_scale <= 0:
        raise ValueError("nominal_global_loss_scale must be positive")
    if float(global_loss_weight.detach().item()) <= 0:
        raise ValueError("global_loss_weight must be positive")
    return nominal_global_loss_scale / global_loss_weight


def synthetic_gpt_batch(sample_ids, sequence_length, vocab_size, device):
    ids = torch.as_tensor(sample_ids, dtype=torch.long, device=device)
    positions = torch.arange(sequence_length, dtype=torch.long, device=device)
    tokens = (ids[:, None] * 1103515245 + positions[None, :] * 12345).remainder(vocab_size)
    loss_mask = ((ids[:, None] + positions[None, :]) % 4 != 0).float()
    position_ids = positions[None, :].expand(ids.numel(), -1).clone()
    attention_mask = torch.triu(
        torch.ones(ids.numel(), 1, sequence_length, sequence_length, dtype=torch.bool, device=device), diagonal=1
    )
    return tokens, loss_mask, position_ids, attention_mask


@dataclass
class TrainingClock:
    total_gbs: int
    global_data_cursor: int = 0
    successful_optimizer_steps: int = 0

    def __post_init__(self):
        if self.total_gbs <= 0:
            raise ValueError("total_gbs must be positive")

    def after_attempt(self, update_successful):
        self.global_data_cursor += self.total_gbs
        if not update_successful:
            return 0
        self.successful_optimizer_steps += 1
        return self.total_gbs
