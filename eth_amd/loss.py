"""Loss contract, sample ownership, synthetic batch and training clock.

The last stage reports its loss as a (numerator, weight) pair instead of a
mean, so that the global mean over every microbatch and data-parallel rank
is formed once, by the gradient sync (eth/runtime/megatron/grad_sync/loss.py):

* `gpt_loss_output` (:16-30): numerator = sum(loss * mask) in fp32,
  weight = sum(mask); the backward runs on numerator / nominal
  (schedules.py:97-104) times the loss scale (schedules.py:215);
* `global_normalization_scale` (:33-39): nominal / global weight, the factor
  GradientSyncManager.execute applies to the summed gradients;
* `sum_loss_outputs` (:42-48), the training clock (:51-67, :123-137) and
  `local_sample_slots` (:70-97): which global sample ids a (pipeline,
  microbatch, DP rank) consumes;
* `synthetic_gpt_batch` (:100-119): the reference's deterministic batch,
  token = (id * 1103515245 + pos * 12345) mod vocab and mask
  (id + pos) % 4 != 0; on the GPU its tokens, mask and position ids come
  from one kernel (`eth_synthetic_batch`), and the stages skip the boolean
  attention mask, which the causal attention kernels imply.

All of it is [b, s]-sized or scalar orchestration; none of it is on the
HBM- or MFMA-bound part of the step.
"""

import functools
from dataclasses import dataclass

import torch

# the reference's synthetic-token LCG (grad_sync/loss.py:104-106)
_LCG_SAMPLE, _LCG_POSITION = 1103515245, 12345


def _require_positive(name, value):
    if not value > 0:
        raise ValueError(f"{name} must be positive, got {value!r}")


@dataclass(frozen=True)
class LossOutput:
    local_loss_sum: object
    local_loss_weight: object
    nominal_global_loss_scale: float
    metrics: dict


def gpt_loss_output(losses, loss_mask, nominal_global_loss_scale, metrics=None):
    """(sum of masked per-token losses, sum of the mask) in fp32."""
    _require_positive("nominal_global_loss_scale", nominal_global_loss_scale)
    values = losses.reshape(-1).to(torch.float32)
    weights = loss_mask.reshape(-1).to(device=values.device, dtype=torch.float32)
    if values.shape != weights.shape:
        raise ValueError(
            f"GPT loss has {values.numel()} elements but loss_mask has {weights.numel()}"
        )
    return LossOutput(
        local_loss_sum=torch.dot(values, weights),
        local_loss_weight=weights.sum(),
        nominal_global_loss_scale=float(nominal_global_loss_scale),
        metrics=dict(metrics or {}),
    )


def global_normalization_scale(nominal_global_loss_scale, global_loss_weight):
    """Factor that turns gradients of sum(loss)/nominal into gradients of the
    global masked mean."""
    _require_positive("nominal_global_loss_scale", nominal_global_loss_scale)
    if not float(global_loss_weight.detach().item()) > 0:
        raise ValueError("global_loss_weight must be positive (no unmasked token in the global batch)")
    return nominal_global_loss_scale / global_loss_weight


def sum_loss_outputs(loss_outputs):
    """(numerator, weight) summed over microbatches before any division."""
    pairs = [(o.local_loss_sum, o.local_loss_weight) for o in loss_outputs]
    if not pairs:
        raise ValueError("loss_outputs must not be empty")
    return functools.reduce(lambda a, b: (a[0] + b[0], a[1] + b[1]), pairs)


def local_sample_slots(pipeline_id, microbatch_index, dp_degree, dp_rank, mbs_sequences, pipeline_sample_offsets,
                       global_data_cursor):
    """Global sample ids of one DP rank's share of one microbatch.

    A pipeline's microbatches tile its block of the global batch in order
    (prefix sums of their sizes), the block starts at the pipeline's sample
    offset past the cursor, and DP ranks split each microbatch evenly."""
    if pipeline_id not in range(len(mbs_sequences)):
        raise ValueError(f"unknown pipeline_id {pipeline_id}")
    sizes = [entry[0] for entry in mbs_sequences[pipeline_id]]
    if microbatch_index not in range(len(sizes)):
        raise ValueError(f"unknown microbatch_index {microbatch_index}")
    if dp_degree <= 0 or dp_rank not in range(dp_degree):
        raise ValueError(f"invalid DP coordinate {dp_rank} of {dp_degree}")
    share, rest = divmod(sizes[microbatch_index], dp_degree)
    if rest:
        raise ValueError("global microbatch size must be divisible by DP degree")
    start = global_data_cursor + pipeline_sample_offsets[pipeline_id] + sum(sizes[:microbatch_index])
    start += dp_rank * share
    return tuple(range(start, start + share))


def synthetic_gpt_batch(sample_ids, sequence_length, vocab_size, device, attention_mask=True):
    """(tokens [b, s] int64, loss_mask [b, s] fp32, position_ids [b, s],
    attention_mask [b, 1, s, s] bool, True above the diagonal -- or None
    when `attention_mask` is False).  On a GPU the first three come from the
    eth_synthetic_batch kernel; on the CPU from torch."""
    device = torch.device(device)
    pos = torch.arange(sequence_length, dtype=torch.long, device=device).reshape(1, -1)
    if device.type == "cuda":
        from . import kernels

        tokens, loss_mask, position_ids = kernels.synthetic_batch(sample_ids, sequence_length, vocab_size, device)
        n = tokens.shape[0]
    else:
        ids = torch.as_tensor(sample_ids, dtype=torch.long, device=device).reshape(-1, 1)
        tokens = torch.remainder(ids * _LCG_SAMPLE + pos * _LCG_POSITION, vocab_size)
        loss_mask = torch.remainder(ids + pos, 4).ne(0).to(torch.float32)
        position_ids = pos.repeat(ids.shape[0], 1)
        n = ids.shape[0]
    if not attention_mask:
        return tokens, loss_mask, position_ids, None
    future = pos.reshape(-1, 1) < pos  # key position after the query position
    mask = future.expand(n, 1, sequence_length, sequence_length).clone()
    return tokens, loss_mask, position_ids, mask


def restore_training_clock(checkpoint_args, iteration):
    """(global_data_cursor, successful_optimizer_steps) from checkpoint args;
    older checkpoints only carry consumed_train_samples and the iteration."""
    consumed = getattr(checkpoint_args, "consumed_train_samples", 0)
    cursor = getattr(checkpoint_args, "global_data_cursor", consumed)
    return cursor, getattr(checkpoint_args, "successful_optimizer_steps", iteration)


def validate_training_clock_states(clock_states):
    states = list(clock_states)
    if not states:
        raise ValueError("training clock states must not be empty")
    if any(state != states[0] for state in states):
        raise ValueError(f"training clock mismatch across ranks: {tuple(states)}")


@dataclass
class TrainingClock:
    """Samples consumed by every attempted step vs optimizer steps applied."""

    total_gbs: int
    global_data_cursor: int = 0
    successful_optimizer_steps: int = 0

    def __post_init__(self):
        _require_positive("total_gbs", self.total_gbs)

    def after_attempt(self, update_successful):
        """Advance past this step's samples; returns the samples that count
        as trained (0 for a skipped step)."""
        self.global_data_cursor += self.total_gbs
        self.successful_optimizer_steps += int(bool(update_successful))
        return self.total_gbs if update_successful else 0
