"""Pipeline schedules over stages that share one GPU.

The non-interleaved 1F1B schedule of
eth/runtime/megatron/schedules.py:595-713
(forward_backward_pipelining_without_interleaving): rank r of p runs
min(p - r - 1, m) warm-up forwards, then alternates one forward and one
backward, then drains the remaining backwards.  Here the p ranks are stage
objects in one process (MiddleStageTrainer, or anything with its
forward_step / backward_step contract), and the P2P sends and receives of
p2p_communication.py:200-538 become an in-process link that hands the
dict-of-tensor messages from one stage to the next: the `hidden_states` /
`output_tensor` dict plus the cross-stage side-channel tensors going
forward, their gradients coming back.

One process runs the ranks' actions in the order a pipeline clock would:
in every tick each rank runs its next action if its input arrived in an
earlier tick (a forward needs the previous stage's output, a backward the
next stage's input gradient), so the recorded timeline is the schedule's
own diagram, with the 2 (m + p - 1)-tick makespan of 1F1B with unit-time
forwards and backwards.  Each stage accumulates its main grads in
microbatch order whatever the schedule, so a 1F1B step gives the same
gradients, bit for bit, as running the microbatches one after another
through the stages.
"""

import collections

import torch

from .loss import global_normalization_scale, sum_loss_outputs
from .optimizer.optimizer import step_model_parallel_group


def get_num_warmup_microbatches(pipeline_size, rank, num_microbatches):
    """Warm-up forwards of `rank` (schedules.py:609-616)."""
    if not 0 <= rank < pipeline_size:
        raise ValueError(f"rank {rank} outside a pipeline of {pipeline_size}")
    return min(pipeline_size - rank - 1, num_microbatches)


def one_f_one_b_order(pipeline_size, rank, num_microbatches, forward_only=False):
    """[("F", i) | ("B", i)]: the actions `rank` runs, in order
    (schedules.py:627-711): the warm-up forwards, then forward i + warm-up
    and backward i alternating, then the cool-down backwards.  Forward-only
    runs just the forwards."""
    if num_microbatches < 0:
        raise ValueError("negative microbatch count")
    if forward_only:
        return [("F", i) for i in range(num_microbatches)]
    warmup = get_num_warmup_microbatches(pipeline_size, rank, num_microbatches)
    remaining = num_microbatches - warmup
    order = [("F", i) for i in range(warmup)]
    for i in range(remaining):
        order += [("F", warmup + i), ("B", i)]
    order += [("B", remaining + i) for i in range(warmup)]
    return order


def sequential_order(pipeline_size, rank, num_microbatches, forward_only=False):
    """Every microbatch's forward and backward before the next one's (the
    order forward_backward_no_pipelining, schedules.py:236-281, gives a
    single stage), for comparison with the pipelined order."""
    if forward_only:
        return [("F", i) for i in range(num_microbatches)]
    return [a for i in range(num_microbatches) for a in (("F", i), ("B", i))]


SCHEDULES = {"1f1b": one_f_one_b_order, "sequential": sequential_order}


class StageLink:
    """The messages between stage r and stage r + 1, keyed by microbatch
    (the P2P pair of p2p_communication.py: send_forward / recv_forward and
    send_backward / recv_backward).  A message posted in tick t can be
    received from tick t + 1 on."""

    def __init__(self):
        self.forward = {}   # microbatch -> (tick, tensors, extra tensors)
        self.backward = {}  # microbatch -> (tick, grads, extra grads)

    def send_forward(self, tick, mb, tensors, extra_tensors):
        if mb in self.forward:
            raise RuntimeError(f"microbatch {mb} sent forward twice")
        self.forward[mb] = (tick, {k: v.detach() for k, v in tensors.items()},
                            {k: v.detach() for k, v in extra_tensors.items()})

    def send_backward(self, tick, mb, grads, extra_grads):
        if mb in self.backward:
            raise RuntimeError(f"microbatch {mb} sent backward twice")
        self.backward[mb] = (tick, grads, extra_grads)

    @staticmethod
    def _ready(box, tick, mb):
        return mb in box and box[mb][0] < tick

    def recv_forward(self, mb):
        _, tensors, extras = self.forward.pop(mb)
        return tensors, extras

    def recv_backward(self, mb):
        _, grads, extras = self.backward.pop(mb)
        return grads, extras


def forward_backward_pipelining_without_interleaving(stages, microbatches, forward_only=False, schedule="1f1b"):
    """Run the microbatches through the stages (stage 0 first) in the
    pipeline order `schedule` ("1f1b", or "sequential" for one microbatch at
    a time).  Each microbatch is a dict with `input_tensors` (and optionally
    `input_extra_tensors`) for the first stage and `output_grads` (and
    optionally `output_extra_grads`) for the last one -- the upstream
    gradient of the last stage's outputs, standing in for its loss.  A GPT
    pipeline's first and last stages (PipelineStageTrainer) read
    `sample_ids` (and optionally `labels`) instead: the first builds its
    tokens from them and the last ends in the loss.

    Returns (results, timeline): per microbatch (outputs of the last stage,
    its output extra tensors, input gradients of the first stage, its input
    extra-tensor gradients); the timeline is [(tick, rank, action, mb)] plus
    the peak number of forwards each rank held for a later backward."""
    p, m = len(stages), len(microbatches)
    if p == 0:
        raise ValueError("no stages")
    if schedule not in SCHEDULES:
        raise ValueError(f"unknown schedule {schedule!r}")
    orders = [collections.deque(SCHEDULES[schedule](p, r, m, forward_only)) for r in range(p)]
    links = [StageLink() for _ in range(p - 1)]
    saved = [collections.deque() for _ in range(p)]
    peak = [0] * p
    last_out = [None] * m
    first_grads = [None] * m
    events = []
    tick = 0
    while any(orders):
        ran = False
        for r in range(p):
            if not orders[r]:
                continue
            kind, mb = orders[r][0]
            if kind == "F":
                if r > 0 and not StageLink._ready(links[r - 1].forward, tick, mb):
                    continue
                if r == 0:
                    ins = microbatches[mb].get("input_tensors")
                    extras = microbatches[mb].get("input_extra_tensors")
                else:
                    ins, extras = links[r - 1].recv_forward(mb)
                # stages that read the batch (a first stage's tokens, a last
                # stage's loss mask and labels) get the microbatch too
                kw = {"microbatch": microbatches[mb]} if getattr(stages[r], "takes_microbatch", False) else {}
                if forward_only:
                    with torch.no_grad():
                        out, out_extra, leaves = stages[r].forward_step(ins, extras, **kw)
                else:
                    out, out_extra, leaves = stages[r].forward_step(ins, extras, **kw)
                    saved[r].append((mb, out, out_extra, leaves))
                    peak[r] = max(peak[r], len(saved[r]))
                if r < p - 1:
                    links[r].send_forward(tick, mb, out, out_extra)
                else:
                    last_out[mb] = ({k: v.detach() for k, v in out.items()},
                                    {k: v.detach() for k, v in out_extra.items()})
            else:
                if r < p - 1 and not StageLink._ready(links[r].backward, tick, mb):
                    continue
                if r == p - 1:
                    # (none for a stage that ends in the loss)
                    grads = microbatches[mb].get("output_grads")
                    extra_grads = microbatches[mb].get("output_extra_grads")
                else:
                    grads, extra_grads = links[r].recv_backward(mb)
                # backwards pop the oldest saved forward (schedules.py:669-671)
                held, out, out_extra, leaves = saved[r].popleft()
                if held != mb:
                    raise RuntimeError(f"rank {r} runs backward {mb} before backward {held}")
                in_g, extra_g = stages[r].backward_step(out, grads, out_extra, extra_grads, leaves)
                if r > 0:
                    links[r - 1].send_backward(tick, mb, in_g, extra_g)
                else:
                    first_grads[mb] = (in_g, extra_g)
            orders[r].popleft()
            events.append((tick, r, kind, mb))
            ran = True
        if not ran:
            raise RuntimeError(f"pipeline schedule stalled at tick {tick}")
        tick += 1
    results = []
    for mb in range(m):
        out, out_extra = last_out[mb]
        in_g, extra_g = first_grads[mb] if first_grads[mb] is not None else ({}, {})
        results.append((out, out_extra, in_g, extra_g))
    return results, {"events": events, "ticks": tick, "peak_in_flight": peak}


class PipelineTrainer:
    """A training step of several pipeline stages on one GPU: the
    microbatches through the stages in the 1F1B order, then each stage's
    gradient sync, the tied word-embedding gradients summed across the
    first and last stages, and one optimizer step for the group, with one
    clip norm and one overflow decision over all stages (the train_step of
    pipeline-parallel ranks, training.py:904-1020).  `stages` are
    MiddleStageTrainer objects in pipeline order, or PipelineStageTrainer
    objects from the embedding to the loss."""

    def __init__(self, stages, schedule="1f1b"):
        if schedule not in SCHEDULES:
            raise ValueError(f"unknown schedule {schedule!r}")
        self.stages = list(stages)
        self.schedule = schedule
        self.last_timeline = None
        self.loss_stage = getattr(self.stages[-1], "is_last", False)
        self.last_loss = None
        if self.loss_stage and not getattr(self.stages[0], "is_first", False):
            raise ValueError("a pipeline that ends in the loss starts at the embedding")

    def tie_embeddings(self):
        """Give the LM head's copy of the word embedding the root's values
        and reload the last stage's fp32 masters from them (the copy starts
        from the root, training.py:349-470)."""
        first, last = self.stages[0], self.stages[-1]
        if not self.loss_stage or first is last:
            return
        with torch.no_grad():
            last.tied_copy.copy_(first.tied_root)
        last.optimizer.reload_model_params()

    def _tie_gradients(self):
        """synchronize_shared_weights_grads (training.py:489-531): root and
        copy main grads both become their sum; the root's optimizer takes
        the sum's statistics (its norm share and overflow check), which the
        group's step shares with the copy's stage."""
        if not self.loss_stage:
            return
        first, last = self.stages[0], self.stages[-1]
        first.optimizer.sum_tied_gradients(first.tied_root, last.tied_copy)

    def train_step(self, microbatches, normalization_scale=1.0):
        """Returns (results as forward_backward_pipelining_without_interleaving
        gives them, [(update_successful, grad_norm, num_zeros)] per stage).
        A pipeline that ends in the loss normalizes by the step's nominal
        token count over its summed loss weight (global_normalization_scale)
        and leaves the summed (numerator, weight) in `last_loss`."""
        if hasattr(normalization_scale, "item"):
            normalization_scale = float(normalization_scale.item())
        last = self.stages[-1]
        if self.loss_stage:
            cfg = last.cfg
            nominal = float(len(microbatches) * cfg.micro_batch_size * cfg.seq_length)
            last.begin_step(nominal)
        for s in self.stages:
            s.ddp.zero_grad_buffer(defer=True)
        results, self.last_timeline = forward_backward_pipelining_without_interleaving(
            self.stages, microbatches, schedule=self.schedule)
        for s in self.stages:
            s.optimizer.join_overlapped_update()
            s.ddp.settle_grad_buffer()
        if self.loss_stage:
            self.last_loss = sum_loss_outputs(last.loss_outputs)
            normalization_scale = global_normalization_scale(nominal, last.step_loss_weight())
        for s in self.stages:
            s.grad_sync.execute(normalization_scale)
        self._tie_gradients()
        return results, step_model_parallel_group([s.optimizer for s in self.stages])


def build_gpt_pipeline(cfg, cuts, schedule="1f1b", **stage_kwargs):
    """A GPT pipeline of PipelineStageTrainer stages over the consecutive
    op ranges `cuts` (from the embedding, op 0, to the loss, the last op),
    stage r holding rank r.  As the manager plans it across ranks
    (manager.py:122-214), every stage's gradient-sync plan comes from the
    descriptors of all stages -- the word embedding's root on the first
    stage and its copy on the last form one shared weight -- and each
    stage runs its own rank's buckets.  The head's copy of the word
    embedding starts from the root.  Returns the PipelineTrainer."""
    from .stage import PipelineStageTrainer

    n_ops = 10 * cfg.num_layers + 3
    cuts = [tuple(c) for c in cuts]
    if not cuts or cuts[0][0] != 0 or cuts[-1][1] != n_ops or any(
            a[1] != b[0] or a[0] >= a[1] for a, b in zip(cuts, cuts[1:] + [(n_ops, n_ops + 1)])):
        raise ValueError(f"cuts {cuts} do not split ops [0, {n_ops}) into consecutive stages")
    stages = [PipelineStageTrainer(cfg, cut, global_rank=r, defer_grad_sync=True, **stage_kwargs)
              for r, cut in enumerate(cuts)]
    parts = [tuple(st.descriptors) for st in stages]

    def gather(obj):  # the descriptor exchange; the plan hash is checked below
        return list(parts) if isinstance(obj, tuple) else [obj]

    for st in stages:
        st.finish_setup(gather)
    if len({st.grad_sync.plan.global_plan_hash for st in stages}) != 1:
        raise ValueError("gradient sync plan hash mismatch across stages")
    pipe = PipelineTrainer(stages, schedule=schedule)
    pipe.tie_embeddings()
    return pipe
