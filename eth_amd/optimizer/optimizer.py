"""Megatron optimizer wrappers on the fused HIP path.

Step contract of eth/runtime/megatron/optimizer/optimizer.py:493-531:
`step() -> (update_successful, grad_norm, num_zeros)`; copy model grads to
main grads, unscale + inf/nan check (fp16 loss scaling), skip the step and
back off the scale on overflow, clip to `clip_grad` by the global L2 norm,
AdamW on fp32 masters, copy masters to the 16-bit model parameters.

How it runs here: the unscale / flag / sum of squares are either already
done by the gradient-sync unpack (when an executor is bound with
`bind_gradient_sync`) or done by one standalone statistics launch; the norm
and clip coefficient are finalized on the device; the AdamW launch reads the
coefficient and the overflow flag from device memory and writes the model
copy itself.  The host reads the flag and the norm once, after everything is
queued.
"""

import functools

import numpy as np
import torch

from .. import _native as nat
from ..grad_sync.executor import GradientStatistics, chunk_table, split_block
from .fused_adam import FusedAdamW


def _flat_master_copies(model_params):
    """fp32 master copies of `model_params`, views of one 16-byte aligned buffer."""
    sizes = [(p.numel() + 3) // 4 * 4 for p in model_params]
    device = model_params[0].device
    flat = torch.empty(sum(sizes), dtype=torch.float32, device=device)
    masters, off = [], 0
    for p, n in zip(model_params, sizes):
        m = flat[off : off + p.numel()].view_as(p)
        m.copy_(p.detach())
        m.requires_grad_(True)
        for attr in ("tensor_model_parallel", "partition_dim", "partition_stride", "shared"):
            if hasattr(p, attr):
                setattr(m, attr, getattr(p, attr))
        masters.append(m)
        off += n
    return flat, masters


class MegatronOptimizer:
    def __init__(self, optimizer, clip_grad, log_num_zeros_in_grad, params_have_main_grad):
        self.optimizer = optimizer
        self.clip_grad = float(clip_grad)
        self.log_num_zeros_in_grad = log_num_zeros_in_grad
        self.params_have_main_grad = params_have_main_grad
        self.grad_scaler = None
        self._executor = None
        self._statistics = None
        self._stats_tables = None
        self._stats_key = None
        self._model_to_optimizer_param = {}
        self._host_flags = None
        self._overlap = None  # (side stream, [[model params] per part]) when the update overlaps the next forward
        self._unlaunched_parts = set()  # parts of a deferred overlapped update not issued yet
        self._join_pending = False  # an overlapped update not yet joined by the current stream
        # parts of a deferred update issued by step() itself, before the host
        # waits for the read-back: the GPU work queued while the host returns
        # and starts the next forward
        self.eager_update_parts = 3
        self._post_sync = (None, 0)  # chunk table of norm-owned gradients summed after the sync
        self._shared_copies = []  # model parameters updated through another's optimizer parameter
        self._post_sync_params = []  # model parameters whose gradients the post-sync table covers
        self._post_sync_done = None  # statistics generation whose post-sync pass the tied sum already made

    # ----------------------------------------------------------- plumbing --
    @property
    def param_groups(self):
        return self.optimizer.param_groups

    def get_parameters(self):
        return [p for g in self.optimizer.param_groups for p in g["params"]]

    def get_loss_scale(self):
        if self.grad_scaler is None:
            return torch.ones(1, dtype=torch.float32, device=self._device())
        return self.grad_scaler.scale

    def scale_loss(self, loss):
        return self.get_loss_scale() * loss

    def _device(self):
        dev = getattr(self, "_dev", None)
        if dev is None:
            dev = self._dev = self.get_parameters()[0].device
        return dev

    def state_for_model_parameter(self, model_parameter):
        p = self._model_to_optimizer_param.get(id(model_parameter))
        if p is None:
            raise ValueError("model parameter is not owned by this optimizer")
        return self.optimizer.state.get(p, {})

    def optimizer_parameter_for_model_parameter(self, model_parameter):
        p = self._model_to_optimizer_param.get(id(model_parameter))
        if p is None:
            raise ValueError("model parameter is not owned by this optimizer")
        return p

    def hyperparameters_for_model_parameter(self, model_parameter):
        """{beta1, beta2, epsilon, weight_decay} of the parameter's group (what
        the evidence snapshots record, optimizer/optimizer.py:113-131)."""
        p = self.optimizer_parameter_for_model_parameter(model_parameter)
        for group in self.optimizer.param_groups:
            if any(q is p for q in group["params"]):
                beta1, beta2 = group.get("betas", (None, None))
                return {"beta1": beta1, "beta2": beta2, "epsilon": group.get("eps"),
                        "weight_decay": group.get("weight_decay", 0.0)}
        raise ValueError("optimizer parameter has no parameter group")

    def overlap_with_next_forward(self, model_param_parts):
        """Run the AdamW update on a side stream (default priority), one
        launch per part of `model_param_parts` (lists of model parameters, in
        the order the next forward reads them), and leave on each model
        parameter the event after which its new value is written
        (`_eth_ready_event`, shared by the parameters of a part listed in
        `_eth_ready_part`).  The stage's forward waits for a part's event at
        the first op that reads one of its parameters, so the update of later
        layers overlaps the forward of earlier ones; every result is the same
        as with the update in line."""
        dev = self._device()
        # an optimizer parameter that serves several model parameters (a
        # shared tied copy) updates in the first part that holds one of them
        parts, placed = [], set()
        for part in model_param_parts:
            parts.append([])
            for p in part:
                o = self.optimizer_parameter_for_model_parameter(p)
                if id(o) not in placed:
                    placed.add(id(o))
                    parts[-1].append(o)
        missing = [p for g in self.optimizer.param_groups for p in g["params"] if id(p) not in placed]
        if missing:
            # the deferred launches only cover the given parts: a parameter in
            # none of them would never be updated
            raise ValueError(f"overlapped update parts miss {len(missing)} optimizer parameter(s)")
        self.optimizer.set_partition(parts)
        self._overlap = (torch.cuda.Stream(device=dev), [list(part) for part in model_param_parts])

    def launch_update_part(self, k, wait=True):
        """Issue part k of a deferred overlapped update (once) on the side
        stream, behind everything queued on the current stream so far (with
        wait=False, behind what the side stream already waited for: the
        step's own launches, issued right after that wait, skip a second
        one, which would cost the side stream a few microseconds)."""
        side, model_parts = self._overlap
        if k not in self._unlaunched_parts:
            return
        self._unlaunched_parts.discard(k)
        # (the parameters keep their launch hook: a second call returns above)
        if wait:
            side.wait_stream(torch.cuda.current_stream(self._device()))
        with torch.cuda.stream(side):
            self.optimizer.launch_part(k)

    def join_overlapped_update(self):
        """Issue the parts of an overlapped update not launched yet and make
        the current stream wait for every part that no forward op has waited
        for yet."""
        if self._overlap is None or not self._join_pending:
            return
        self._join_pending = False
        for k in sorted(self._unlaunched_parts):
            self.launch_update_part(k)
        stream = torch.cuda.current_stream(self._device())
        waited = set()
        for part in self._overlap[1]:
            for p in part:
                ev = getattr(p, "_eth_ready_event", None)
                if ev is not None:
                    if id(ev) not in waited:
                        stream.wait_event(ev)
                        waited.add(id(ev))
                    p._eth_ready_event = None

    def share_tied_copy(self, root, copy):
        """Make the tied copy `copy` of model parameter `root` (the LM head's
        word embedding beside the embedding's, on one GPU) share the root's
        storage: its weight becomes a view of the root's, and the root's fp32
        master and AdamW moments serve both, so one update writes both.  The
        reference keeps two parameters whose gradients it sums and updates
        alike (training.py:489-531); from equal starting values, equal
        gradients and equal hyper-parameters the two updates are identical,
        so the shared one gives the same bits.  The copy keeps its own main
        grad, which the sync and the tied gradient sum treat as before."""
        if self._overlap is not None or self._executor is not None:
            raise ValueError("share the tied copy before binding the sync or overlapping the update")
        r = self.optimizer_parameter_for_model_parameter(root)
        c = self.optimizer_parameter_for_model_parameter(copy)
        if r is c:
            return
        if root.shape != copy.shape or root.dtype != copy.dtype:
            raise ValueError("tied copies must have one shape and dtype")
        hyper = [{k: v for k, v in g.items() if k != "params"} for q in (r, c)
                 for g in self.optimizer.param_groups if any(x is q for x in g["params"])]
        if len(hyper) != 2 or hyper[0] != hyper[1]:
            raise ValueError("tied copies must be in parameter groups with equal hyper-parameters")
        st_r, st_c = self.optimizer.state.get(r, {}), self.optimizer.state.get(c, {})
        if float(st_r.get("step", 0)) != float(st_c.get("step", 0)) or not torch.equal(root, copy):
            raise ValueError("tied copies must have equal values and step counts to share storage")
        with torch.no_grad():
            copy.data = root.data
        self.optimizer.remove_param(c)
        self._drop_model_parameter(copy)
        self._model_to_optimizer_param[id(copy)] = r
        self._shared_copies.append(copy)

    def sum_tied_gradients(self, root, copy):
        """root.main_grad = copy.main_grad = their sum: the same-rank branch of
        synchronize_shared_weights_grads (training.py:489-531).  When the
        sync's statistics are bound and the post-sync table covers the root
        alone, the sum and the root's post-sync statistics (its norm share
        and the check of its loss-scaled values) are one pass
        (eth_tied_grad_sum_stats) and the step skips its own pass; the bits
        are those of the sum followed by that pass."""
        from .. import kernels as K

        rg, cg = root.main_grad, copy.main_grad
        table, n = self._post_sync
        st = self._statistics
        if (n and st is not None and st.fresh and len(self._post_sync_params) == 1
                and self._post_sync_params[0] is root and rg.dtype == cg.dtype == torch.float32
                and rg.shape == cg.shape and rg.is_contiguous() and cg.is_contiguous()):
            scale = self.grad_scaler.host_scale if self.grad_scaler is not None else 1.0
            nat.call("eth_tied_grad_sum_stats", nat.ptr(table), n, nat.ptr(rg), nat.ptr(cg), float(scale),
                     nat.ptr(st.found_inf), nat.ptr(st.partials), self._executor.n_partials,
                     nat.stream_ptr(self._device()))
            self._post_sync_done = st.generation
            return
        K.tied_grad_sum(rg, cg)

    def _drop_model_parameter(self, param):
        """Forget the bookkeeping that pairs `param` with an optimizer
        parameter of its own (subclasses that keep masters)."""

    def bind_gradient_sync(self, executor, resynced=()):
        """Fuse unscale / inf-nan flag / L2 partials into `executor`'s unpack.

        Only valid when every optimizer gradient is an fp32 main_grad the
        executor writes (bf16 or fp32 training).  `resynced`: model
        parameters whose main grads change after the sync (the tied word
        embedding, summed by the stage afterwards).  The unpack still
        unscales them -- the loss scale is a power of two, so unscaling each
        addend first gives the bits of unscaling the sum -- but leaves them
        out of the norm; the step then takes the norm-owned ones' sum of
        squares and re-checks them for overflow in one pass."""
        covered = executor.covered_gradients()
        by_ptr = {g.data_ptr(): lid for lid, g in covered.items()}
        grads = self._bound_main_grads()
        if any(g is None or g.dtype != torch.float32 or g.data_ptr() not in by_ptr for g in grads):
            raise ValueError("fused gradient statistics need fp32 main grads written by the executor")
        post = [p for p in resynced if self._norm_owned(p)]
        if any(getattr(p, "main_grad", None) is None or p.main_grad.data_ptr() not in by_ptr for p in resynced):
            raise ValueError("re-synced parameters must have main grads written by the executor")
        executor.exclude_from_norm(by_ptr[p.main_grad.data_ptr()] for p in post)
        entries = []
        for p in post:
            g = p.main_grad
            split_block(g.data_ptr(), 4, 1, g.numel(), g.numel(), 0, 1.0, nat.CHUNK_NORM, entries)
        table = chunk_table(entries)
        self._post_sync = (nat.table_to_device(table, self._device()) if len(table) else None, len(table))
        self._post_sync_params = list(post)
        self._executor = executor
        self._statistics = GradientStatistics(executor.n_partials + len(table), self._device())
        self._statistics.before_reuse = self.join_overlapped_update
        executor.bind_statistics(self._statistics)
        executor.set_inv_loss_scale(self._inv_scale())

    def unbind_gradient_sync(self):
        """Undo bind_gradient_sync: the sync only moves gradients again and
        the step takes every statistic itself (one standalone pass)."""
        if self._executor is not None:
            self._executor.bind_statistics(None)
            self._executor.exclude_from_norm(())
        self._executor = None
        self._statistics = None
        self._post_sync = (None, 0)
        self._post_sync_params = []
        self._post_sync_done = None

    @property
    def grads_unscaled_by_sync(self):
        """True when the gradient sync's unpack unscales the main grads (a
        fused binding): after the sync they hold the unscaled gradients."""
        return self._executor is not None

    def _bound_main_grads(self):
        raise NotImplementedError

    def _inv_scale(self):
        return self.grad_scaler.inv_scale_value if self.grad_scaler is not None else 1.0

    # --------------------------------------------------------- statistics --
    def _norm_owned(self, param):
        return not getattr(param, "shared", False) or getattr(param, "shared_root", False)

    def _widen_sources(self):
        """{id(optimizer parameter): 16-bit main grad} of the gradients the
        step still has to widen into the parameter's fp32 grad (none here)."""
        return {}

    def _widen_target(self):
        """The fp32 buffer the widened gradients are views of."""
        raise NotImplementedError

    def _standalone_statistics(self, unscale, stats=True):
        """One statistics pass over every optimizer gradient: unscale (when
        `unscale`), overflow flag and per-chunk sums of squares (when
        `stats`).  Gradients still held as 16-bit main grads are widened into
        their fp32 grads in the same pass (eth_widen_grad_stats); the others
        are done in place (eth_grad_stats).  Returns the statistics, or None
        without `stats`."""
        widen = self._widen_sources()
        params = [p for p in self.get_parameters() if p.grad is not None]
        # the fp32 main grads of shared tied copies are nobody's optimizer
        # gradient, but the reference unscales them in place like every main
        # grad (and checks them): they join the pass outside the norm
        extra = [c.main_grad for c in self._shared_copies
                 if self.params_have_main_grad and getattr(c, "main_grad", None) is not None
                 and c.main_grad.dtype == torch.float32]
        key = tuple((p.grad.data_ptr(), p.grad.numel(), widen[id(p)].data_ptr() if id(p) in widen else 0)
                    for p in params) + tuple((g.data_ptr(), g.numel(), -1) for g in extra)
        if key != self._stats_key:
            wide, plain, code = [], [], None
            base = self._widen_target().data_ptr() if widen else 0
            for p in params:
                g = p.grad
                if g.dtype != torch.float32 or not g.is_contiguous():
                    raise ValueError("optimizer gradients must be contiguous fp32")
                flags = nat.CHUNK_NORM if self._norm_owned(p) else 0
                src = widen.get(id(p))
                if src is None:
                    split_block(g.data_ptr(), 4, 1, g.numel(), g.numel(), 0, 1.0, flags, plain)
                    continue
                if src.shape != g.shape or not src.is_contiguous():
                    raise ValueError("16-bit main grads must be contiguous and shaped like their parameters")
                if code is not None and nat.dtype_code(src.dtype) != code:
                    raise ValueError("16-bit main grads of one optimizer must share a dtype")
                code = nat.dtype_code(src.dtype)
                dst = (g.data_ptr() - base) // 4
                split_block(src.data_ptr(), 2, 1, src.numel(), src.numel(), dst, 1.0, flags, wide)
            for g in extra:
                if not g.is_contiguous():
                    raise ValueError("main grads must be contiguous")
                split_block(g.data_ptr(), 4, 1, g.numel(), g.numel(), 0, 1.0, 0, plain)
            self._stats_tables = tuple(
                (nat.table_to_device(chunk_table(e), self._device()) if e else None, len(e)) for e in (wide, plain))
            self._widen_code = code
            self._stats_key = key
            n_total = len(wide) + len(plain)
            if self._statistics is None or self._statistics.n_partials < n_total:
                self._statistics = GradientStatistics(n_total, self._device())
                if self._executor is not None:
                    self._executor.bind_statistics(None)
                    self._executor = None
        (wtable, nw), (table, n) = self._stats_tables
        st = self._statistics
        if stats:
            st.reset()
        flags = nat.UNPACK_UNSCALE if unscale else 0
        stream = nat.stream_ptr(self._device())
        if nw:
            nat.call("eth_widen_grad_stats", nat.ptr(wtable), nw, self._widen_target().data_ptr(), self._widen_code,
                     float(self._inv_scale()), flags | (nat.UNPACK_STATS if stats else 0), nat.ptr(st.found_inf),
                     nat.ptr(st.partials), 0, stream)
        if not stats:
            if unscale:
                raise ValueError("unscaling without statistics is not a step of this optimizer")
            return None
        if n:
            nat.call("eth_grad_stats", nat.ptr(table), n, float(self._inv_scale()), flags, nat.ptr(st.found_inf),
                     nat.ptr(st.partials), nw, stream)
        # partials past this pass's chunks must not leak into the norm
        st.n_partials_used = nw + n
        return st

    def count_zeros(self):
        total = 0
        for p in self.get_parameters():
            if p.grad is not None and self._norm_owned(p):
                total += p.grad.numel() - int(torch.count_nonzero(p.grad).item())
        return float(total)

    # --------------------------------------------------------------- step --
    def _copy_model_grads_to_main_grads(self):
        raise NotImplementedError

    @torch.no_grad()
    def step(self):
        st = self.gather_statistics()
        return self.apply_statistics(st)

    @torch.no_grad()
    def gather_statistics(self):
        """The first half of step(): the pending update joined, the model
        grads copied to the main grads, and the statistics passes queued
        (found_inf and the per-chunk partial sums of squares, before the norm
        is finalized).  Returns the statistics (None when the step needs
        neither a norm nor an overflow check).  Stages that clip by one norm
        combine their statistics between the two halves
        (step_model_parallel_group)."""
        self.join_overlapped_update()
        self._copy_model_grads_to_main_grads()
        scaler = self.grad_scaler
        need_norm = self.clip_grad > 0.0
        st = self._statistics
        fused = st is not None and self._executor is not None and st.fresh
        if fused and scaler is not None and st.inv_scale_used != self._inv_scale():
            raise RuntimeError("loss scale changed between gradient sync and optimizer step")
        if fused:
            st.n_partials_used = self._executor.n_partials
            table, n = self._post_sync
            done, self._post_sync_done = self._post_sync_done == st.generation, None
            if n and not done:
                # statistics of the gradients changed after the sync (already
                # unscaled by the unpack): sum of squares into the slots after
                # the executor's; found_inf where a sum, loss-scaled again,
                # is not finite -- the reference sums the scaled addends
                # (training.py:997-1004) and flags that overflow at step()
                scale = scaler.host_scale if scaler is not None else 1.0
                nat.call("eth_grad_stats", nat.ptr(table), n, float(scale), nat.STATS_SCALED_OVERFLOW,
                         nat.ptr(st.found_inf), nat.ptr(st.partials), st.n_partials_used,
                         nat.stream_ptr(self._device()))
            st.n_partials_used += n  # slots the pass above, or the fused tied sum, wrote
        elif scaler is not None or need_norm:
            st = self._standalone_statistics(unscale=scaler is not None)
        elif self._widen_sources():
            # 16-bit main grads still to be widened, no statistics wanted
            self._standalone_statistics(unscale=False, stats=False)
        if st is not None:
            st.fresh = False
        return st if (scaler is not None or need_norm) else None

    @torch.no_grad()
    def apply_statistics(self, st, partials=None, n_partials=None):
        """The second half of step(): finalize the norm from `partials`
        (default: the statistics' own), read the norm and the overflow flag
        back, and update.  Returns (update_successful, grad_norm, num_zeros)."""
        scaler = self.grad_scaler
        need_norm = self.clip_grad > 0.0
        if need_norm:
            if partials is None:
                partials, n_partials = st.partials, st.n_partials_used
            nat.call(
                "eth_grad_norm_finalize",
                nat.ptr(partials),
                n_partials,
                self.clip_grad,
                nat.ptr(st.stats),
                nat.stream_ptr(self._device()),
            )
        # the host reads the norm and the inf flag from a pinned copy queued
        # before the update kernel, so it waits for the statistics only, not
        # for the update (the next step's launches overlap the update)
        host = None
        if self._overlap is not None:
            # the overlapped update needs the statistics on the device, not
            # the copies to the host queued next
            self._overlap[0].wait_stream(torch.cuda.current_stream(self._device()))
        if st is not None and (need_norm or scaler is not None):
            host = self._read_back(st)
        if self._overlap is None:
            self.optimizer.step(
                stats=st.stats if need_norm else None,
                found_inf=st.found_inf if scaler is not None else None,
            )
        else:
            # every part's launch is prepared now and issued later: the first
            # layer's at once, each later one when the next forward is a few
            # ops before it (launch_update_part), so the updates overlap the
            # forward's GEMMs rather than its attention
            side, model_parts = self._overlap
            with torch.cuda.stream(side):
                self.optimizer.step(
                    stats=st.stats if need_norm else None,
                    found_inf=st.found_inf if scaler is not None else None,
                    deferred=True,
                )
            self._unlaunched_parts = set(range(len(model_parts)))
            self._join_pending = True
            # the eager parts go out before the per-parameter bookkeeping,
            # which the GPU would otherwise wait for at the step boundary
            eager = min(self.eager_update_parts, len(model_parts))
            # (the side stream waited for the current one above; since then
            # only the statistics read-back is queued there, which the update
            # does not touch)
            for k in range(eager):
                self.launch_update_part(k, wait=False)
            for k, (part, ev) in enumerate(zip(model_parts, self.optimizer.part_events)):
                launch = functools.partial(self.launch_update_part, k) if k >= eager else None
                for p in part:
                    p._eth_ready_event = ev
                    p._eth_ready_part = part
                    p._eth_update_launch = launch
            if scaler is None:
                # no overflow to wait for: the step counters advance now
                self.optimizer.commit_step(True)
        if host is not None:
            host[1].synchronize()
        if scaler is not None:
            found = bool(host[0][1][0].item() > 0)
            scaler.update(found)
            self.optimizer.commit_step(not found)
            if self._executor is not None:
                self._executor.set_inv_loss_scale(self._inv_scale())
            if found:
                return False, None, None
        grad_norm = float(host[0][0][1].item()) if need_norm else None
        num_zeros = self.count_zeros() if self.log_num_zeros_in_grad else None
        return True, grad_norm, num_zeros

    def _read_back(self, st):
        """Queue copies of stats ([Σg², ‖g‖, clip]) and found_inf into pinned
        host memory on the current stream; returns ((stats, found_inf) host
        tensors, event marking the copies)."""
        dev = self._device()
        if self._host_flags is None:
            self._host_flags = (torch.empty(3, dtype=torch.float64, pin_memory=True),
                                torch.empty(1, dtype=torch.float32, pin_memory=True))
        host_stats, host_inf = self._host_flags
        # two direct copies into pinned memory, no device staging kernels
        host_stats.copy_(st.stats, non_blocking=True)
        host_inf.copy_(st.found_inf.reshape(-1)[0:1], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dev))
        return (host_stats, host_inf), ev

    def zero_grad(self, set_to_none=True):
        for p in self.get_parameters():
            p.grad = None

    def state_dict(self):
        out = {"optimizer": self.optimizer.state_dict()}
        if self.grad_scaler is not None:
            out["grad_scaler"] = self.grad_scaler.state_dict()
        return out


class Float16OptimizerWithFloat16Params(MegatronOptimizer):
    """bf16/fp16 model parameters with fp32 masters
    (eth/runtime/megatron/optimizer/optimizer.py:228-572)."""

    def __init__(
        self,
        param_groups,
        lr,
        betas,
        eps,
        weight_decay,
        clip_grad,
        log_num_zeros_in_grad=False,
        params_have_main_grad=True,
        use_contiguous_buffers_in_ddp=True,
        bf16=True,
        grad_scaler=None,
    ):
        self.float16_groups = []
        self.fp32_from_float16_groups = []
        self.fp32_from_fp32_groups = []
        model_params = [p for g in param_groups for p in g["params"]]
        half = [p for p in model_params if p.dtype in (torch.float16, torch.bfloat16)]
        self._master_flat, masters = _flat_master_copies(half) if half else (None, [])
        master_of = {id(p): m for p, m in zip(half, masters)}
        groups = []
        for g in param_groups:
            f16, f32m, f32 = [], [], []
            for p in g["params"]:
                if id(p) in master_of:
                    f16.append(p)
                    f32m.append(master_of[id(p)])
                elif p.dtype == torch.float32:
                    f32.append(p)
                else:
                    raise TypeError(f"unsupported parameter dtype {p.dtype}")
            self.float16_groups.append(f16)
            self.fp32_from_float16_groups.append(f32m)
            self.fp32_from_fp32_groups.append(f32)
            ng = {k: v for k, v in g.items() if k != "params"}
            ng["params"] = f32m + f32
            groups.append(ng)
        optimizer = FusedAdamW(groups, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        super().__init__(optimizer, clip_grad, log_num_zeros_in_grad, params_have_main_grad)
        self.bf16 = bf16
        self.grad_scaler = grad_scaler
        self._f32_grads = {}
        self._f32_flat = None
        self._widen = {}  # {id(master): 16-bit main grad} widened by this step's statistics pass
        self.use_contiguous_buffers_in_ddp = use_contiguous_buffers_in_ddp
        model_dtypes = {p.dtype for p in half}
        if len(model_dtypes) > 1:
            raise TypeError("mixed bf16/fp16 model parameters")
        if half:
            optimizer.set_model_copies({master_of[id(p)]: p for p in half}, half[0].dtype)
        for p in model_params:
            self._model_to_optimizer_param[id(p)] = master_of.get(id(p), p)

    def _bound_main_grads(self):
        out = []
        for mg, fg in zip(self.float16_groups, self.fp32_from_float16_groups):
            out.extend(getattr(p, "main_grad", None) for p in mg)
        for group in self.fp32_from_fp32_groups:
            out.extend(getattr(p, "main_grad", None) for p in group)
        return out

    def _fp32_grad_view(self, main_param):
        """The persistent fp32 gradient of a master whose main_grad is 16-bit
        (one flat buffer, carved in master order on first use), so the
        statistics and AdamW tables keyed by gradient addresses stay valid
        across steps."""
        view = self._f32_grads.get(id(main_param))
        if view is None:
            masters = [m for g in self.fp32_from_float16_groups for m in g]
            sizes = [(m.numel() + 3) // 4 * 4 for m in masters]  # 16-byte aligned views
            flat = torch.empty(sum(sizes), dtype=torch.float32, device=masters[0].device)
            self._f32_flat = flat
            off = 0
            for m, n in zip(masters, sizes):
                self._f32_grads[id(m)] = flat[off : off + m.numel()].view(m.shape)
                off += n
            view = self._f32_grads[id(main_param)]
        return view

    def _widen_sources(self):
        return self._widen

    def _widen_target(self):
        return self._f32_flat

    def _copy_model_grads_to_main_grads(self):
        self._widen = {}
        for mg, fg in zip(self.float16_groups, self.fp32_from_float16_groups):
            for model_param, main_param in zip(mg, fg):
                if self.params_have_main_grad:
                    g = model_param.main_grad
                    if g.dtype == torch.float32:
                        # (the alias usually stands from the previous step)
                        if main_param.grad is not g:
                            main_param.grad = g
                    else:
                        # main_grad.float() (optimizer.py:392-397) into a
                        # persistent buffer: an exact widening copy, which the
                        # step's statistics pass makes (eth_widen_grad_stats)
                        main_param.grad = self._fp32_grad_view(main_param)
                        self._widen[id(main_param)] = g
                elif model_param.grad is not None:
                    main_param.grad = model_param.grad.float()
                if model_param.grad is not None:
                    model_param.grad = None
        if self.params_have_main_grad:
            for group in self.fp32_from_fp32_groups:
                for p in group:
                    if p.grad is not p.main_grad:
                        p.grad = p.main_grad

    def _norm_owned(self, param):
        return super()._norm_owned(param)

    def _drop_model_parameter(self, param):
        for mg, fg in zip(self.float16_groups, self.fp32_from_float16_groups):
            for k, p in enumerate(mg):
                if p is param:
                    del mg[k], fg[k]
                    return

    def reload_model_params(self):
        for mg, fg in zip(self.float16_groups, self.fp32_from_float16_groups):
            for p, m in zip(mg, fg):
                m.data.copy_(p.data)


class FP32Optimizer(MegatronOptimizer):
    """fp32 model parameters (eth/runtime/megatron/optimizer/optimizer.py:576-659)."""

    def __init__(self, param_groups, lr, betas, eps, weight_decay, clip_grad, log_num_zeros_in_grad=False, params_have_main_grad=True):
        optimizer = FusedAdamW(param_groups, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
        super().__init__(optimizer, clip_grad, log_num_zeros_in_grad, params_have_main_grad)
        for p in self.get_parameters():
            self._model_to_optimizer_param[id(p)] = p

    def _bound_main_grads(self):
        return [getattr(p, "main_grad", None) for p in self.get_parameters()]

    def _copy_model_grads_to_main_grads(self):
        if self.params_have_main_grad:
            for p in self.get_parameters():
                p.grad = p.main_grad


@torch.no_grad()
def step_model_parallel_group(optimizers):
    """One optimizer step of several pipeline stages that share one GPU, as
    the ranks of one model-parallel group step together: the clip norm is
    the L2 norm over every stage's gradients (clip_grads.py:100-113 sums the
    ranks' squared norms over the model-parallel group), the overflow flag
    is the maximum of the stages' flags (optimizer.py:449-461 takes it over
    every rank), so every stage skips or applies the step alike, and the
    zero count is the sum (clip_grads.py:150-155).  The stages' partial sums of squares are joined
    into one vector that every stage finalizes its norm from, in fp64.
    Returns [(update_successful, grad_norm, num_zeros)] per stage."""
    if not optimizers:
        return []
    clip = {o.clip_grad for o in optimizers}
    scaled = {o.grad_scaler is not None for o in optimizers}
    if len(clip) != 1 or len(scaled) != 1:
        raise ValueError("the stages of one group must clip alike and all (or none) scale the loss")
    if scaled == {True} and len({o.grad_scaler.host_scale for o in optimizers}) != 1:
        raise ValueError("the stages of one group must hold one loss scale")
    devices = {o._device() for o in optimizers}
    if len(devices) != 1:
        raise ValueError("the in-process group steps stages of one GPU")
    sts = [o.gather_statistics() for o in optimizers]
    if sts[0] is None:
        return [o.apply_statistics(None) for o in optimizers]
    if scaled == {True}:
        flag = sts[0].found_inf.clone()
        for st in sts[1:]:
            torch.maximum(flag, st.found_inf, out=flag)
        for st in sts:
            st.found_inf.copy_(flag)
    partials, n = None, None
    if clip.pop() > 0.0:
        parts = [st.partials[: st.n_partials_used] for st in sts if st.n_partials_used]
        partials = torch.cat(parts) if parts else sts[0].partials
        n = sum(st.n_partials_used for st in sts)
    out = [o.apply_statistics(st, partials, n) for o, st in zip(optimizers, sts)]
    zeros = [z for _, _, z in out]
    if all(z is not None for z in zeros):
        total = float(sum(zeros))
        out = [(ok, norm, total) for ok, norm, _ in out]
    return out


def get_params_for_weight_decay_optimization(modules, layernorm_types=()):
    """LayerNorm parameters and every `bias` get weight decay 0
    (eth/runtime/megatron/optimizer/__init__.py:37-58)."""
    from ..model.layers import LayerNorm

    ln_types = (LayerNorm, torch.nn.LayerNorm, *layernorm_types)
    decay = {"params": []}
    no_decay = {"params": [], "weight_decay": 0.0}
    for module in modules:
        for sub in module.modules():
            items = [(n, p) for n, p in sub._parameters.items() if p is not None]
            if isinstance(sub, ln_types):
                no_decay["params"].extend(p for _, p in items)
            else:
                decay["params"].extend(p for n, p in items if n != "bias")
                no_decay["params"].extend(p for n, p in items if n == "bias")
    return decay, no_decay


def get_megatron_optimizer(
    modules,
    lr,
    weight_decay,
    betas=(0.9, 0.999),
    eps=1e-8,
    clip_grad=1.0,
    fp16=False,
    bf16=False,
    loss_scale=None,
    initial_loss_scale=2.0**32,
    min_loss_scale=1.0,
    loss_scale_window=1000,
    hysteresis=2,
    log_num_zeros_in_grad=False,
    params_have_main_grad=True,
):
    """Factory with the decisions of eth/runtime/megatron/optimizer/__init__.py:61-126."""
    from .grad_scaler import ConstantGradScaler, DynamicGradScaler

    groups = [g for g in get_params_for_weight_decay_optimization(modules) if g["params"]]
    if fp16 or bf16:
        scaler = None
        device = groups[0]["params"][0].device
        if loss_scale:
            scaler = ConstantGradScaler(loss_scale, device=device)
        elif fp16:
            scaler = DynamicGradScaler(
                initial_scale=initial_loss_scale,
                min_scale=min_loss_scale,
                growth_factor=2.0,
                backoff_factor=0.5,
                growth_interval=loss_scale_window,
                hysteresis=hysteresis,
                device=device,
            )
        return Float16OptimizerWithFloat16Params(
            groups, lr, betas, eps, weight_decay, clip_grad, log_num_zeros_in_grad, params_have_main_grad, True, bf16, scaler
        )
    return FP32Optimizer(groups, lr, betas, eps, weight_decay, clip_grad, log_num_zeros_in_grad, params_have_main_grad)
