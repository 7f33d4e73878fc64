"""FusedAdamW: torch.optim-compatible AdamW whose step is one HIP launch.

Drop-in for the optimizer built by
eth/runtime/megatron/optimizer/__init__.py:61-72 (apex FusedAdam in AdamW
mode, falling back to torch.optim.AdamW): same param_groups keys
(params, lr, betas, eps, weight_decay) and the same per-parameter state
(`step`, `exp_avg`, `exp_avg_sq`) that evidence and checkpoints read.

Moment buffers of all parameters live in two flat fp32 allocations (one
view per parameter), and the per-step launch walks a device table of
(tensor, chunk) records built once; the table is rebuilt only when a
parameter's or gradient's storage changes.
"""

import numpy as np
import torch

from .. import _native as nat


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        if lr < 0.0 or eps < 0.0 or weight_decay < 0.0:
            raise ValueError("invalid AdamW hyper-parameter")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        defaults = dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay)
        super().__init__(params, defaults)
        self._table_key = None
        self._tables = None
        self._model_copies = {}
        self._model_dtype = nat.ETH_F32
        self._partition = None
        self.part_events = []
        self._allocate_state()

    # ---------------------------------------------------------------- state --
    def _all_params(self):
        return [p for g in self.param_groups for p in g["params"]]

    def _allocate_state(self):
        params = self._all_params()
        for p in params:
            if p.dtype != torch.float32:
                raise ValueError("FusedAdamW keeps fp32 parameters (masters); got " + str(p.dtype))
            if not p.is_contiguous():
                raise ValueError("FusedAdamW parameters must be contiguous")
        if not params:
            return
        device = params[0].device
        # 16-byte aligned views: pad every tensor to a multiple of 4 elements
        sizes = [(p.numel() + 3) // 4 * 4 for p in params]
        total = sum(sizes)
        self._exp_avg_flat = torch.zeros(total, dtype=torch.float32, device=device)
        self._exp_avg_sq_flat = torch.zeros(total, dtype=torch.float32, device=device)
        off = 0
        for p, n in zip(params, sizes):
            st = self.state[p]
            st["step"] = torch.tensor(0.0)
            st["exp_avg"] = self._exp_avg_flat[off : off + p.numel()].view_as(p)
            st["exp_avg_sq"] = self._exp_avg_sq_flat[off : off + p.numel()].view_as(p)
            off += n

    def remove_param(self, param):
        """Stop updating `param`: it leaves its group, its state, its model
        copy and the partition (its moment views stay allocated, unused)."""
        for g in self.param_groups:
            g["params"] = [q for q in g["params"] if q is not param]
        self.state.pop(param, None)
        self._model_copies.pop(param, None)
        if self._partition:
            self._partition = [[q for q in part if q is not param] for part in self._partition]
        self._table_key = None

    def set_partition(self, parts):
        """Split every step into one launch per part (a list of parameter
        lists, in launch order; parameters in no part form a last part),
        with a HIP event recorded after each launch in `part_events`, so
        later work can wait for the parameters it reads only."""
        self._partition = [list(part) for part in parts] if parts else None
        self._table_key = None

    def set_model_copies(self, mapping, model_dtype):
        """Master parameter -> 16-bit model parameter written by every step."""
        self._model_copies = dict(mapping)
        self._model_dtype = nat.dtype_code(model_dtype)
        self._table_key = None

    # ---------------------------------------------------------------- table --
    def _key(self):
        return tuple(
            (p.data_ptr(), p.grad.data_ptr() if p.grad is not None else 0, g["lr"], g["weight_decay"])
            for g in self.param_groups
            for p in g["params"]
        )

    def _parts(self):
        if not self._partition:
            return [[p for g in self.param_groups for p in g["params"]]]
        placed = {id(p) for part in self._partition for p in part}
        rest = [p for g in self.param_groups for p in g["params"] if id(p) not in placed]
        return [*self._partition, rest] if rest else list(self._partition)

    def _build_tables(self):
        group_of = {id(p): g for g in self.param_groups for p in g["params"]}
        cap = nat.CHUNK_ELEMS
        device = self._all_params()[0].device
        self._tables = []
        for part in self._parts():
            tensors, chunks = [], []
            for p in part:
                if p.grad is None:
                    continue
                if p.grad.dtype != torch.float32 or not p.grad.is_contiguous() or p.grad.shape != p.shape:
                    raise ValueError("FusedAdamW needs contiguous fp32 gradients shaped like the parameter")
                g = group_of[id(p)]
                st = self.state[p]
                model = self._model_copies.get(p)
                idx = len(tensors)
                tensors.append(
                    (
                        p.data_ptr(),
                        p.grad.data_ptr(),
                        st["exp_avg"].data_ptr(),
                        st["exp_avg_sq"].data_ptr(),
                        model.data_ptr() if model is not None else 0,
                        p.numel(),
                        float(g["lr"]),
                        float(g["weight_decay"]),
                    )
                )
                for start in range(0, p.numel(), cap):
                    chunks.append((idx, min(cap, p.numel() - start), start))
            ttab = np.zeros(len(tensors), dtype=nat.ADAM_TENSOR_DTYPE)
            for i, name in enumerate(nat.ADAM_TENSOR_DTYPE.names):
                ttab[name] = [t[i] for t in tensors]
            ctab = np.zeros(len(chunks), dtype=nat.ADAM_CHUNK_DTYPE)
            if chunks:
                arr = np.asarray(chunks, dtype=np.int64)
                ctab["tensor"] = arr[:, 0]
                ctab["n"] = arr[:, 1]
                ctab["start"] = arr[:, 2]
            self._tables.append(
                (
                    nat.table_to_device(ttab, device) if len(ttab) else None,
                    nat.table_to_device(ctab, device) if len(ctab) else None,
                    len(ctab),
                )
            )

    # ----------------------------------------------------------------- step --
    @torch.no_grad()
    def step(self, closure=None, stats=None, found_inf=None, deferred=False):
        """One AdamW step.  `stats` (device double[3], clip coefficient at
        index 2) and `found_inf` (device float[1]) are optional; with
        found_inf set to non-zero the launch leaves every tensor unchanged.
        With `deferred` (a partitioned optimizer) nothing is launched yet:
        launch_part(k) later issues part k, on the stream step() ran on, and
        records part_events[k] after it; a wait on an event must come after
        its part's launch."""
        loss = closure() if closure is not None else None
        params = self._all_params()
        if not params:
            return loss
        key = self._key()
        if key != self._table_key:
            self._build_tables()
            self._table_key = key
        groups = {(g["betas"], g["eps"]) for g in self.param_groups}
        if len(groups) != 1:
            raise ValueError("FusedAdamW needs identical betas/eps across parameter groups")
        (beta1, beta2), eps = next(iter(groups))
        # all parameters step together; the state mirrors torch's per-param step
        step = int(self.state[params[0]]["step"].item()) + 1
        device = params[0].device
        if deferred and not self._partition:
            raise ValueError("a deferred step needs a partition (set_partition)")
        self._launch_stream = torch.cuda.current_stream(device)
        self._launches = [
            (nat.ptr(ttab), nat.ptr(ctab), n_chunks, float(beta1), float(beta2), float(eps), step,
             self._model_dtype, nat.ptr(stats), nat.ptr(found_inf), nat.stream_ptr(device))
            if n_chunks else None
            for ttab, ctab, n_chunks in self._tables
        ]
        self._launched = [False] * len(self._launches)
        if not self._partition:
            self.part_events = []
        elif len(self.part_events) != len(self._launches):
            # one event per part, re-recorded every step (a wait already
            # queued on it keeps the recording it was queued behind)
            self.part_events = [torch.cuda.Event() for _ in self._launches]
        if not deferred:
            for k in range(len(self._launches)):
                self.launch_part(k)
        self._pending_step = step
        if found_inf is None and not deferred:
            # (a deferred step's caller commits once its first parts are out)
            self.commit_step(True)
        return loss

    def launch_part(self, k):
        """Issue part k of the last step(), once (every part when the
        optimizer is not partitioned), on the stream step() ran on."""
        if self._launched[k]:
            return
        self._launched[k] = True
        args = self._launches[k]
        if args is not None:
            nat.call("eth_adam_step", *args)
        if self._partition:
            self.part_events[k].record(self._launch_stream)

    def launch_all(self):
        for k in range(len(getattr(self, "_launches", ()))):
            self.launch_part(k)

    def commit_step(self, applied=True):
        """Advance the per-parameter step counters after a launched step
        (skipped steps on overflow leave them unchanged, as torch does when
        step() is not called)."""
        step = getattr(self, "_pending_step", None)
        if step is None:
            return
        if applied:
            for p in self._all_params():
                if p.grad is not None:
                    self.state[p]["step"].fill_(float(step))
        self._pending_step = None
