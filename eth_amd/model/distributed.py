"""Local DDP wrapper: contiguous main-grad buffers.

Restates eth/runtime/megatron/model/distributed.py:18-127: one buffer per
gradient dtype (fp32 when accumulate_allreduce_grads_in_fp32, which bf16
forces), parameters carved from the END of the buffer in
module.parameters() order, `param.main_grad` views, a hook that folds any
`param.grad` into main_grad and clears it, and zero_grad_buffer().  The HIP
autograd Functions accumulate straight into main_grad, so the hook only
fires for gradients produced outside them.  Zeroing uses a fill kernel (no
hipMemsetAsync).

zero_grad_buffer(defer=True) zeroes nothing: it marks every parameter's
main_grad stale, the first kernel to contribute a gradient then stores
instead of adding (`main_grad_target`), and settle_grad_buffer() zero-fills
whatever received no gradient before the buffer is read.  The values are
those of zero-then-accumulate (0 + g == g); the fill of the whole buffer and
the first read of every accumulation are saved.
"""

import torch
from torch import nn

from .. import _native as nat


def main_grad_target(param):
    """(main_grad, accumulate) for a kernel about to write param's gradient:
    accumulate is False for the first contribution after a deferred
    zero_grad_buffer() (the buffer then holds stale values and the kernel
    stores), True afterwards.  (None, False) without a main_grad."""
    mg = getattr(param, "main_grad", None)
    if mg is None:
        return None, False
    if getattr(param, "_eth_main_grad_stale", False):
        param._eth_main_grad_stale = False
        return mg, False
    return mg, True


def grad_written(param):
    """Called once the kernels that write param's gradient for the current
    backward have all been launched: a streamed gradient sync registered as
    `param._eth_on_grad` may then sync the buckets holding it."""
    cb = getattr(param, "_eth_on_grad", None)
    if cb is not None:
        cb(param)


def materialize_main_grad(param):
    """param.main_grad with real values: zero-filled now if it is stale."""
    mg = getattr(param, "main_grad", None)
    if mg is not None and getattr(param, "_eth_main_grad_stale", False):
        _zero(mg)
        param._eth_main_grad_stale = False
    return mg


def _zero(t):
    if t.dtype == torch.float32 and t.is_cuda and t.is_contiguous():
        nat.call("eth_fill_f32", nat.ptr(t), t.numel(), 0.0, nat.stream_ptr(t.device))
    else:
        t.zero_()


class MemoryBuffer:
    def __init__(self, numel, dtype, device):
        self.numel = numel
        self.dtype = dtype
        self.data = torch.zeros(numel, dtype=dtype, device=device)

    def zero(self):
        _zero(self.data)

    def get(self, shape, start_index):
        end = start_index + torch.Size(shape).numel()
        if end > self.numel:
            raise ValueError("requested tensor is out of the buffer range")
        return self.data[start_index:end].view(shape)


class DistributedDataParallel(nn.Module):
    def __init__(self, module, accumulate_allreduce_grads_in_fp32=True, use_contiguous_buffers=True):
        super().__init__()
        self.module = module
        self.accumulate_allreduce_grads_in_fp32 = accumulate_allreduce_grads_in_fp32
        self.use_contiguous_buffers = use_contiguous_buffers
        self._grad_buffers = {}
        self._initialize_main_grad_buffers()

    def _grad_dtype(self, p):
        return torch.float32 if self.accumulate_allreduce_grads_in_fp32 else p.dtype

    def _initialize_main_grad_buffers(self):
        numel, device = {}, {}
        for p in self.module.parameters():
            if not p.requires_grad:
                continue
            dt = self._grad_dtype(p)
            dev = torch.device(p.device)
            if device.setdefault(dt, dev) != dev:
                raise ValueError(f"parameters with gradient dtype {dt} span devices")
            numel[dt] = numel.get(dt, 0) + p.numel()
        self._grad_buffers = {dt: MemoryBuffer(n, dt, device[dt]) for dt, n in numel.items()}
        remaining = dict(numel)
        for p in self.module.parameters():
            if not p.requires_grad:
                continue
            dt = self._grad_dtype(p)
            remaining[dt] -= p.numel()
            p.main_grad = self._grad_buffers[dt].get(p.shape, remaining[dt])
        self._grad_params = [p for p in self.module.parameters() if p.requires_grad]
        self.grad_accs = []
        for p in self.module.parameters():
            if not p.requires_grad:
                continue
            acc = p.expand_as(p).grad_fn.next_functions[0][0]
            acc.register_hook(self._make_param_hook(p))
            self.grad_accs.append(acc)

    @staticmethod
    def _make_param_hook(param):
        def hook(*unused):
            if param.grad is not None:
                mg, accumulate = main_grad_target(param)
                if accumulate:
                    mg.add_(param.grad.data)
                else:
                    mg.copy_(param.grad.data)
                param.grad = None
                grad_written(param)

        return hook

    def zero_grad_buffer(self, defer=False):
        if defer:
            for p in self._grad_params:
                p._eth_main_grad_stale = True
            return
        for buf in self._grad_buffers.values():
            buf.zero()
        for p in self._grad_params:
            p._eth_main_grad_stale = False

    def settle_grad_buffer(self):
        """Zero-fill the main_grad of every parameter that received no
        gradient since a deferred zero_grad_buffer(); afterwards the whole
        buffer holds the step's gradients."""
        for p in self._grad_params:
            materialize_main_grad(p)

    @property
    def grad_buffers(self):
        return self._grad_buffers

    def forward(self, *args, **kwargs):
        return self.module(*args, **kwargs)
