"""Bucket-by-bucket gradient sync overlapped with the backward pass.

The reference runs GradientSyncManager.execute after the whole backward
(eth/runtime/megatron/training.py:904-1068 with grad_sync/manager.py:31-32):
every bucket is packed, all-reduced and unpacked once the last gradient of
the step exists.  Here a bucket is synced as soon as the kernels writing all
of its parameters' gradients have been launched: `grad_written(param)`
(model/distributed.py) reports each parameter once per backward, and the
bucket's pack -> all_reduce_sum seam -> fused unpack goes to a dedicated
stream (default priority) that first waits for the streams that wrote the
gradients.  Buckets whose parameters received no gradient are zero-settled
and synced at the end.  The per-bucket work is exactly executor.run_bucket,
so the payloads, main grads and statistics are those of execute(); only the
time they are computed at moves.  (The scratch a streamed pass leaves behind
can differ where a plan-order pass would have packed over a chunk, whose
normalization write-back the unpack skips; nothing reads it.)  What it overlaps with the backward is the
all-reduce seam's communication; the local pack/unpack memory traffic itself
competes with the backward's kernels (on one GPU it costs the GEMMs about
what it hides).

Valid for a backward that produces each gradient in full, i.e. the last (here
the only) micro-batch before the sync.
"""

import torch

from .. import kernels as K
from ..model.distributed import materialize_main_grad


class StreamedGradSync:
    def __init__(self, executor, device):
        self.ex = executor
        self.device = torch.device(device)
        self.buckets = executor.bucket_parameters()
        self.where = {}
        for b, params in enumerate(self.buckets):
            for p in params:
                self.where.setdefault(id(p), []).append(b)
        self.params = {id(p): p for params in self.buckets for p in params}
        self.stream = torch.cuda.Stream(device=self.device)
        self._active = False

    def start(self, normalization_scale=1.0):
        """Arm the sync for the backward about to run."""
        main = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(main)
        with torch.cuda.stream(self.stream):
            self.ex.begin(normalization_scale)
        self.remaining = [len(ps) for ps in self.buckets]
        self.launched = [False] * len(self.buckets)
        self.seen = set()
        for p in self.params.values():
            p._eth_on_grad = self._on_grad
        self._active = True

    def _on_grad(self, param):
        if id(param) in self.seen:
            return
        self.seen.add(id(param))
        for b in self.where.get(id(param), ()):
            self.remaining[b] -= 1
            if self.remaining[b] == 0:
                self._launch(b)

    def _launch(self, b):
        main = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(main)
        self.stream.wait_stream(K.side_stream(self.device))
        with torch.cuda.stream(self.stream):
            for p in self.buckets[b]:
                materialize_main_grad(p)  # a parameter that got no gradient
            self.ex.run_bucket(b)
        self.launched[b] = True

    def finish(self):
        """Sync every bucket not synced yet, close the pass and make the
        current stream wait for all of it."""
        if not self._active:
            return
        for p in self.params.values():
            p._eth_on_grad = None
        for b, done in enumerate(self.launched):
            if not done:
                self._launch(b)
        with torch.cuda.stream(self.stream):
            self.ex.end()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        self._active = False
