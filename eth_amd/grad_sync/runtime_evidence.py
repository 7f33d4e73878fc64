"""Opt-in record of what every gradient collective carried.

Writes `rank-{rank:05d}.json` in the layout of
eth/runtime/megatron/grad_sync/runtime_evidence.py:21-138 (same keys and
meaning), so the reference's tools/validation/compare_runtime_evidence.py
can judge a run of this build: per execution the normalization scale, the
collective count, the payload bytes, every packed bucket's SHA-256 and the
SHA-256 of all packed payloads back to back, plus the process-group and
scratch-allocation signatures that must stay stable across executions.

The payloads live in device memory.  Instead of a blocking copy per bucket,
each packed payload is copied into one of two pinned host slots on the
stream that packed it (before the collective seam can change it), and the
host hashes a slot while the device goes on with the next buckets; a slot is
only reused after its hash is taken.  The hashes are those of the payload
bytes, so they are independent of how the copy is scheduled.
"""

import collections
import hashlib
import json
from pathlib import Path

import torch


def scratch_signature(scratch):
    """((dtype, numel, storage address), ...) of the executor's scratch."""
    return tuple(
        (dtype, int(t.numel()), int(t.untyped_storage().data_ptr())) for dtype, t in sorted(scratch.items())
    )


def _signature_records(signature):
    return [{"dtype": d, "numel": n, "data_ptr": p} for d, n, p in signature]


class _PinnedSlots:
    """Two pinned host buffers, each with the event marking its last copy."""

    def __init__(self, nbytes):
        self.host = [torch.empty(max(1, nbytes), dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.pending = collections.deque()  # (bucket, slot, nbytes, event)
        self.next = 0


class GradientRuntimeEvidenceRecorder:
    def __init__(self, plan, global_rank, registry, scratch, output_dir):
        self._plan = plan
        self._rank = int(global_rank)
        self._registry = registry
        self._scratch = scratch
        self._output_dir = Path(output_dir)
        self._groups0 = int(registry.group_count)
        self._creations0 = int(registry.creation_count)
        self._scratch0 = scratch_signature(scratch)
        self._iterations = []
        self._current = None
        self._run_hash = None
        self._slots = None

    # ------------------------------------------------------------ phases --
    def begin_execution(self, normalization_scale):
        if self._current is not None:
            raise RuntimeError("runtime evidence execution already active")
        self._run_hash = hashlib.sha256()
        self._current = {
            "iteration": len(self._iterations) + 1,
            "normalization_scale": float(normalization_scale),
            "collective_count": 0,
            "payload_bytes": 0,
            "buckets": [],
        }

    def observe_packed_bucket(self, bucket, payload):
        """Record one packed payload.  A device payload is staged through a
        pinned slot on the current stream and hashed later (in order); a host
        payload is hashed now."""
        if self._current is None:
            raise RuntimeError("runtime evidence execution is not active")
        flat = payload.detach().reshape(-1).view(torch.uint8)
        if not flat.is_cuda:
            self._record(bucket, flat.contiguous().numpy().tobytes())
            return
        if self._slots is None:
            biggest = max((b.exact_bytes for b in self._plan.global_bucket_order), default=1)
            self._slots = _PinnedSlots(biggest)
        slots = self._slots
        if len(slots.pending) == len(slots.host):
            self._drain_one()
        slot = slots.next
        slots.next = (slot + 1) % len(slots.host)
        n = flat.numel()
        slots.host[slot][:n].copy_(flat, non_blocking=True)
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(flat.device))
        slots.pending.append((bucket, slot, n, event))

    def finish_execution(self):
        if self._current is None:
            raise RuntimeError("runtime evidence execution is not active")
        while self._slots is not None and self._slots.pending:
            self._drain_one()
        cur = self._current
        cur["packed_payload_sha256"] = self._run_hash.hexdigest()
        cur["process_group_count"] = int(self._registry.group_count)
        cur["process_group_creation_count"] = int(self._registry.creation_count)
        cur["scratch_signature"] = _signature_records(scratch_signature(self._scratch))
        self._iterations.append(cur)
        self._current = None
        self._run_hash = None
        self._write()

    # ----------------------------------------------------------- helpers --
    def _drain_one(self):
        bucket, slot, n, event = self._slots.pending.popleft()
        event.synchronize()
        self._record(bucket, self._slots.host[slot][:n].numpy().tobytes())

    def _record(self, bucket, raw):
        self._run_hash.update(raw)
        cur = self._current
        cur["collective_count"] += 1
        cur["payload_bytes"] += len(raw)
        cur["buckets"].append(
            {
                "bucket_id": bucket.bucket_id,
                "semantic_hash": bucket.semantic_hash,
                "process_group_id": bucket.process_group_id,
                "exact_numel": int(bucket.exact_numel),
                "exact_bytes": int(bucket.exact_bytes),
                "packed_payload_sha256": hashlib.sha256(raw).hexdigest(),
            }
        )

    def report(self):
        plan, its = self._plan, self._iterations
        now = scratch_signature(self._scratch)
        return {
            "version": 1,
            "global_rank": self._rank,
            "sync_mode": plan.sync_mode,
            "global_topology_hash": plan.global_topology_hash,
            "global_manifest_hash": plan.global_manifest_hash,
            "global_fragment_hash": plan.global_fragment_hash,
            "global_plan_hash": plan.global_plan_hash,
            "exact_payload_bytes_by_rank": [[int(r), int(v)] for r, v in plan.exact_payload_bytes_by_rank],
            "padding_payload_bytes": int(plan.padding_payload_bytes),
            "process_group_count": self._groups0,
            "process_group_creation_count": self._creations0,
            "scratch": _signature_records(self._scratch0),
            "process_group_count_stable": all(i["process_group_count"] == self._groups0 for i in its),
            "process_group_creation_count_stable": all(
                i["process_group_creation_count"] == self._creations0 for i in its
            ),
            "scratch_stable": now == self._scratch0
            and all(i["scratch_signature"] == _signature_records(self._scratch0) for i in its),
            "iterations": its,
        }

    def _write(self):
        self._output_dir.mkdir(parents=True, exist_ok=True)
        path = self._output_dir / f"rank-{self._rank:05d}.json"
        tmp = path.with_name(path.name + ".tmp")
        tmp.write_text(json.dumps(self.report(), indent=2, sort_keys=True) + "\n", encoding="utf-8")
        tmp.replace(path)
