"""Execution of an immutable gradient synchronization plan on the GPU.

Drop-in for eth/runtime/megatron/grad_sync/executor.py:24-261
(GradientBucketExecutor): same constructor (including the opt-in
`runtime_evidence_dir`, grad_sync/runtime_evidence.py), `execute(
normalization_scale)`, `scratch(dtype)`, `scratch_dtypes`, same validation
errors carrying `bucket {id} rank {r} logical_param_id {id} fragment {id}`
context.

What differs is how a bucket is moved.  Instead of one `copy_` per segment
plus a `mul_` per bucket, every segment of every bucket is resolved once, at
construction, into a device table of chunks (2-D strided blocks of at most
ETH_CHUNK_ELEMS elements).  Per bucket and step the executor then issues one
pack launch, the unchanged `all_reduce_sum(payload, handle)` collective seam,
and one unpack launch that also applies the normalization scale.  When an
optimizer binds a GradientStatistics object, the same unpack launch also
unscales the gradients, raises the inf/nan flag and writes per-chunk sums of
squares for the global L2 norm, so the optimizer does not re-read them.
With the identity seam (`local_all_reduce_sum`: a data-parallel group of one
rank) and no evidence recorder, one native call issues the whole pass, so
the host is not the bottleneck of a pass of many small buckets.
"""

import ctypes
import math

import numpy as np
import torch

from .. import _native as nat
from .runtime_evidence import GradientRuntimeEvidenceRecorder


def local_all_reduce_sum(payload, handle):
    """The all-reduce of a process group that holds this rank alone: the
    payload is already the sum (torch.distributed.all_reduce over one rank)."""
    return None


def _dtype_name(dtype):
    return str(dtype).removeprefix("torch.")


def _normalize_axis(axis, shape, logical_param_id):
    if axis < 0:
        axis += len(shape)
    if not 0 <= axis < len(shape):
        raise ValueError(f"logical_param_id {logical_param_id} has invalid partition axis {axis}")
    return axis


def split_block(base, elem_size, rows, row_len, stride, dst, scale, flags, out):
    """Append chunks covering a rows x row_len block (row stride `stride`)."""
    cap = nat.CHUNK_ELEMS
    if rows == 1 or row_len == stride:
        total = rows * row_len
        for start in range(0, total, cap):
            n = min(cap, total - start)
            out.append((base + start * elem_size, dst + start, n, 1, n, scale, flags))
        return
    if row_len >= cap:
        for r in range(rows):
            for start in range(0, row_len, cap):
                n = min(cap, row_len - start)
                out.append((base + (r * stride + start) * elem_size, dst + r * row_len + start, stride, 1, n, scale, flags))
        return
    per = max(1, cap // row_len)
    for r0 in range(0, rows, per):
        nr = min(per, rows - r0)
        out.append((base + r0 * stride * elem_size, dst + r0 * row_len, stride, nr, row_len, scale, flags))


def chunk_table(entries):
    table = np.zeros(len(entries), dtype=nat.CHUNK_DTYPE)
    if entries:
        cols = list(zip(*entries))
        table["src"] = np.asarray(cols[0], dtype=np.uint64)
        table["dst"] = cols[1]
        table["src_stride"] = cols[2]
        table["rows"] = cols[3]
        table["row_len"] = cols[4]
        table["scale"] = cols[5]
        table["flags"] = cols[6]
    return table


def shadowed_prefixes(buckets):
    """Per bucket of a pass in plan order, the payload prefix (elements) of
    its scratch buffer that a later bucket of the same grad dtype packs over.
    The normalization write-back of a chunk inside that prefix is overwritten
    unread, so the unpack may skip it and the pass still leaves the scratch as
    the reference's in-place payload.mul_ does (executor.py:247-261)."""
    covered = [0] * len(buckets)
    reach = {}
    for i in range(len(buckets) - 1, -1, -1):
        covered[i] = reach.get(buckets[i].grad_dtype, 0)
        reach[buckets[i].grad_dtype] = max(covered[i], buckets[i].exact_numel)
    return covered


def mark_shadowed(entries, shadow):
    """Set ETH_CHUNK_SHADOWED on the chunk entries (split_block tuples) lying
    wholly inside the first `shadow` payload elements."""
    return [e[:6] + (e[6] | nat.CHUNK_SHADOWED,) if e[1] + e[3] * e[4] <= shadow else e for e in entries]


class GradientStatistics:
    """Device-side found_inf flag, per-chunk L2 partials and the finalized
    [sum of squares, norm, clip coefficient] of one optimizer step."""

    def __init__(self, n_partials, device):
        self.device = torch.device(device)
        self.found_inf = torch.zeros(1, dtype=torch.float32, device=self.device)
        self.partials = torch.zeros(max(1, n_partials), dtype=torch.float64, device=self.device)
        self.stats = torch.zeros(3, dtype=torch.float64, device=self.device)
        self.n_partials = n_partials
        self.n_partials_used = n_partials
        self.fresh = False
        self.inv_scale_used = None
        # called before the buffers are rewritten: an update still reading
        # the previous step's values is issued and waited for first
        self.before_reuse = None
        self.generation = 0  # counts resets: statistics taken after one belong to that pass

    def reset(self):
        if self.before_reuse is not None:
            self.before_reuse()
        self.generation += 1
        nat.call("eth_fill_f32", nat.ptr(self.found_inf), 1, 0.0, nat.stream_ptr(self.device))

    def finalize(self, max_norm):
        nat.call(
            "eth_grad_norm_finalize",
            nat.ptr(self.partials),
            self.n_partials_used,
            float(max_norm),
            nat.ptr(self.stats),
            nat.stream_ptr(self.device),
        )


class GradientBucketExecutor:
    def __init__(
        self,
        plan,
        global_rank,
        local_descriptors,
        local_runtime_bindings,
        process_group_registry,
        all_reduce_sum,
        runtime_evidence_dir=None,
    ):
        self.plan = plan
        self.global_rank = global_rank
        self._registry = process_group_registry
        self._all_reduce_sum = all_reduce_sum
        self._fragments = {f.fragment_id: f for f in plan.canonical_fragments}
        self._groups = {g.process_group_id: g for g in plan.process_groups}
        self._descriptors = self._unique_by_logical_id(local_descriptors, "descriptor")
        self._runtime_bindings = self._unique_by_logical_id(local_runtime_bindings, "runtime binding")
        self._binding_specs = {
            b.fragment_id: b
            for rank, bindings in plan.local_fragment_bindings_by_rank
            if rank == global_rank
            for b in bindings
        }
        self._validate_local_contract()
        self._scratch = self._allocate_scratch()
        self._norm_excluded = frozenset()
        self._tables = self._build_tables()
        self._statistics = None
        self._inv_scale = 1.0
        self._pass = None
        # opt-in record of every packed payload (executor.py:59-67,248-260)
        self._evidence = (
            GradientRuntimeEvidenceRecorder(plan, global_rank, process_group_registry, self._scratch,
                                            runtime_evidence_dir)
            if runtime_evidence_dir
            else None
        )

    # ------------------------------------------------------------ contract --
    @staticmethod
    def _unique_by_logical_id(items, kind):
        out = {}
        for item in items:
            if item.logical_param_id in out:
                raise ValueError(f"duplicate {kind} for logical_param_id {item.logical_param_id}")
            out[item.logical_param_id] = item
        return out

    def _rank_buckets(self):
        for bucket in self.plan.global_bucket_order:
            if self.global_rank in self._groups[bucket.process_group_id].ranks:
                yield bucket

    def _bucket_error(self, bucket, message, binding=None):
        context = f"bucket {bucket.bucket_id} rank {self.global_rank}"
        if binding is not None:
            context += f" logical_param_id {binding.logical_param_id} fragment {binding.fragment_id}"
        return ValueError(f"{context}: {message}")

    def _validate_local_contract(self):
        devices = set()
        for bucket in self._rank_buckets():
            for placement in bucket.placements:
                binding = self._binding_specs.get(placement.fragment_id)
                if binding is None:
                    frag = self._fragments[placement.fragment_id]

                    class _Missing:
                        logical_param_id = frag.logical_param_id
                        fragment_id = frag.fragment_id

                    raise self._bucket_error(bucket, "missing local binding", _Missing)
                runtime = self._runtime_bindings.get(binding.logical_param_id)
                descriptor = self._descriptors.get(binding.logical_param_id)
                if runtime is None or descriptor is None:
                    raise self._bucket_error(bucket, "missing descriptor or main_grad binding", binding)
                if tuple(runtime.main_grad.shape) != tuple(binding.source_segments[0].source_shape):
                    raise self._bucket_error(bucket, "main_grad shape mismatch", binding)
                if _dtype_name(runtime.main_grad.dtype) != bucket.grad_dtype.removeprefix("torch."):
                    raise self._bucket_error(bucket, "main_grad dtype mismatch", binding)
                if torch.device(runtime.main_grad.device) != torch.device(runtime.device):
                    raise self._bucket_error(bucket, "main_grad device mismatch", binding)
                devices.add(torch.device(runtime.main_grad.device))
        if len(devices) > 1:
            raise ValueError(
                f"rank {self.global_rank} has multiple gradient execution devices: {sorted(map(str, devices))}"
            )
        self._device = next(iter(devices), None)
        if self._device is not None and self._device.type != "cuda":
            raise ValueError(
                f"rank {self.global_rank}: the eth_amd executor runs on the GPU only, got {self._device}"
            )

    def _allocate_scratch(self):
        wanted = {
            dtype: numel
            for (rank, dtype), numel in self.plan.max_scratch_numel_by_rank_and_dtype
            if rank == self.global_rank
        }
        if not wanted:
            return {}
        if self._device is None:
            raise ValueError(f"rank {self.global_rank} participates in gradient buckets without a device")
        by_name = {_dtype_name(r.main_grad.dtype): r.main_grad.dtype for r in self._runtime_bindings.values()}
        scratch = {}
        for name, numel in wanted.items():
            dtype = by_name.get(name.removeprefix("torch."))
            if dtype is None:
                raise ValueError(f"rank {self.global_rank} has no main_grad with dtype {name}")
            scratch[name] = torch.empty(numel, dtype=dtype, device=self._device)
        return scratch

    @property
    def scratch_dtypes(self):
        return tuple(sorted(self._scratch))

    def scratch(self, dtype_name):
        return self._scratch[dtype_name]

    # -------------------------------------------------------- chunk tables --
    def _segment_block(self, binding, segment):
        """(address, rows, row_len, stride) of one segment of main_grad."""
        runtime = self._runtime_bindings[binding.logical_param_id]
        descriptor = self._descriptors[binding.logical_param_id]
        grad = runtime.main_grad
        if not grad.is_contiguous():
            raise ValueError(f"logical_param_id {binding.logical_param_id} main_grad must be contiguous")
        esize = grad.element_size()
        tensor_parallel = getattr(descriptor, "tensor_parallel", descriptor.partition_dim >= 0)
        if not tensor_parallel:
            if segment.flattened_numel != grad.numel():
                raise ValueError(f"logical_param_id {binding.logical_param_id} replicated source numel mismatch")
            return grad.data_ptr(), 1, grad.numel(), grad.numel()
        shape = tuple(grad.shape)
        axis = _normalize_axis(descriptor.partition_dim, shape, binding.logical_param_id)
        if math.prod(segment.source_shape) != grad.numel():
            raise ValueError(f"logical_param_id {binding.logical_param_id} source shape mismatch")
        if segment.source_dim_offset + segment.source_dim_length > shape[axis] or segment.source_dim_offset < 0:
            raise ValueError(f"logical_param_id {binding.logical_param_id} segment outside the tensor")
        outer = math.prod(shape[:axis])
        inner = math.prod(shape[axis + 1 :])
        addr = grad.data_ptr() + segment.source_dim_offset * inner * esize
        return addr, outer, segment.source_dim_length * inner, shape[axis] * inner

    def _build_tables(self):
        tables = []
        partial_base = 0
        buckets = list(self._rank_buckets())
        for bucket, shadow in zip(buckets, shadowed_prefixes(buckets)):
            entries = []
            for placement in bucket.placements:
                fragment = self._fragments[placement.fragment_id]
                binding = self._binding_specs[placement.fragment_id]
                owned = (fragment.include_in_optimizer_norm and fragment.norm_owner_rank == self.global_rank
                         and binding.logical_param_id not in self._norm_excluded)
                flags = nat.CHUNK_NORM if owned else 0
                esize = self._runtime_bindings[binding.logical_param_id].main_grad.element_size()
                dst = placement.destination_offset
                copied = 0
                for segment in binding.source_segments:
                    addr, rows, row_len, stride = self._segment_block(binding, segment)
                    n = rows * row_len
                    if n != segment.flattened_numel:
                        raise self._bucket_error(bucket, "source segment numel mismatch", binding)
                    if dst + n > bucket.exact_numel:
                        raise self._bucket_error(bucket, "placement exceeds exact_numel", binding)
                    split_block(addr, esize, rows, row_len, stride, dst, float(binding.contribution_scale), flags, entries)
                    dst += n
                    copied += n
                if copied != fragment.numel:
                    raise self._bucket_error(bucket, f"packed {copied} elements, expected {fragment.numel}", binding)
            table = chunk_table(mark_shadowed(entries, shadow))
            dev = nat.table_to_device(table, self._device) if len(table) else None
            tables.append((bucket, dev, len(table), partial_base))
            partial_base += len(table)
        self._n_partials = partial_base
        # the same pass as one host array for eth_bucket_sync_local
        local = np.zeros(len(tables), dtype=nat.BUCKET_DTYPE)
        for i, (bucket, dev, n_chunks, base) in enumerate(tables):
            payload = self._scratch[bucket.grad_dtype]
            local[i] = (dev.data_ptr() if dev is not None else 0, n_chunks, payload.data_ptr(), base,
                        nat.dtype_code(payload.dtype), 0)
        self._local_pass = local
        # staging for the single-rank pass: two halves, each the largest
        # payload of the pass, so one launch unpacks a bucket while it packs
        # the next (the identity seam only; a real collective reads the
        # scratch buffer itself)
        self._staging, self._staging_half = None, 0
        if self._all_reduce_sum is local_all_reduce_sum and tables and self._device is not None:
            half = max(b.exact_numel * self._scratch[b.grad_dtype].element_size() for b, *_ in tables)
            half = (half + 255) // 256 * 256
            self._staging = torch.empty(2 * half, dtype=torch.uint8, device=self._device)
            self._staging_half = half
        return tables

    # ----------------------------------------------------------- statistics --
    @property
    def n_partials(self):
        return self._n_partials

    def covered_gradients(self):
        """main_grad tensors this executor writes, by logical id."""
        return {lid: r.main_grad for lid, r in self._runtime_bindings.items()}

    def exclude_from_norm(self, logical_param_ids):
        """Leave these gradients out of the fused L2 partials (their partial
        slots read 0): gradients that change after the sync, such as a tied
        pair summed afterwards, get their statistics taken later."""
        excluded = frozenset(logical_param_ids)
        unknown = excluded - set(self._runtime_bindings)
        if unknown:
            raise ValueError(f"rank {self.global_rank} has no gradients for {sorted(unknown)}")
        if excluded != self._norm_excluded:
            self._norm_excluded = excluded
            self._tables = self._build_tables()

    def bind_statistics(self, statistics):
        """Let execute() also unscale, flag inf/nan and collect L2 partials."""
        if statistics is not None and statistics.n_partials < self._n_partials:
            raise ValueError("statistics buffer is smaller than the executor's chunk count")
        self._statistics = statistics

    def set_inv_loss_scale(self, inv_scale):
        self._inv_scale = float(inv_scale)

    # ------------------------------------------------------------ execute --
    def bucket_parameters(self):
        """Per bucket, in execution order, the parameters whose main_grad it
        reads (each once)."""
        out = []
        for bucket, _table, _n, _base in self._tables:
            seen = {}
            for placement in bucket.placements:
                binding = self._binding_specs[placement.fragment_id]
                param = self._runtime_bindings[binding.logical_param_id].parameter
                seen.setdefault(id(param), param)
            out.append(list(seen.values()))
        return out

    @property
    def n_buckets(self):
        return len(self._tables)

    def begin(self, normalization_scale=1.0):
        """Start a pass over the buckets on the current stream: resets the
        bound statistics; run_bucket(i) then syncs bucket i, in any order,
        each once, on the current stream, and end() closes the pass."""
        stats = self._statistics
        flags = 0
        if stats is not None:
            stats.reset()
            flags |= nat.UNPACK_STATS
            if self._inv_scale != 1.0:
                flags |= nat.UNPACK_UNSCALE
        if normalization_scale != 1.0:
            flags |= nat.UNPACK_WRITEBACK
        self._pass = (float(normalization_scale), flags)
        self._next_bucket = 0
        if self._evidence is not None:
            self._evidence.begin_execution(normalization_scale)

    def run_bucket(self, i):
        """pack -> all_reduce_sum seam -> fused unpack of bucket i
        (executor.py:199-261) on the current stream."""
        normalization_scale, flags = self._pass
        stats = self._statistics
        stream = nat.stream_ptr(self._device) if self._device is not None else None
        bucket, table, n_chunks, base = self._tables[i]
        payload = self._scratch[bucket.grad_dtype][: bucket.exact_numel]
        dcode = nat.dtype_code(payload.dtype)
        if self._evidence is not None:
            # the evidence hashes the plan's buckets in plan order, each once
            if i != self._next_bucket:
                raise ValueError("runtime evidence records buckets in plan order; the streamed sync reorders them")
            self._next_bucket += 1
        if n_chunks:
            nat.call("eth_bucket_pack", nat.ptr(table), n_chunks, nat.ptr(payload), dcode, stream)
        if self._evidence is not None:
            self._evidence.observe_packed_bucket(bucket, payload)
        self._all_reduce_sum(payload, self._registry.handle(bucket.process_group_id))
        if n_chunks:
            f = flags if (dcode == nat.ETH_F32 or not (flags & nat.UNPACK_UNSCALE)) else flags & ~nat.UNPACK_UNSCALE
            nat.call(
                "eth_bucket_unpack",
                nat.ptr(table),
                n_chunks,
                nat.ptr(payload),
                dcode,
                normalization_scale,
                float(self._inv_scale),
                f,
                nat.ptr(stats.found_inf) if stats is not None else None,
                nat.ptr(stats.partials) if stats is not None else None,
                base,
                stream,
            )

    def end(self):
        stats = self._statistics
        if stats is not None:
            stats.fresh = True
            stats.inv_scale_used = self._inv_scale
        self._pass = None
        if self._evidence is not None:
            self._evidence.finish_execution()

    def execute(self, normalization_scale=1.0):
        self.begin(normalization_scale)
        if self._all_reduce_sum is local_all_reduce_sum and self._evidence is None and len(self._tables):
            # the identity seam: one native call issues every bucket's pack
            # and unpack (the launches run_bucket would make, in its order)
            normalization_scale, flags = self._pass
            stats = self._statistics
            nat.call(
                "eth_bucket_sync_local",
                ctypes.c_void_p(self._local_pass.ctypes.data),
                len(self._local_pass),
                normalization_scale,
                float(self._inv_scale),
                flags,
                nat.ptr(stats.found_inf) if stats is not None else None,
                nat.ptr(stats.partials) if stats is not None else None,
                nat.ptr(self._staging) if self._staging is not None else None,
                self._staging_half,
                nat.stream_ptr(self._device),
            )
        else:
            for i in range(len(self._tables)):
                self.run_bucket(i)
        self.end()
