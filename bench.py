"""Benchmark: one ETH pipeline stage's training step on one MI355X.

Workload: a 6-layer middle stage of GPT-1.3B in
bf16 -- hidden 2048, 16 heads (hn 128), FFN 8192, seq 2048, micro-batch 4,
TP = 1 -- with x ~ N(0,1) [2048, 4, 2048], weights N(0, 0.02), upstream
gradient N(0, 1e-3), dropout 0.  A step is: zero main grads, forward,
backward (input + weight gradients into fp32 main grads), Block-wise grad
sync (32 MiB buckets; pack / unpack with the fused unscale-flag-L2
statistics), clip at 1.0, fused AdamW (lr 1e-4, betas .9/.95, eps 1e-8,
wd 0.1) with the bf16 model copy.  Inputs are resident in HBM before the
timed region.

Prints one JSON line.  `value` is tokens/s of the K timed steps (wall clock
between two device synchronizations); `step_ms_median` / `step_ms_p90` come
from HIP events around each step on the compute stream.  `roofline` covers
the dominant kernel, the MFMA GEMM: its algorithmic FLOPs per launch over
its average launch duration, both from HIP events recorded on the launch
stream around every GEMM of separate instrumented steps (the timed steps run
without the events).  `attention` gives the same for the attention forward
and backward.  `hbm_path` reports grad pack+unscale(2^-16)+inf flag+L2+
unpack (also with 0.1 % of the gradients +inf) and AdamW at BASELINE
configs[2]/[3] scale (1,208,598,528 fp32 elements).  `first_last_stage`
times the GPT-6.7B first+last stage in fp16.
`cpu_baseline` times this build's torch-CPU restatement of the same step on
the host cores (the oracle; the reference's Python does not travel).
"""

import argparse
import gc
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.0  # MI355X dense bf16 MFMA (2.5 PFLOP/s)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
H, HEADS, FFN, SEQ, MB, LAYERS = 2048, 16, 8192, 2048, 4, 6
# the committed FETCH_SIZE / WRITE_SIZE counter summary of the GEMM launches
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_traffic_stage_step_gpt1p3b.md")


def quiet_gc():
    """Collect, then move every object alive now (torch, the model, the
    trainer: ~270K objects) into the collector's permanent generation.  A
    full collection otherwise traverses all of them, a 40-80 ms host stall
    that leaves the GPU idle whenever one falls inside the timed steps; after
    the freeze a collection walks only the objects the steps create.  No GPU
    work changes."""
    gc.collect()
    gc.freeze()


def step_flops(layers=LAYERS, s=SEQ, b=MB, h=H, f=FFN):
    """3 x (dense GEMMs + causal attention) per layer (fwd + 2x bwd)."""
    T = s * b
    per_layer = 2 * T * (3 * h * h + h * h + 2 * h * f) + 2 * b * s * s * h
    return 3 * per_layer * layers


def percentile(values, q):
    v = sorted(values)
    if not v:
        return None
    k = (len(v) - 1) * q
    lo, hi = math.floor(k), math.ceil(k)
    return v[lo] + (v[hi] - v[lo]) * (k - lo)


class KernelMeter:
    """HIP events around every GEMM / attention launch, recorded on the
    stream the launch goes to, with the launch's algorithmic FLOPs.
    Weight-gradient GEMMs run on a side stream, overlapped with the
    data-gradient chain, so launches can overlap in time."""

    def __init__(self, torch):
        self.torch = torch
        self.launches = {}  # kind -> [[begin, end, flops]]
        self.base = torch.cuda.Event(enable_timing=True)
        self.base.record()

    def __call__(self, kind, phase, flops):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        if phase == "begin":
            self.launches.setdefault(kind, []).append([e, None, flops])
        else:
            self.launches[kind][-1][1] = e

    def summary(self, kind, steps):
        rec = self.launches.get(kind, [])
        if not rec:
            return None
        durs = [a.elapsed_time(b) for a, b, _ in rec]
        flops = sum(f for _, _, f in rec)
        spans = sorted((self.base.elapsed_time(a), self.base.elapsed_time(b)) for a, b, _ in rec)
        union, c0, c1 = 0.0, None, None
        for t0, t1 in spans:
            if c1 is None or t0 > c1:
                if c1 is not None:
                    union += c1 - c0
                c0, c1 = t0, t1
            else:
                c1 = max(c1, t1)
        union += (c1 - c0) if c1 is not None else 0.0
        n = len(rec)
        return {
            "launches_per_step": n / steps,
            "flops_per_launch": flops / n,
            "avg_launch_us": 1e3 * sum(durs) / n,
            "achieved_tflops": flops / (sum(durs) * 1e-3) / 1e12,
            "launch_sum_ms_per_step": sum(durs) / steps,
            "busy_union_ms_per_step": union / steps,
            "achieved_over_busy_union_tflops": flops / (union * 1e-3) / 1e12,
        }


def traffic_from_profile():
    """(HBM bytes per GEMM launch, algorithmic bytes per launch, source) from
    the committed counter summary, or (None, None, reason)."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None, None, "no counter summary in profiles/"
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    a = re.search(r"algorithmic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    if not m:
        return None, None, "counter summary lacks traffic_bytes_per_launch"
    return float(m.group(1)), float(a.group(1)) if a else None, os.path.relpath(TRAFFIC_PROFILE, ROOT)


def cpu_info():
    model, logical, cores_per_socket, sockets = "unknown", os.cpu_count(), None, None
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            val = val.strip()
            if key == "Model name":
                model = val
            elif key == "Core(s) per socket":
                cores_per_socket = int(val)
            elif key == "Socket(s)":
                sockets = int(val)
    except Exception:  # lscpu missing: report what Python knows
        pass
    physical = cores_per_socket * sockets if cores_per_socket and sockets else None
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = logical
    return {"model": model, "logical_cpus": logical, "physical_cores": physical, "affinity_cpus": affinity}


def cpu_threads(info):
    """Every CPU this process may run on (its affinity set), bounded by
    OMP_NUM_THREADS when the environment sets it: a GPU box exports its CPU
    share per GPU there, and the host may hold more cores than that share."""
    threads = info["affinity_cpus"] or info["logical_cpus"] or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    return max(1, threads)


def cpu_baseline(torch):
    """This build's torch-CPU fp32 restatement (the oracle) of the reference
    sequence on the host: the whole 6-layer stage forward+backward at the
    full shape once, then the grad sync (per-segment copy_ pack/unpack,
    torch._amp_foreach_non_finite_check_and_unscale_, per-tensor
    pow(2).sum()) and torch.optim.AdamW over the stage's 302 M parameters;
    plus the grad-sync and AdamW legs alone on a 2-layer slice of the
    C3/C4 tensor list, reported in GB/s of the same algorithmic bytes as
    the GPU legs."""
    from oracle import layer as ol

    info = cpu_info()
    threads = cpu_threads(info)
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)

    def layer_params():
        return {
            "ln1_w": torch.ones(H), "ln1_b": torch.zeros(H),
            "qkv_w": torch.randn(3 * H, H, generator=gen) * 0.02, "qkv_b": torch.zeros(3 * H),
            "proj_w": torch.randn(H, H, generator=gen) * 0.02, "proj_b": torch.zeros(H),
            "ln2_w": torch.ones(H), "ln2_b": torch.zeros(H),
            "fc1_w": torch.randn(FFN, H, generator=gen) * 0.02, "fc1_b": torch.zeros(FFN),
            "fc2_w": torch.randn(H, FFN, generator=gen) * 0.02, "fc2_b": torch.zeros(H),
        }

    layers = [layer_params() for _ in range(LAYERS)]
    x = torch.randn(SEQ, MB, H, generator=gen)
    dy = torch.randn(SEQ, MB, H, generator=gen) * 1e-3
    params = [torch.nn.Parameter(v.clone()) for lp in layers for v in lp.values()]
    opt = torch.optim.AdamW(params, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)

    def grad_sync(grads, scratch):
        """executor.py:199-261 + optimizer.py:436-461 + the canonical norm."""
        off = 0
        for g in grads:  # pack: one copy_ per segment
            n = g.numel()
            scratch[off : off + n].copy_(g.reshape(-1))
            off += n
        off = 0
        for g in grads:  # unpack
            n = g.numel()
            g.reshape(-1).copy_(scratch[off : off + n])
            off += n
        found = torch.zeros(1)
        torch._amp_foreach_non_finite_check_and_unscale_(grads, found, torch.full((1,), 2.0**-16))
        return math.sqrt(sum(float(g.pow(2).sum()) for g in grads))

    t0 = time.perf_counter()
    _, _, grads = ol.middle_stage_fwd_bwd(x, layers, HEADS, dy)
    t_fwd_bwd = time.perf_counter() - t0
    flat_grads = [g for gl in grads for g in gl.values()]
    scratch = torch.empty(sum(g.numel() for g in flat_grads))
    t1 = time.perf_counter()
    grad_sync(flat_grads, scratch)
    for p, g in zip(params, flat_grads):
        p.grad = g
    opt.step()
    t_tail = time.perf_counter() - t1
    step_s = t_fwd_bwd + t_tail
    del grads, flat_grads, scratch, opt, params

    # C3 / C4 legs alone on the first 2 of the 24 layers of the tensor list
    from eth_amd.grad_sync.synthetic import gpt_layer_shapes

    shapes = gpt_layer_shapes(H, FFN, 2)
    n_elem = sum(math.prod(s[1]) for s in shapes)
    gs = [torch.randn(s[1], generator=gen) * 1e-3 for s in shapes]
    scratch = torch.empty(n_elem)
    t2 = time.perf_counter()
    grad_sync(gs, scratch)
    t_sync = time.perf_counter() - t2
    adam = {}
    for label, kw in (("foreach_false", {"foreach": False}), ("default", {})):
        ps = [torch.nn.Parameter(torch.randn(s[1], generator=gen) * 0.02) for s in shapes]
        o = torch.optim.AdamW(ps, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, **kw)
        for p, g in zip(ps, gs):
            p.grad = g
        o.step()  # state allocation outside the timing
        t3 = time.perf_counter()
        o.step()
        adam[label] = time.perf_counter() - t3
        del o, ps
    return {
        "value": (SEQ * MB) / step_s,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"one full step of the 6-layer stage in fp32 torch-CPU (oracle restatement): fwd+bwd at s {SEQ} b {MB} "
            f"{t_fwd_bwd:.2f} s, grad sync + unscale + L2 + AdamW over 302M params {t_tail:.2f} s; "
            f"{threads} threads (the CPUs this process may use, bounded by OMP_NUM_THREADS) on {info['model']}"
        ),
        "cpu": info,
        "grad_sync_gbps": 16.0 * n_elem / t_sync / 1e9,
        "adamw_gbps": {k: 30.0 * n_elem / v / 1e9 for k, v in adam.items()},
        "hbm_leg_sample": f"2 of the 24 layers of the C3/C4 tensor list ({n_elem} fp32 elements); GB/s of 16 B "
                          "(grad sync) and 30 B (AdamW) per element",
    }


def hbm_path(torch, iters=10):
    """Grad pack+unscale+flag+L2+unpack and AdamW over the 24-layer
    GPT-1.3B grad list ([3]), HIP-event timed."""
    from eth_amd.grad_sync import bucket_plan as bp
    from eth_amd.grad_sync.bucket_plan import ProcessGroupRegistry
    from eth_amd.grad_sync.executor import GradientBucketExecutor, GradientStatistics, local_all_reduce_sum
    from eth_amd.grad_sync.metadata import LocalGradientBinding
    from eth_amd.grad_sync.planner import plan_canonical_fragments
    from eth_amd.grad_sync.synthetic import descriptors_for, gpt_layer_shapes
    from eth_amd.optimizer.fused_adam import FusedAdamW

    dev = torch.device("cuda:0")
    shapes = gpt_layer_shapes(H, FFN, 24)
    descs = descriptors_for(shapes)
    plan = bp.build_gradient_sync_plan(plan_canonical_fragments(descs, (0,)), "block", 32 << 20, "gpt", "m", "t")
    total = sum(math.prod(s[1]) for s in shapes)
    buf = torch.empty(total, dtype=torch.float32, device=dev)
    g = torch.Generator(device=dev).manual_seed(1234)
    buf.normal_(0, 1e-3, generator=g)
    grads, off = {}, total
    for lid, shape, *_ in shapes:
        n = math.prod(shape)
        off -= n
        grads[lid] = buf[off : off + n].view(shape)
    registry = ProcessGroupRegistry(plan.process_groups, lambda ranks: ranks)
    registry.initialize()
    bindings = [LocalGradientBinding(l, None, grads[l], grads[l].device) for l, *_ in shapes]
    ex = GradientBucketExecutor(plan, 0, descs, bindings, registry, local_all_reduce_sum)
    st = GradientStatistics(ex.n_partials, dev)
    ex.bind_statistics(st)
    ex.set_inv_loss_scale(2.0**-16)

    def timed(fn, prepare=None):
        """Mean of `iters` event-timed calls; `prepare` runs before each
        call, outside the events."""
        fn()
        total_ms = 0.0
        for _ in range(iters):
            if prepare is not None:
                prepare()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            total_ms += a.elapsed_time(b)
        return total_ms / iters

    def timed_back_to_back(fn):
        """Mean of `iters` calls issued back to back between two events, the
        first event queued behind a warm-up call: the host's work of each
        call then overlaps the previous call's kernels, as it does in
        training, instead of sitting in front of an idle GPU."""
        fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / iters

    sync = lambda: (ex.execute(1.0), st.finalize(1.0))  # noqa: E731
    # the unpack writes the unscaled gradients back; scaling them up again
    # by 2^16 (exact) outside the timing keeps every call on the same data
    rescale = lambda: buf.mul_(2.0**16)  # noqa: E731
    t_sync = timed(sync, rescale)
    found_clean = float(st.found_inf.item())
    # 0.1 % of the elements +inf (a seeded index set), the C3 overflow variant
    idx = torch.randint(0, total, (total // 1000,), generator=g, device=dev)
    buf[idx] = float("inf")
    del idx
    t_sync_inf = timed(sync, rescale)
    found_inf = float(st.found_inf.item())
    buf.normal_(0, 1e-3, generator=g)
    params = [torch.nn.Parameter(torch.empty(s[1], device=dev).normal_(0, 0.02, generator=g)) for s in shapes]
    model = [torch.empty(s[1], device=dev, dtype=torch.bfloat16) for s in shapes]
    for p, (lid, *_) in zip(params, shapes):
        p.grad = grads[lid]
    opt = FusedAdamW([{"params": params}], lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    opt.set_model_copies(dict(zip(params, model)), torch.bfloat16)
    ex.set_inv_loss_scale(1.0)
    sync()
    t_adam = timed_back_to_back(lambda: opt.step(stats=st.stats))
    out = {
        "elements": total,
        "inv_loss_scale": 2.0**-16,
        "grad_sync_ms": t_sync,
        "grad_sync_gbps": 16.0 * total / t_sync / 1e6,
        "grad_sync_found_inf": found_clean,
        "grad_sync_inf_variant_ms": t_sync_inf,
        "grad_sync_inf_variant_gbps": 16.0 * total / t_sync_inf / 1e6,
        "grad_sync_inf_variant_found_inf": found_inf,
        "adam_ms": t_adam,
        "adam_gbps": 30.0 * total / t_adam / 1e6,
        "peak_gbps": PEAK_HBM_GBPS,
        "bytes_per_element": {"grad_sync": 16, "adam": 30},
    }
    out["grad_sync_frac"] = out["grad_sync_gbps"] / PEAK_HBM_GBPS
    out["adam_frac"] = out["adam_gbps"] / PEAK_HBM_GBPS
    del ex, st, opt, params, model, buf, grads
    torch.cuda.empty_cache()
    # the practical ceiling of mixed read/write traffic on this box: a 1 GiB
    # device-to-device copy (1 GiB read + 1 GiB written), same timing method
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    t_copy = timed_back_to_back(lambda: dst.copy_(src))
    out["copy_ms"] = t_copy
    out["copy_gbps"] = 2.0 * src.numel() * 4 / t_copy / 1e6
    out["copy_frac"] = out["copy_gbps"] / PEAK_HBM_GBPS
    out["adam_over_copy"] = out["adam_gbps"] / out["copy_gbps"]
    out["grad_sync_over_copy"] = out["grad_sync_gbps"] / out["copy_gbps"]
    del src, dst
    torch.cuda.empty_cache()
    return out


def gemm_layer_products(torch, reps=10):
    """The twelve GEMMs of one C2 layer alone, as LinearFn issues them
    (forward X W^T with bias, data gradient dY W, weight gradient dY^T X
    stored into an fp32 main_grad), each HIP-event timed over `reps` calls,
    beside torch.matmul (hipBLASLt) on the same bf16 operands."""
    from eth_amd import kernels as K

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    T = SEQ * MB

    def rnd(*shape):
        return torch.randn(*shape, device=dev, generator=g).to(torch.bfloat16)

    def timed(fn):
        fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    rows, tot, tot_lib = [], 0.0, 0.0
    for name, n_in, n_out in (("qkv", H, 3 * H), ("proj", H, H), ("fc1", H, FFN), ("fc2", FFN, H)):
        x, w, dy, bias = rnd(T, n_in), rnd(n_out, n_in), rnd(T, n_out), rnd(n_out)
        mg = torch.empty(n_out, n_in, dtype=torch.float32, device=dev)
        for kind, fn, lib, (m, n, k) in (
            ("fwd", lambda: K.gemm(x, w.t(), bias=bias), lambda: torch.matmul(x, w.t()), (T, n_out, n_in)),
            ("dgrad", lambda: K.gemm(dy, w), lambda: torch.matmul(dy, w), (T, n_in, n_out)),
            ("wgrad", lambda: K.gemm(dy.t(), x, out=mg), lambda: torch.matmul(dy.t(), x), (n_out, n_in, T)),
        ):
            us, us_lib = timed(fn), timed(lib)
            flops = 2.0 * m * n * k
            rows.append({"product": f"{name} {kind}", "M": m, "N": n, "K": k, "us": us,
                         "tflops": flops / us / 1e6, "hipblaslt_us": us_lib, "hipblaslt_tflops": flops / us_lib / 1e6})
            tot += us
            tot_lib += us_lib
        del x, w, dy, bias, mg
    return {"products": rows, "layer_us": tot, "hipblaslt_layer_us": tot_lib,
            "layer_tflops": 3 * 2.0 * T * (H * 3 * H + H * H + 2 * H * FFN) / tot / 1e6}


def first_last_stage(torch, steps=5, warmup=2, overlap_optimizer=True):
    """the GPT-6.7B first+last stage in fp16 -- token +
    position embedding, 2 layers (hidden 4096, 32 heads, FFN 16384), final
    LN, tied LM head over the padded vocabulary (50304) and vocab cross
    entropy on the reference's synthetic batch, seq 2048, micro-batch 2;
    dynamic loss scale (2^16), grad sync, tied-gradient sum, unscale + clip
    1.0, AdamW with the fp16 model copy.

    Labels are drawn uniformly over the vocabulary from a seed, fresh for
    every step (made before the timing).  The reference's labels = 0
    (flex_ops.py:1962) would stop training after the first update: every
    gradient pushes the same logit, and AdamW's first step saturates the
    fp16 softmax, so later steps would run on a zero loss and zero
    gradients.  Each timed step's mean loss and gradient norm are reported,
    read after the timed region."""
    from eth_amd.model.flex_ops import GPTConfig
    from eth_amd.stage import FirstLastStageTrainer

    h, heads, f, layers, s, b, V = 4096, 32, 16384, 2, 2048, 2, 50304
    cfg = GPTConfig(hidden_size=h, num_attention_heads=heads, ffn_hidden_size=f, num_layers=layers, seq_length=s,
                    micro_batch_size=b, padded_vocab_size=V, params_dtype=torch.float16, device="cuda", seed=1234)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0,
                               bucket_cap_bytes=32 << 20, initial_loss_scale=2.0**16,
                               overlap_optimizer=overlap_optimizer)
    gen = torch.Generator(device="cuda").manual_seed(4321)
    labels = [torch.randint(0, 50257, (b, s), generator=gen, device="cuda") for _ in range(warmup + steps)]
    for i in range(warmup):
        if i == warmup - 1:  # the freeze before the last warm-up step (see main)
            torch.cuda.synchronize()
            quiet_gc()
        tr.train_step([2 * i, 2 * i + 1], labels[i])
    if warmup == 0:
        quiet_gc()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    oks, means, norms = 0, [], []
    for i in range(steps):
        _, lo, ok, norm = tr.train_step([2 * (warmup + i), 2 * (warmup + i) + 1], labels[warmup + i])
        oks += bool(ok)
        means.append(lo.local_loss_sum / lo.local_loss_weight)  # device scalars, read after the timing
        norms.append(norm)
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / steps
    step_losses = [float(m.item()) for m in means]
    T = s * b
    flops = step_flops(layers, s, b, h, f) + 3 * 2.0 * T * h * V  # + LM head fwd, dgrad, wgrad
    tflops = flops / (ms * 1e-3) / 1e12
    del tr
    torch.cuda.empty_cache()
    return {
        "workload": "GPT-6.7B first+last stage: embedding + 2 layers (h 4096, 32 heads, FFN 16384) + final LN + "
                    "tied LM head (V 50304) + vocab CE, seq 2048, micro-batch 2, fp16, dynamic loss scale 2^16",
        "tokens_per_s": T / (ms * 1e-3),
        "ms_per_step": ms,
        "steps": steps,
        "steps_applied": oks,
        "labels": "uniform over [0, 50257) from seed 4321, fresh per step",
        "step_mean_loss": step_losses,
        "step_grad_norm": norms,
        "step_tflops": tflops,
        "step_mfma_frac": tflops / PEAK_BF16_TFLOPS,
        "dtype": "f16",
    }


def pipeline_stage_step(torch, steps=5, warmup=2, microbatches=4, overlap_optimizer=True):
    """The C2 stage's 6 layers as two 3-layer stages in the 1F1B order
    (eth_amd.schedules.PipelineTrainer) beside the same 6 layers as one
    stage running the microbatches one at a time (train_step_microbatches):
    the step's 8192 tokens as `microbatches` microbatches of one sequence,
    one clip norm over both stages.  On one GPU the two stages run one
    after the other, so the figures differ by the driver's host work only."""
    from eth_amd.model.flex_ops import GPTConfig
    from eth_amd.schedules import PipelineTrainer
    from eth_amd.stage import MiddleStageTrainer

    mb = MB * SEQ // (SEQ * microbatches)
    kw = dict(lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0,
              overlap_optimizer=overlap_optimizer)

    def cfg(layers):
        return GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=layers,
                         seq_length=SEQ, micro_batch_size=mb, params_dtype=torch.bfloat16, device="cuda", seed=1234)

    g = torch.Generator(device="cuda").manual_seed(99)
    mbs = [{"input_tensors": {"hidden_states": torch.randn(SEQ, mb, H, device="cuda", generator=g).to(torch.bfloat16)},
            "output_grads": {"hidden_states": (torch.randn(SEQ, mb, H, device="cuda", generator=g) * 1e-3)
                             .to(torch.bfloat16)}} for _ in range(microbatches)]

    def timed(step):
        for i in range(warmup):
            if i == warmup - 1:
                torch.cuda.synchronize()
                quiet_gc()
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return 1e3 * (time.perf_counter() - t0) / steps

    one = MiddleStageTrainer(cfg(LAYERS), **kw)
    ms_one = timed(lambda: one.train_step_microbatches(mbs))
    del one
    torch.cuda.empty_cache()
    half = LAYERS // 2
    stages = [MiddleStageTrainer(cfg(LAYERS), first_layer=0, num_layers=half, **kw),
              MiddleStageTrainer(cfg(LAYERS), first_layer=half, num_layers=LAYERS - half, **kw)]
    pipe = PipelineTrainer(stages)
    ms_pipe = timed(lambda: pipe.train_step(mbs))
    ticks = pipe.last_timeline["ticks"]
    del pipe, stages
    torch.cuda.empty_cache()
    T = MB * SEQ
    return {
        "workload": f"C2 widths, {LAYERS} layers, {microbatches} microbatches of micro-batch {mb} x seq {SEQ} "
                    f"({T} tokens per step), bf16",
        "one_stage_ms_per_step": ms_one,
        "one_stage_tokens_per_s": T / (ms_one * 1e-3),
        "two_stage_1f1b_ms_per_step": ms_pipe,
        "two_stage_1f1b_tokens_per_s": T / (ms_pipe * 1e-3),
        "pipeline_ticks": ticks,
        "steps": steps,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--meter-steps", type=int, default=3,
                    help="extra steps with HIP events around every GEMM / attention launch (roofline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-hbm-path", action="store_true")
    ap.add_argument("--no-first-last", action="store_true")
    ap.add_argument("--inline-update", action="store_true",
                    help="run the AdamW update in line instead of overlapped with the next step's forward")
    ap.add_argument("--first-last-only", action="store_true",
                    help="time only the configs[4] first+last stage (for its kernel profile)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="time only the twelve GEMMs of one layer alone, beside hipBLASLt (for their counter runs)")
    ap.add_argument("--hbm-only", action="store_true",
                    help="time only the grad-sync and AdamW legs and their copy ceiling (for their "
                         "FETCH_SIZE / WRITE_SIZE counter runs)")
    ap.add_argument("--pipeline-only", action="store_true",
                    help="time only the C2 layers as two 1F1B pipeline stages beside one stage")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed steps, copy 1 GiB once (the calibration kernel of the "
                         "FETCH_SIZE / WRITE_SIZE counter runs behind roofline.traffic)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every GPU box of this build has a single MI355X, so no "
              "collective is exercised and the stage's data-, tensor- and pipeline-parallel "
              "sharding is design only", file=sys.stderr)
        sys.exit(2)

    import torch

    from eth_amd import kernels as K
    from eth_amd.model.flex_ops import GPTConfig
    from eth_amd.stage import MiddleStageTrainer

    if args.first_last_only:
        fl = first_last_stage(torch, steps=args.steps, warmup=args.warmup, overlap_optimizer=not args.inline_update)
        print(json.dumps({"first_last_stage": fl}), flush=True)
        return
    if args.hbm_only:
        print(json.dumps({"hbm_path": hbm_path(torch)}), flush=True)
        return
    if args.gemm_only:
        print(json.dumps({"gemm_layer_products": gemm_layer_products(torch)}), flush=True)
        return
    if args.pipeline_only:
        print(json.dumps({"pipeline": pipeline_stage_step(torch, steps=args.steps, warmup=args.warmup,
                                                          overlap_optimizer=not args.inline_update)}), flush=True)
        return

    cfg = GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=LAYERS,
                    seq_length=SEQ, micro_batch_size=MB, params_dtype=torch.bfloat16, device="cuda", seed=1234)
    tr = MiddleStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0,
                            overlap_optimizer=not args.inline_update)
    g = torch.Generator(device="cuda").manual_seed(1234)
    x = torch.randn(SEQ, MB, H, device="cuda", generator=g).to(torch.bfloat16)
    dy = (torch.randn(SEQ, MB, H, device="cuda", generator=g) * 1e-3).to(torch.bfloat16)
    # the collector freeze idles the GPU for a fraction of a second, and the
    # shader clock ramps back up over the next step: it goes before the last
    # warm-up step, so the timed steps start on a busy-clocked GPU
    for i in range(args.warmup):
        if i == args.warmup - 1:
            torch.cuda.synchronize()
            quiet_gc()
        tr.train_step(x, dy)
    if args.warmup == 0:
        quiet_gc()
    torch.cuda.synchronize()

    # timed steps: no instrumentation besides one event pair per step
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        out, dx, ok, norm = tr.train_step(x, dy)
        marks[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = [marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
    ms = 1e3 * elapsed / args.steps
    tokens = SEQ * MB
    value = tokens * args.steps / elapsed
    step_tflops = step_flops() / (ms * 1e-3) / 1e12

    # instrumented steps for the kernel rooflines
    meter = KernelMeter(torch)
    K.set_kernel_observer(meter)
    for _ in range(args.meter_steps):
        tr.train_step(x, dy)
    torch.cuda.synchronize()
    K.set_kernel_observer(None)
    gemm = meter.summary("gemm", args.meter_steps)
    attn_f = meter.summary("attn_fwd", args.meter_steps)
    attn_b = meter.summary("attn_bwd", args.meter_steps)
    traffic, algo_bytes, traffic_src = traffic_from_profile()

    result = {
        "metric": "stage train tokens/s (GPT-1.3B, 6 layers) on 1 GPU; grad-pack+Adam HBM GB/s",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "step_ms_median": percentile(step_ms, 0.5),
        "step_ms_p90": percentile(step_ms, 0.9),
        "step_ms": [round(v, 3) for v in step_ms],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x~N(0,1), weights N(0,0.02), dy~N(0,1e-3), seeded)",
        "config": {
            "workload": "GPT-1.3B middle pipeline stage: 6 of 24 layers, hidden 2048, 16 heads, FFN 8192, "
                        "seq 2048, micro-batch 4, TP=1, bf16; fwd+bwd+grad sync (32 MiB buckets)+clip+AdamW",
            "global_batch": MB,
            "seq_len": SEQ,
            "parallelism": "single GPU (TP=1, DP=1, one pipeline stage)",
        },
        "step_tflops": step_tflops,
        "step_mfma_frac": step_tflops / PEAK_BF16_TFLOPS,
        "grad_norm": norm,
        "roofline": {
            "kernel": "eth_gemm (gemm256_m16/m32 and gemm_kernel instantiations: every GEMM launch of a step)",
            "bound": "mfma",
            "achieved": gemm["achieved_tflops"],
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm["achieved_tflops"] / PEAK_BF16_TFLOPS,
            "traffic": traffic,
            "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": algo_bytes,
            "basis": "algorithmic FLOPs per launch / average launch duration (HIP events on the launch stream, "
                     f"{args.meter_steps} instrumented steps)",
            **{k: gemm[k] for k in ("launches_per_step", "flops_per_launch", "avg_launch_us",
                                    "launch_sum_ms_per_step", "busy_union_ms_per_step",
                                    "achieved_over_busy_union_tflops")},
        },
        "attention": {
            "bound": "mfma",
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "flops_basis": "fwd 2*b*s^2*h (causal half of QK^T and PV); bwd 2.5x fwd (recomputed S, dP, dV, dQ, dK)",
            "fwd": {**attn_f, "frac": attn_f["achieved_tflops"] / PEAK_BF16_TFLOPS} if attn_f else None,
            "bwd": {**attn_b, "frac": attn_b["achieved_tflops"] / PEAK_BF16_TFLOPS} if attn_b else None,
        },
    }
    del tr, out, dx
    torch.cuda.empty_cache()
    if args.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_hbm_path:
        result["hbm_path"] = hbm_path(torch)
    if not args.no_first_last:
        result["first_last_stage"] = first_last_stage(torch, overlap_optimizer=not args.inline_update)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
