"""Benchmark: one ETH pipeline stage's training step on one MI355X.

Workload: a 6-layer middle stage of GPT-1.3B in
bf16 -- hidden 2048, 16 heads (hn 128), FFN 8192, seq 2048, micro-batch 4,
TP = 1 -- with x ~ N(0,1) [2048, 4, 2048], weights N(0, 0.02), upstream
gradient N(0, 1e-3), dropout 0.  A step is: zero main grads, forward,
backward (input + weight gradients into fp32 main grads), Block-wise grad
sync (32 MiB buckets; pack / unpack with the fused unscale-flag-L2
statistics), clip at 1.0, fused AdamW (lr 1e-4, betas .9/.95, eps 1e-8,
wd 0.1) with the bf16 model copy.

Prints one JSON line.  `value` is tokens/s of the whole step; `roofline`
covers the dominant kernel (the MFMA GEMM): algorithmic FLOPs of its
launches / their summed duration, from HIP events recorded on the launch
stream around every GEMM of the timed steps.  `hbm_path` reports the
grad-pack+unscale+L2 pass and AdamW at BASELINE configs[2]/[3] scale
(1,208,598,528 fp32 elements).  `first_last_stage` times the GPT-6.7B
first+last stage in fp16.  `cpu_baseline` times the oracle's torch-CPU
fp32 restatement of one layer (forward + backward + grad sync + AdamW) on
the host cores, on a bounded sample, scaled to the 6-layer stage.
"""

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.0  # MI355X dense bf16 MFMA (2.5 PFLOP/s)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
H, HEADS, FFN, SEQ, MB, LAYERS = 2048, 16, 8192, 2048, 4, 6
# HBM (L2-miss) bytes per GEMM launch of one stage step, from the FETCH_SIZE /
# WRITE_SIZE counter runs (each scaled by what it reads for a 1 GiB copy:
# 2.0 and 1.0) recorded in profiles/gemm_traffic_stage_step_gpt1p3b.md; the
# algorithmic bytes (A + B + C, a weight gradient storing its fp32 main_grad:
# the step's only contribution after the deferred zeroing) of the same
# launches for comparison
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 409.0e6
GEMM_ALGORITHMIC_BYTES_PER_LAUNCH = 167.8e6


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


class GemmMeter:
    """Records HIP events around every GEMM launch, on the stream the launch
    goes to, and sums FLOPs.  The weight-gradient GEMMs of the timed steps
    run on a side stream, overlapped with the data-gradient chain, so
    launches can overlap in time: `busy_ms` is the length of the union of
    the launch intervals (time during which at least one GEMM ran), and
    `total_ms` the plain sum of launch durations."""

    def __init__(self, torch):
        self.torch = torch
        self.events = []
        self.flops = 0.0
        self.base = torch.cuda.Event(enable_timing=True)
        self.base.record()

    def __call__(self, phase, M, N, K):
        if phase == "begin":
            e = self.torch.cuda.Event(enable_timing=True)
            e.record()
            self.events.append([e, None])
            self.flops += 2.0 * M * N * K
        else:
            e = self.torch.cuda.Event(enable_timing=True)
            e.record()
            self.events[-1][1] = e

    def total_ms(self):
        return sum(a.elapsed_time(b) for a, b in self.events)

    def busy_ms(self):
        spans = sorted((self.base.elapsed_time(a), self.base.elapsed_time(b)) for a, b in self.events)
        busy, cur0, cur1 = 0.0, None, None
        for t0, t1 in spans:
            if cur1 is None or t0 > cur1:
                if cur1 is not None:
                    busy += cur1 - cur0
                cur0, cur1 = t0, t1
            else:
                cur1 = max(cur1, t1)
        if cur1 is not None:
            busy += cur1 - cur0
        return busy


def cpu_baseline(budget_s=20.0):
    """oracle torch-CPU fp32: one layer fwd+bwd at s=2048, b=1 (+ numpy grad
    pack/unpack + torch.optim.AdamW over that layer), scaled to 6 layers."""
    import numpy as np
    import torch

    from oracle import layer as ol

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    p = {
        "ln1_w": torch.ones(H), "ln1_b": torch.zeros(H),
        "qkv_w": torch.randn(3 * H, H, generator=gen) * 0.02, "qkv_b": torch.zeros(3 * H),
        "proj_w": torch.randn(H, H, generator=gen) * 0.02, "proj_b": torch.zeros(H),
        "ln2_w": torch.ones(H), "ln2_b": torch.zeros(H),
        "fc1_w": torch.randn(FFN, H, generator=gen) * 0.02, "fc1_b": torch.zeros(FFN),
        "fc2_w": torch.randn(H, FFN, generator=gen) * 0.02, "fc2_b": torch.zeros(H),
    }
    s, b = SEQ, 1
    x = torch.randn(s, b, H, generator=gen)
    dy = torch.randn(s, b, H, generator=gen) * 1e-3
    params = [torch.nn.Parameter(v.clone()) for v in p.values()]
    opt = torch.optim.AdamW(params, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < 3):
        out, dx, grads = ol.middle_stage_fwd_bwd(x, [p], HEADS, dy)
        flat = np.concatenate([g.numpy().ravel() for g in grads[0].values()])  # pack
        payload = flat * np.float32(1.0)
        off = 0
        for prm, g in zip(params, grads[0].values()):  # unpack
            n = g.numel()
            prm.grad = torch.from_numpy(payload[off : off + n].reshape(g.shape))
            off += n
        opt.step()
        reps += 1
    per_layer = (time.perf_counter() - t0) / reps
    tokens_per_s = (s * b) / (per_layer * LAYERS)
    import platform

    return {
        "value": tokens_per_s,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 layer fwd+bwd fp32 torch-CPU at s={s} b={b} + grad pack/unpack + AdamW, {reps} reps, "
                  f"{per_layer:.2f} s/layer, scaled to {LAYERS} layers ({platform.processor() or 'cpu'})",
    }


def hbm_path(torch, iters=5):
    """Grad pack+unscale+flag+L2+unpack and AdamW over the 24-layer
    GPT-1.3B grad list ([3])."""
    from eth_amd.grad_sync import bucket_plan as bp
    from eth_amd.grad_sync.executor import GradientBucketExecutor, GradientStatistics
    from eth_amd.grad_sync.planner import plan_canonical_fragments
    from eth_amd.grad_sync.bucket_plan import ProcessGroupRegistry
    from eth_amd.grad_sync.metadata import LocalGradientBinding
    from eth_amd.grad_sync.synthetic import descriptors_for, gpt_layer_shapes
    from eth_amd.optimizer.fused_adam import FusedAdamW

    dev = torch.device("cuda:0")
    shapes = gpt_layer_shapes(H, FFN, 24)
    descs = descriptors_for(shapes)
    plan = bp.build_gradient_sync_plan(plan_canonical_fragments(descs, (0,)), "block", 32 << 20, "gpt", "m", "t")
    total = sum(math.prod(s[1]) for s in shapes)
    buf = torch.empty(total, dtype=torch.float32, device=dev)
    buf.normal_(0, 1e-3)
    grads, off = {}, total
    for lid, shape, *_ in shapes:
        n = math.prod(shape)
        off -= n
        grads[lid] = buf[off : off + n].view(shape)
    registry = ProcessGroupRegistry(plan.process_groups, lambda ranks: ranks)
    registry.initialize()
    bindings = [LocalGradientBinding(l, None, grads[l], grads[l].device) for l, *_ in shapes]
    ex = GradientBucketExecutor(plan, 0, descs, bindings, registry, lambda p, h: None)
    st = GradientStatistics(ex.n_partials, dev)
    ex.bind_statistics(st)
    ex.set_inv_loss_scale(1.0)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    t_sync = timed(lambda: (ex.execute(1.0), st.finalize(1.0)))
    params = [torch.nn.Parameter(torch.empty(s[1], device=dev).normal_(0, 0.02)) for s in shapes]
    model = [torch.empty(s[1], device=dev, dtype=torch.bfloat16) for s in shapes]
    for p, (lid, *_) in zip(params, shapes):
        p.grad = grads[lid]
    opt = FusedAdamW([{"params": params}], lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    opt.set_model_copies(dict(zip(params, model)), torch.bfloat16)
    t_adam = timed(lambda: opt.step(stats=st.stats))
    out = {
        "elements": total,
        "grad_sync_ms": t_sync,
        "grad_sync_gbps": 16.0 * total / t_sync / 1e6,
        "adam_ms": t_adam,
        "adam_gbps": 30.0 * total / t_adam / 1e6,
        "peak_gbps": PEAK_HBM_GBPS,
    }
    out["grad_sync_frac"] = out["grad_sync_gbps"] / PEAK_HBM_GBPS
    out["adam_frac"] = out["adam_gbps"] / PEAK_HBM_GBPS
    del ex, st, opt, params, model, buf, grads
    torch.cuda.empty_cache()
    return out


def first_last_stage(torch, steps=5, warmup=2):
    """the GPT-6.7B first+last stage in fp16 -- token +
    position embedding, 2 layers (hidden 4096, 32 heads, FFN 16384), final
    LN, tied LM head over the padded vocabulary (50304) and vocab cross
    entropy on the reference's synthetic batch (labels 0), seq 2048,
    micro-batch 2; dynamic loss scale (2^16), grad sync, tied-gradient sum,
    unscale + clip 1.0, AdamW with the fp16 model copy."""
    from eth_amd.model.flex_ops import GPTConfig
    from eth_amd.stage import FirstLastStageTrainer

    h, heads, f, layers, s, b, V = 4096, 32, 16384, 2, 2048, 2, 50304
    cfg = GPTConfig(hidden_size=h, num_attention_heads=heads, ffn_hidden_size=f, num_layers=layers, seq_length=s,
                    micro_batch_size=b, padded_vocab_size=V, params_dtype=torch.float16, device="cuda", seed=1234)
    tr = FirstLastStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0,
                               bucket_cap_bytes=32 << 20, initial_loss_scale=2.0**16)
    for i in range(warmup):
        tr.train_step([2 * i, 2 * i + 1])
    torch.cuda.synchronize()
    quiet_gc()
    t0 = time.perf_counter()
    oks = 0
    for i in range(steps):
        _, _, ok, _ = tr.train_step([2 * (warmup + i), 2 * (warmup + i) + 1])
        oks += bool(ok)
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / steps
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
        "step_tflops": tflops,
        "step_mfma_frac": tflops / PEAK_BF16_TFLOPS,
        "dtype": "f16",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-hbm-path", action="store_true")
    ap.add_argument("--no-first-last", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed steps, copy 1 GiB once (the calibration kernel of the "
                         "FETCH_SIZE / WRITE_SIZE counter runs behind roofline.traffic)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every GPU box of this build has a single MI355X and no "
              "collective is exercised (see DESIGN.md for how the stage shards)", file=sys.stderr)
        sys.exit(2)

    import torch

    from eth_amd import kernels as K
    from eth_amd.model.flex_ops import GPTConfig
    from eth_amd.stage import MiddleStageTrainer

    cfg = GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=LAYERS,
                    seq_length=SEQ, micro_batch_size=MB, params_dtype=torch.bfloat16, device="cuda", seed=1234)
    tr = MiddleStageTrainer(cfg, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad=1.0)
    g = torch.Generator(device="cuda").manual_seed(1234)
    x = torch.randn(SEQ, MB, H, device="cuda", generator=g).to(torch.bfloat16)
    dy = (torch.randn(SEQ, MB, H, device="cuda", generator=g) * 1e-3).to(torch.bfloat16)
    for _ in range(args.warmup):
        tr.train_step(x, dy)
    torch.cuda.synchronize()
    quiet_gc()

    meter = GemmMeter(torch)
    K.set_gemm_observer(meter)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out, dx, ok, norm = tr.train_step(x, dy)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    K.set_gemm_observer(None)
    ms = 1e3 * elapsed / args.steps
    tokens = SEQ * MB
    value = tokens * args.steps / elapsed
    gemm_ms = meter.busy_ms()
    gemm_sum_ms = meter.total_ms()
    gemm_tflops = meter.flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0
    step_tflops = step_flops() / (ms * 1e-3) / 1e12

    result = {
        "metric": "stage train tokens/s (GPT-1.3B, 6 layers) on 1 GPU; grad-pack+Adam HBM GB/s",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
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
            "kernel": "eth_gemm (gemm256_m16_kernel, gemm256_m32_kernel and gemm_kernel: all GEMM launches of the timed steps)",
            "bound": "mfma",
            "achieved": gemm_tflops,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_tflops / PEAK_BF16_TFLOPS,
            "traffic": GEMM_TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "algorithmic_bytes_per_launch": GEMM_ALGORITHMIC_BYTES_PER_LAUNCH,
            "launches": len(meter.events),
            "gemm_ms_per_step": gemm_ms / args.steps,
            "time_basis": "union of the GEMM launch intervals (weight-gradient GEMMs run on a side stream, "
                          "overlapped with the data-gradient chain)",
            "launch_sum_ms_per_step": gemm_sum_ms / args.steps,
            "achieved_over_launch_sum": meter.flops / (gemm_sum_ms * 1e-3) / 1e12 if gemm_sum_ms > 0 else 0.0,
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
        result["first_last_stage"] = first_last_stage(torch)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
