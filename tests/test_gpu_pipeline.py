"""GPU tests of the 1F1B pipeline step over stages sharing the GPU
(schedules.py:595-713, p2p_communication.py:200-538): the pipelined order
against one microbatch at a time, bit for bit, with cuts at and inside a
layer; the step's one clip norm over all stages and its AdamW result
against the fp32 oracle; one overflow decision for every stage; and a GPT
pipeline from the embedding to the loss, with the tied word embedding
split between its first and last stages, against the first+last stage and
the fp64 oracle."""

import numpy as np
import pytest
import torch

from eth_amd.loss import global_normalization_scale
from eth_amd.model.flex_ops import GPTConfig
from eth_amd.optimizer.optimizer import step_model_parallel_group
from eth_amd.schedules import PipelineTrainer, build_gpt_pipeline, forward_backward_pipelining_without_interleaving
from eth_amd.stage import FirstLastStageTrainer, MiddleStageTrainer
from oracle import adamw as oadam
from oracle import gradsync as og
from oracle import layer as ol
from tests.conftest import announce

pytestmark = pytest.mark.gpu
H, HEADS, FFN, SEQ, MB = 256, 4, 1024, 128, 2


def _cfg(dtype=torch.bfloat16, dropout=0.0):
    return GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=2, seq_length=SEQ,
                     micro_batch_size=MB, hidden_dropout=dropout, params_dtype=dtype, device="cuda", seed=5)


def _rel(a, b):
    a, b = torch.as_tensor(a).double().cpu(), torch.as_tensor(b).double().cpu()
    return (a - b).norm().item() / (b.norm().item() + 1e-30)


def _stages(cuts, gen, dtype=torch.bfloat16, dropout=0.0, **kw):
    """Stages over the op ranges `cuts`, with the weights (biases random) of
    one uncut 2-layer stage."""
    whole = MiddleStageTrainer(_cfg(dtype, dropout))
    with torch.no_grad():
        for name, p in whole.model.named_parameters():
            if name.endswith("bias"):
                p.copy_((torch.randn(p.shape, generator=gen) * 0.02).to(p.dtype))
    whole.optimizer.reload_model_params()
    by_index = {op.op_index: op for op in whole.model.language_model.ops}
    stages = []
    for lo, hi in cuts:
        st = MiddleStageTrainer(_cfg(dtype, dropout), op_range=(lo, hi), **kw)
        with torch.no_grad():
            for op in st.model.language_model.ops:
                for (n1, p1), (n2, p2) in zip(op.named_parameters(), by_index[op.op_index].named_parameters()):
                    assert n1 == n2
                    p1.copy_(p2)
        st.optimizer.reload_model_params()
        stages.append(st)
    return whole, stages


def _microbatches(gen, m, dtype=torch.bfloat16):
    out = []
    for _ in range(m):
        x = torch.randn(SEQ, MB, H, generator=gen).to(dtype).cuda()
        dy = (torch.randn(SEQ, MB, H, generator=gen) * 1e-2).to(dtype).cuda()
        out.append({"input_tensors": {"hidden_states": x}, "output_grads": {"hidden_states": dy}})
    return out


def _masters(stages):
    return [{n: st.optimizer.optimizer_parameter_for_model_parameter(p).detach().clone()
             for n, p in st.model.named_parameters()} for st in stages]


def _main_grads(stages):
    return [{n: p.main_grad.detach().clone() for n, p in st.model.named_parameters()} for st in stages]


@pytest.mark.parametrize("cuts,m,dropout", [
    (((1, 5), (5, 21)), 4, 0.0),            # inside a layer: side-channel tensors cross
    (((1, 11), (11, 21)), 4, 0.1),          # at the layer boundary, with dropout
    (((1, 8), (8, 14), (14, 21)), 2, 0.0),  # fewer microbatches than warm-up slots
    (((1, 8), (8, 14), (14, 21)), 5, 0.1),
])
def test_1f1b_step_equals_one_microbatch_at_a_time(cuda, cuts, m, dropout):
    """The 1F1B step against the same stages run one microbatch at a time:
    outputs, input gradients, every main grad, the norm and every fp32
    master after the step are identical, and the pipeline held at most
    min(p - r, m) microbatches' activations on stage r."""
    announce(f"1F1B vs sequential, cuts {cuts}, m {m}, dropout {dropout}")
    runs = {}
    for schedule in ("1f1b", "sequential"):
        gen = torch.Generator().manual_seed(11)
        _whole, stages = _stages(cuts, gen, dropout=dropout)
        mbs = _microbatches(gen, m)
        pipe = PipelineTrainer(stages, schedule=schedule)
        results, steps = pipe.train_step(mbs)
        torch.cuda.synchronize()
        runs[schedule] = (results, steps, _main_grads(stages), _masters(stages), pipe.last_timeline)
    (r1, s1, g1, w1, t1), (r0, s0, g0, w0, t0) = runs["1f1b"], runs["sequential"]
    p = len(cuts)
    assert t1["peak_in_flight"] == [min(p - r, m) for r in range(p)] and t0["peak_in_flight"] == [1] * p
    assert t1["ticks"] == 2 * (m + p - 1)
    for (o1, e1, i1, x1), (o0, e0, i0, x0) in zip(r1, r0):
        assert torch.equal(o1["hidden_states"], o0["hidden_states"])
        assert torch.equal(i1["hidden_states"], i0["hidden_states"])
        assert e1 == {} and x1 == {} and e0 == {} and x0 == {}
    assert [ok for ok, _, _ in s1] == [True] * p == [ok for ok, _, _ in s0]
    # one norm for the whole pipeline
    assert len({n for _, n, _ in s1}) == 1 and s1[0][1] == s0[0][1]
    for a, b in zip(g1, g0):
        for name in a:
            assert torch.equal(a[name], b[name]), name
    for a, b in zip(w1, w0):
        for name in a:
            assert torch.equal(a[name], b[name]), name


def test_pipelined_step_matches_the_oracle_with_one_clip_norm(cuda):
    """Two stages cut at the layer boundary, three microbatches, a clip
    threshold the gradients exceed: each microbatch's output and input
    gradient against the fp32 oracle of the uncut stage (2e-2), the
    accumulated main grads against the oracle's sum over the microbatches
    (norm within 2e-2, relative error 5e-2), the returned norm against the
    L2 norm of every stage's gradients together (1e-6; each stage's own
    norm is smaller), and the fp32 masters against the oracle's
    clip / AdamW chain with that norm (1e-6)."""
    announce("pipelined step vs fp32 oracle, one clip norm")
    gen = torch.Generator().manual_seed(12)
    whole, stages = _stages(((1, 11), (11, 21)), gen, clip_grad=0.05, lr=1e-3)
    mbs = _microbatches(gen, 3)
    before = _masters(stages)
    layers = [stages[0].layer_parameters()[0], stages[1].layer_parameters()[0]]
    host = [{k: p.detach().float().cpu() for k, p in layer.items()} for layer in layers]
    results, steps = PipelineTrainer(stages).train_step(mbs)
    torch.cuda.synchronize()
    ref_grads = None
    for mb, (out, _e, in_g, _x) in zip(mbs, results):
        x = mb["input_tensors"]["hidden_states"].float().cpu()
        dy = mb["output_grads"]["hidden_states"].float().cpu()
        ref_out, ref_dx, grads = ol.middle_stage_fwd_bwd(x, host, HEADS, dy)
        assert _rel(out["hidden_states"], ref_out) < 2e-2
        assert _rel(in_g["hidden_states"], ref_dx) < 2e-2
        ref_grads = grads if ref_grads is None else [{k: a[k] + g[k] for k in a} for a, g in zip(ref_grads, grads)]
    got = [{k: p.main_grad.detach().cpu().numpy().copy() for k, p in layer.items()} for layer in layers]
    for li in range(2):
        assert sorted(got[li]) == sorted(ref_grads[li])
        for k, r in ref_grads[li].items():
            gn, rn = np.linalg.norm(got[li][k].astype(np.float64)), r.double().norm().item()
            assert abs(gn - rn) <= 2e-2 * rn + 1e-12, (li, k)
            assert _rel(got[li][k], r) < 5e-2, (li, k)
    norm = steps[0][1]
    assert all(ok for ok, _, _ in steps) and all(n == norm for _, n, _ in steps)
    ref_norm = og.l2_norm([g for layer in got for g in layer.values()])
    assert norm == pytest.approx(ref_norm, rel=1e-6)
    assert all(og.l2_norm(list(layer.values())) < 0.99 * ref_norm for layer in got)
    coef = og.clip_coefficient(ref_norm, 0.05)
    assert coef < 1.0
    for si, (st, layer) in enumerate(zip(stages, layers)):
        names = {id(p): n for n, p in st.model.named_parameters()}
        for k, p in layer.items():
            wd = 0.1 if k.endswith("_w") and not k.startswith("ln") else 0.0
            m0 = before[si][names[id(p)]].cpu().numpy()
            zeros = np.zeros_like(got[si][k])
            ref_p, _, _ = oadam.adamw_step(m0, got[si][k], zeros, zeros, 1, 1e-3, 0.9, 0.95, 1e-8, wd, clip_coef=coef)
            new = st.optimizer.optimizer_parameter_for_model_parameter(p).detach().cpu().numpy()
            np.testing.assert_allclose(new, ref_p, rtol=1e-6, atol=1e-9, err_msg=f"stage {si} {k}")


def test_an_overflow_on_one_stage_skips_every_stage(cuda):
    """fp16 stages: an inf in the last stage's gradients skips the step on
    both stages (one overflow decision, optimizer.py:449-461), the masters
    stay as they were, and the next clean step updates both."""
    announce("fp16 pipeline, overflow on one stage")
    gen = torch.Generator().manual_seed(13)
    _whole, stages = _stages(((1, 11), (11, 21)), gen, dtype=torch.float16)
    mbs = _microbatches(gen, 2, dtype=torch.float16)
    before = _masters(stages)
    for s in stages:
        s.ddp.zero_grad_buffer(defer=True)
    forward_backward_pipelining_without_interleaving(stages, mbs)
    for s in stages:
        s.ddp.settle_grad_buffer()
    with torch.no_grad():
        next(iter(stages[1].model.parameters())).main_grad.view(-1)[5] = float("inf")
    for s in stages:
        s.grad_sync.execute(1.0)
    steps = step_model_parallel_group([s.optimizer for s in stages])
    torch.cuda.synchronize()
    assert [ok for ok, _, _ in steps] == [False, False]
    for a, b in zip(before, _masters(stages)):
        for name in a:
            assert torch.equal(a[name], b[name]), name
    scales = {s.optimizer.grad_scaler.host_scale for s in stages}
    assert len(scales) == 1
    results, steps = PipelineTrainer(stages).train_step(mbs)
    torch.cuda.synchronize()
    assert [ok for ok, _, _ in steps] == [True, True]
    after = _masters(stages)
    for a, b in zip(before, after):
        assert any(not torch.equal(a[n], b[n]) for n in a)


# ------------------------------------------------------------ GPT pipeline --
N_OPS = 23  # embedding, 2 x 10 layer ops, final LayerNorm, LM head + loss


def _gpt_cfg(dtype):
    return GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=2, seq_length=SEQ,
                     micro_batch_size=1, padded_vocab_size=50304, params_dtype=dtype, device="cuda", seed=11)


def _gpt_pipeline(cuts, whole, dtype, **kw):
    """A GPT pipeline over `cuts` holding the weights of the first+last
    stage `whole`, the tied copy initialised from the root."""
    pipe = build_gpt_pipeline(_gpt_cfg(dtype), cuts, **kw)
    assert [st.global_rank for st in pipe.stages] == list(range(len(cuts)))
    by_index = {op.op_index: op for op in whole.model.language_model.ops}
    for st in pipe.stages:
        with torch.no_grad():
            for op in st.model.language_model.ops:
                for (n1, p1), (n2, p2) in zip(op.named_parameters(), by_index[op.op_index].named_parameters()):
                    assert n1 == n2
                    p1.copy_(p2)
        st.optimizer.reload_model_params()
    pipe.tie_embeddings()
    return pipe


def _by_op(trainers):
    """{(op index, parameter name): parameter} over the trainers' ops."""
    out = {}
    for tr in trainers:
        for op in tr.model.language_model.ops:
            for n, p in op.named_parameters():
                out[(op.op_index, n)] = p
    return out


GPT_CUTS = [((0, 11), (11, N_OPS)), ((0, 6), (6, 16), (16, N_OPS)), ((0, N_OPS),)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cuts", GPT_CUTS)
def test_gpt_pipeline_step_equals_the_first_last_stage(cuda, cuts, dtype):
    """Embedding to loss in 1, 2 or 3 stages (cuts at a layer boundary, and
    inside both layers), four one-sample microbatches in the 1F1B order,
    against the same model on one first+last stage running them one at a
    time: per-token losses, the summed loss, every synced and tied main
    grad equal bit for bit, one norm, and the fp32 masters after the step
    within 1e-6.  The one exception: where a cut separates a bias-dropout-add
    from the LayerNorm after it (which one stage runs as one fused kernel),
    the bias gradient of the linear before it is summed by the unfused
    kernel, in another order, and agrees to 1e-6."""
    announce(f"GPT pipeline {cuts} {dtype} vs first+last")
    whole = FirstLastStageTrainer(_gpt_cfg(dtype))
    pipe = _gpt_pipeline(cuts, whole, dtype)
    ids = [[3], [8], [5], [1]]
    losses, (num, weight), ok, norm = whole.train_step_microbatches(ids)
    results, steps = pipe.train_step([{"sample_ids": i} for i in ids])
    torch.cuda.synchronize()
    assert ok and all(o for o, _, _ in steps)
    for (out, _e, in_g, _x), ref in zip(results, losses):
        assert torch.equal(out["losses"], ref) and in_g == {}
    p_num, p_weight = pipe.last_loss
    assert torch.equal(p_num, num) and torch.equal(p_weight, weight)
    assert len({n for _, n, _ in steps}) == 1
    assert steps[0][1] == pytest.approx(norm, rel=1e-9)
    mine, ref = _by_op(pipe.stages), _by_op([whole])
    assert sorted(mine) == sorted(ref)
    stage_of = {key: st for st in pipe.stages for key in _by_op([st])}
    # a stage that ends in a dropout op (index 5 or 0 mod 10) hands the
    # LayerNorm after it to the next stage
    split = {(hi - 2, "dense.bias") for _, hi in cuts[:-1] if (hi - 1) % 10 in (5, 0)}
    for key, p in ref.items():
        if key in split:
            assert _rel(mine[key].main_grad, p.main_grad) < 1e-6, key
        else:
            assert torch.equal(mine[key].main_grad, p.main_grad), key
        got = stage_of[key].optimizer.optimizer_parameter_for_model_parameter(mine[key]).detach()
        want = whole.optimizer.optimizer_parameter_for_model_parameter(p).detach()
        assert _rel(got, want) < 1e-6, key
    # the tied copies stay equal
    assert torch.equal(pipe.stages[0].tied_root, pipe.stages[-1].tied_copy)


def test_gpt_pipeline_gradients_match_the_fp64_oracle(cuda):
    """Two one-sample microbatches through a 2-stage GPT pipeline: the
    per-token losses and the synced, tied main grads against the fp64
    oracle of the whole model on the 2-sample batch (the gradient of the
    masked mean over both samples): losses within 2e-2, each gradient's norm
    within 2e-2 and its relative error within 5e-2."""
    announce("GPT pipeline vs fp64 oracle")
    from eth_amd.loss import synthetic_gpt_batch
    from tests.test_gpu_full_stage import _oracle_params, tr_layer_params

    whole = FirstLastStageTrainer(_gpt_cfg(torch.bfloat16))
    params = _oracle_params(whole)
    pipe = _gpt_pipeline(GPT_CUTS[0], whole, torch.bfloat16)
    tokens, mask, positions, _ = synthetic_gpt_batch([3, 8], SEQ, 50257, "cpu")
    ref_losses, ref_mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, HEADS)
    results, steps = pipe.train_step([{"sample_ids": [3]}, {"sample_ids": [8]}])
    torch.cuda.synchronize()
    assert all(o for o, _, _ in steps)
    assert _rel(torch.cat([r[0]["losses"] for r in results]), ref_losses) < 2e-2
    num, weight = pipe.last_loss
    assert abs((num / weight).item() - ref_mean.item()) < 2e-2 * abs(ref_mean.item())
    first, last = pipe.stages
    ops0 = first.model.language_model.ops
    ops1 = last.model.language_model.ops
    checks = [(first.tied_root, grads["word"]), (last.tied_copy, grads["word"]),
              (ops0[0].position_embeddings.weight, grads["pos"]),
              (ops1[-2].input_layernorm.weight, grads["lnf_w"]), (ops1[-2].input_layernorm.bias, grads["lnf_b"])]
    layer_params = tr_layer_params(first) + tr_layer_params(last)
    assert len(layer_params) == 2
    for lp, gl in zip(layer_params, grads["layers"]):
        checks += [(p, gl[k]) for k, p in lp.items()]
    for p, r in checks:
        g = p.main_grad
        gn, rn = g.double().norm().item(), r.double().norm().item()
        assert abs(gn - rn) <= 2e-2 * rn + 1e-12
        assert _rel(g, r) < 5e-2


def test_gpt_pipeline_overflow_in_the_tied_sum_skips_every_stage(cuda):
    """fp16, three stages: an inf in the LM head's copy of the word
    embedding gradient reaches the root through the cross-stage tied sum;
    the root's stage flags it and every stage skips the step, with its
    masters untouched and one loss scale."""
    announce("GPT pipeline fp16 overflow through the tied sum")
    whole = FirstLastStageTrainer(_gpt_cfg(torch.float16))
    pipe = _gpt_pipeline(GPT_CUTS[1], whole, torch.float16)
    before = _masters(pipe.stages)
    last = pipe.stages[-1]
    mbs = [{"sample_ids": [3]}, {"sample_ids": [8]}]
    last.begin_step(2.0 * SEQ)
    for s in pipe.stages:
        s.ddp.zero_grad_buffer(defer=True)
    forward_backward_pipelining_without_interleaving(pipe.stages, mbs)
    for s in pipe.stages:
        s.ddp.settle_grad_buffer()
    scale = global_normalization_scale(2.0 * SEQ, last.step_loss_weight())
    for s in pipe.stages:
        s.grad_sync.execute(scale)
    with torch.no_grad():
        last.tied_copy.main_grad.view(-1)[17] = float("inf")
    pipe._tie_gradients()
    steps = step_model_parallel_group([s.optimizer for s in pipe.stages])
    torch.cuda.synchronize()
    assert [ok for ok, _, _ in steps] == [False] * 3
    for a, b in zip(before, _masters(pipe.stages)):
        for name in a:
            assert torch.equal(a[name], b[name]), name
    assert len({s.optimizer.grad_scaler.host_scale for s in pipe.stages}) == 1
    # the next clean step applies on every stage
    _results, steps = pipe.train_step(mbs)
    torch.cuda.synchronize()
    assert [ok for ok, _, _ in steps] == [True] * 3


def test_gpt_pipeline_overlapped_update_is_bit_identical_over_steps(cuda):
    """Three steps of a 2-stage GPT pipeline with every stage's AdamW update
    overlapped with its next forward against the same pipeline updating in
    line: per-token losses of every step, norms and the fp32 masters after
    the last step are identical (the second and third steps' forwards wait
    for the overlapped parts op by op)."""
    announce("GPT pipeline, overlapped update vs in line, 3 steps")
    whole = FirstLastStageTrainer(_gpt_cfg(torch.bfloat16))
    runs = []
    for overlap in (False, True):
        pipe = _gpt_pipeline(GPT_CUTS[0], whole, torch.bfloat16, overlap_optimizer=overlap)
        losses, norms = [], []
        for step in range(3):
            results, steps = pipe.train_step([{"sample_ids": [3 + step]}, {"sample_ids": [8 + step]}])
            assert all(ok for ok, _, _ in steps)
            losses.append(torch.cat([r[0]["losses"] for r in results]))
            norms.append(steps[0][1])
        for st in pipe.stages:
            st.optimizer.join_overlapped_update()
        torch.cuda.synchronize()
        runs.append((losses, norms, _masters(pipe.stages)))
    (l0, n0, m0), (l1, n1, m1) = runs
    assert n0 == n1
    for a, b in zip(l0, l1):
        assert torch.equal(a, b)
    for a, b in zip(m0, m1):
        for name in a:
            assert torch.equal(a[name], b[name]), name
