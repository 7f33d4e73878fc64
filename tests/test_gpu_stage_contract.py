"""GPU tests of the stage's dict contract around the kernels: stage cuts
inside a layer with side-channel tensors crossing the cut
(schedules.py:113-227, flex_model.py:63-240), several microbatches per step
(schedules.py:236-281), activation recompute (flex_model.py:395-588), and the
evidence the executor and the trainers write (grad_sync/runtime_evidence.py,
grad_sync/evidence.py)."""

import hashlib
import json

import numpy as np
import pytest
import torch

from eth_amd.grad_sync.evidence import load_rank_snapshot
from eth_amd.grad_sync.executor import GradientBucketExecutor
from eth_amd.model.flex_ops import GPTConfig
from eth_amd.stage import FirstLastStageTrainer, MiddleStageTrainer
from oracle import gradsync as og
from oracle import layer as ol
from tests.conftest import announce
from tests.helpers import known_answers, runtime_binding
from tests.test_evidence_host import evidence_plan

pytestmark = pytest.mark.gpu
KA = known_answers()
H, HEADS, FFN, SEQ, MB = 256, 4, 1024, 128, 2


def _cfg(dtype=torch.bfloat16, layers=2, dropout=0.0, mb=MB, seed=5):
    return GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=layers,
                     seq_length=SEQ, micro_batch_size=mb, hidden_dropout=dropout, params_dtype=dtype, device="cuda",
                     seed=seed)


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return (a - b).norm().item() / (b.norm().item() + 1e-30)


def _named_grads(tr):
    return {name: p.main_grad.clone() for name, p in tr.model.named_parameters()}


def _copy_weights(src, dst):
    """Give dst's parameters (a sub-range of src's ops) src's values."""
    by_index = {op.op_index: op for op in src.model.language_model.ops}
    with torch.no_grad():
        for op in dst.model.language_model.ops:
            for (n1, p1), (n2, p2) in zip(op.named_parameters(), by_index[op.op_index].named_parameters()):
                assert n1 == n2
                p1.copy_(p2)
    dst.optimizer.reload_model_params()


def _randomize(tr, gen):
    with torch.no_grad():
        for name, p in tr.model.named_parameters():
            if name.endswith("bias"):
                p.copy_((torch.randn(p.shape, generator=gen) * 0.02).to(p.dtype))
    tr.optimizer.reload_model_params()


def _check_against_oracle(whole, x, dy, out, dx, grads):
    """The stage's output, input gradient and main grads (`grads`: per layer,
    oracle parameter name -> tensor) against the fp32 CPU oracle of the
    uncut stage on `whole`'s weights: output and input gradient within 2e-2,
    each gradient's norm within 2e-2 and its relative error within 5e-2
    (the north-star bars)."""
    host = [{k: p.detach().float().cpu() for k, p in layer.items()} for layer in whole.layer_parameters()]
    ref_out, ref_dx, ref_grads = ol.middle_stage_fwd_bwd(x.float().cpu(), host, HEADS, dy.float().cpu())
    assert _rel(out, ref_out) < 2e-2
    assert _rel(dx, ref_dx) < 2e-2
    assert len(grads) == len(ref_grads)
    for li, ref in enumerate(ref_grads):
        assert sorted(grads[li]) == sorted(ref)
        for k, r in ref.items():
            g = grads[li][k]
            gn, rn = g.double().norm().item(), r.double().norm().item()
            assert abs(gn - rn) <= 2e-2 * rn + 1e-12, (li, k, gn, rn)
            assert _rel(g, r) < 5e-2, (li, k, _rel(g, r))


def _layer_main_grads(*trainers):
    """{layer: {oracle name: main grad}} merged over stages that together
    cover whole layers (a cut layer's ops come from two trainers)."""
    merged = {}
    for tr in trainers:
        for li, layer in enumerate(tr.layer_parameters()):
            first = (min(op.op_index for op in tr.model.language_model.ops) - 1) // 10
            merged.setdefault(first + li, {}).update({k: p.main_grad for k, p in layer.items()})
    return [merged[k] for k in sorted(merged)]


def _inputs(gen, dtype=torch.bfloat16, mb=MB):
    x = torch.randn(SEQ, mb, H, generator=gen).to(dtype).cuda()
    dy = (torch.randn(SEQ, mb, H, generator=gen) * 1e-2).to(dtype).cuda()
    return x, dy


def test_stage_cut_inside_a_layer_gives_the_uncut_gradients(cuda):
    """Ops [1, 5) and [5, 21) of a 2-layer model: the first stage ends at the
    attention projection, so the LayerNorm residual (hidden_states_1) and the
    projection bias (output_bias) cross the cut as side-channel tensors.
    Outputs, the input gradient and every main grad equal the uncut stage's
    bit for bit, except the projection bias, whose gradient crosses the cut
    as a bf16 tensor (as in the reference) instead of straight into fp32;
    and the cut pair's outputs, input gradient and main grads match the fp32
    oracle of the whole stage."""
    announce("stage cut inside a layer")
    gen = torch.Generator().manual_seed(3)
    whole = MiddleStageTrainer(_cfg())
    _randomize(whole, gen)
    first = MiddleStageTrainer(_cfg(), op_range=(1, 5))
    second = MiddleStageTrainer(_cfg(), op_range=(5, 21))
    _copy_weights(whole, first)
    _copy_weights(whole, second)
    x, dy = _inputs(gen)
    for tr in (whole, first, second):
        tr.ddp.zero_grad_buffer()
    out_w, dx_w = whole.forward_backward(x, dy)
    a_out, a_extra, a_leaves = first.forward_step({"hidden_states": x})
    assert sorted(a_out) == ["output_tensor"] and sorted(a_extra) == ["hidden_states_1", "output_bias"]
    b_out, b_extra, b_leaves = second.forward_step(a_out, a_extra)
    assert b_extra == {}
    b_in_grads, b_extra_grads = second.backward_step(b_out, {"hidden_states": dy}, b_extra, {}, b_leaves)
    assert sorted(b_extra_grads) == ["hidden_states_1", "output_bias"]
    a_in_grads, _ = first.backward_step(a_out, b_in_grads, a_extra, b_extra_grads, a_leaves)
    torch.cuda.synchronize()
    assert torch.equal(b_out["hidden_states"], out_w)
    assert torch.equal(a_in_grads["hidden_states"], dx_w)
    gw = _named_grads(whole)
    cut = {**{f"0.{k}": v for k, v in _named_grads(first).items()}, **{f"1.{k}": v for k, v in _named_grads(second).items()}}
    by_index = {}
    for tr, tag in ((first, "0"), (second, "1")):
        for op in tr.model.language_model.ops:
            for n, p in op.named_parameters():
                by_index[(op.op_index, n)] = p.main_grad
    for op in whole.model.language_model.ops:
        for n, p in op.named_parameters():
            g = by_index[(op.op_index, n)]
            if op.name == "enc-attention-dense" and n == "dense.bias" and op.op_index == 4:
                assert _rel(g, p.main_grad) < 1e-2, (op.op_index, n)
            else:
                assert torch.equal(g, p.main_grad), (op.op_index, n)
    assert len(cut) == len(gw)
    _check_against_oracle(whole, x, dy, b_out["hidden_states"], a_in_grads["hidden_states"],
                          _layer_main_grads(first, second))


def test_microbatches_accumulate_main_grads(cuda):
    """Two microbatches in one step: every main grad is the fp32 sum of the
    two microbatches' gradients (bit for bit against running them one at a
    time), the outputs and input gradients are each microbatch's own, and
    the step applies once."""
    announce("two microbatches per step")
    gen = torch.Generator().manual_seed(4)
    tr = MiddleStageTrainer(_cfg())
    _randomize(tr, gen)
    mbs = [_inputs(gen) for _ in range(2)]
    singles = []
    for x, dy in mbs:
        tr.ddp.zero_grad_buffer()
        out, dx = tr.forward_backward(x, dy)
        singles.append((out.clone(), dx.clone(), _named_grads(tr)))
    results, ok, norm = tr.train_step_microbatches(
        [{"input_tensors": {"hidden_states": x}, "output_grads": {"hidden_states": dy}} for x, dy in mbs]
    )
    torch.cuda.synchronize()
    assert ok and np.isfinite(norm)
    for (out, _extra, in_g, _eg), (s_out, s_dx, _) in zip(results, singles):
        assert torch.equal(out["hidden_states"], s_out)
        assert torch.equal(in_g["hidden_states"], s_dx)
    # the main grads after the step hold the synced (unscaled, unclipped)
    # sum; recompute it from the single runs
    for name, p in tr.model.named_parameters():
        expect = singles[0][2][name] + singles[1][2][name]
        assert torch.equal(p.main_grad, expect), name


@pytest.mark.parametrize("pattern", ["all", "attention-only"])
@pytest.mark.parametrize("dropout", [0.0, 0.1])
def test_recompute_is_bit_identical(cuda, pattern, dropout):
    """Activation recompute over whole layers, or over the middle of each
    layer (ops 1-6: QKV to the 2nd LayerNorm, so side-channel tensors cross
    the segment edges), gives the outputs, input gradient and main grads of
    the plain stage bit for bit, with dropout masks replayed; without
    dropout the recomputed stage also matches the fp32 oracle (which has no
    dropout)."""
    announce(f"recompute {pattern} dropout {dropout}")
    gen = torch.Generator().manual_seed(6)
    flags = {"all": [1] * 20, "attention-only": ([0] + [1] * 6 + [0] * 3) * 2}[pattern]
    plain = MiddleStageTrainer(_cfg(dropout=dropout))
    ckpt = MiddleStageTrainer(_cfg(dropout=dropout), recompute_ops=flags)
    _randomize(plain, gen)
    _copy_weights(plain, ckpt)
    x, dy = _inputs(gen)
    for tr in (plain, ckpt):
        tr.model.train()
        tr.ddp.zero_grad_buffer()
    out_p, dx_p = plain.forward_backward(x, dy)
    out_c, dx_c = ckpt.forward_backward(x, dy)
    torch.cuda.synchronize()
    assert torch.equal(out_p, out_c)
    assert torch.equal(dx_p, dx_c)
    gp, gc = _named_grads(plain), _named_grads(ckpt)
    for name in gp:
        assert torch.equal(gp[name], gc[name]), name
    if dropout:
        assert any(getattr(op, "_calls", 0) for op in ckpt.model.language_model.ops)
    else:
        _check_against_oracle(ckpt, x, dy, out_c, dx_c, _layer_main_grads(ckpt))


def test_first_last_microbatches_match_the_fp64_oracle(cuda):
    """Two microbatches of one sample each on the first+last stage: the
    synced main grads are the gradients of the masked mean over both
    samples (fp64 oracle on the 2-sample batch)."""
    announce("first+last, two microbatches")
    from tests.test_gpu_full_stage import _oracle_params, tr_layer_params

    cfg = GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=2, seq_length=SEQ,
                    micro_batch_size=1, padded_vocab_size=50304, params_dtype=torch.bfloat16, device="cuda", seed=11)
    tr = FirstLastStageTrainer(cfg, initial_loss_scale=1.0)
    params = _oracle_params(tr)
    from eth_amd.loss import synthetic_gpt_batch

    tokens, mask, positions, _ = synthetic_gpt_batch([3, 8], SEQ, 50257, "cpu")
    ref_losses, ref_mean, grads = ol.full_model_fwd_bwd(tokens, positions, mask, params, HEADS)
    # stop before the optimizer: run the pieces of train_step_microbatches
    tr.ddp.zero_grad_buffer(defer=True)
    outs = [tr.forward_backward([i], nominal=2.0 * SEQ) for i in (3, 8)]
    tr.ddp.settle_grad_buffer()
    from eth_amd.loss import global_normalization_scale, sum_loss_outputs

    num, weight = sum_loss_outputs([lo for _, lo in outs])
    tr.grad_sync.execute(global_normalization_scale(2.0 * SEQ, weight))
    tr.tie_gradients()
    torch.cuda.synchronize()
    assert _rel(torch.cat([l for l, _ in outs]), ref_losses) < 2e-2
    assert abs((num / weight).item() - ref_mean.item()) < 2e-2 * abs(ref_mean.item())
    checks = [(tr.embedding.word_embeddings.weight, grads["word"]), (tr.embedding.position_embeddings.weight, grads["pos"])]
    for lp, gl in zip(tr_layer_params(tr), grads["layers"]):
        checks += [(p, gl[k]) for k, p in lp.items()]
    for p, ref in checks:
        assert _rel(p.main_grad, ref) < 5e-2
    # and the packaged step applies
    losses, (num, weight), ok, norm = tr.train_step_microbatches([[3], [8]])
    assert ok and np.isfinite(norm)


def test_executor_runtime_evidence_hashes_the_packed_bytes(cuda, tmp_path):
    """The reference's known answer (4 tensor-mode vs 2 block-mode
    collectives, equal payload hash) through the HIP pack: every bucket's
    hash is the SHA-256 of the oracle's packed payload."""
    announce("runtime evidence through the executor")
    rec = KA["runtime_evidence_four_to_two"]

    class Registry:
        group_count = 2
        creation_count = 2

        def handle(self, gid):
            return gid

    reports = {}
    for mode in ("tensor", "block"):
        plan = evidence_plan(rec, mode)
        grads = {lid: torch.tensor(v, device=cuda) for lid, v in rec["tensors"].items()}
        descs = [type("D", (), {"logical_param_id": lid, "partition_dim": 0})() for lid in grads]
        ex = GradientBucketExecutor(plan, 0, descs, [runtime_binding(l, t) for l, t in grads.items()], Registry(),
                                    lambda payload, handle: None, runtime_evidence_dir=tmp_path / mode)
        for _ in range(rec["iterations"]):
            for lid, v in rec["tensors"].items():
                grads[lid].copy_(torch.tensor(v))
            ex.execute()
        host = {lid: np.asarray(v, dtype=np.float32) for lid, v in rec["tensors"].items()}
        packed = og.execute(plan, 0, {l: type("D", (), {"partition_dim": 0})() for l in host}, host)
        report = json.loads((tmp_path / mode / "rank-00000.json").read_text())
        reports[mode] = report
        it = report["iterations"][-1]
        assert it["collective_count"] == rec["expected_collectives"][mode]
        assert [b["packed_payload_sha256"] for b in it["buckets"]] == [hashlib.sha256(p.tobytes()).hexdigest()
                                                                        for p in packed]
        assert report["scratch_stable"]
    assert reports["tensor"]["iterations"][0]["packed_payload_sha256"] == \
        reports["block"]["iterations"][0]["packed_payload_sha256"]


def test_trainer_evidence_snapshot_and_runtime_record(cuda, tmp_path):
    """A training step with runtime evidence on, then a post_step snapshot:
    the JSON lists every bucket of the plan, and the snapshot holds the
    step's main grads, fp32 masters and AdamW state for every parameter."""
    announce("trainer evidence")
    tr = MiddleStageTrainer(_cfg(), runtime_evidence_dir=tmp_path / "runtime")
    gen = torch.Generator().manual_seed(9)
    x, dy = _inputs(gen)
    _, _, ok, _ = tr.train_step(x, dy)
    path = tr.record_evidence(tmp_path / "numerical", "post_step", 1, metrics={"grad_norm": 1.0})
    torch.cuda.synchronize()
    report = json.loads((tmp_path / "runtime" / "rank-00000.json").read_text())
    assert report["iterations"][0]["collective_count"] == len(tr.grad_sync.plan.global_bucket_order)
    snap = load_rank_snapshot(path)
    assert snap["phase"] == "post_step" and len(snap["records"]) == len(tr.bindings)
    by_id = {b.logical_param_id: b for b in tr.bindings}
    for r in snap["records"]:
        b = by_id[r["descriptor"]["logical_param_id"]]
        assert torch.equal(r["main_grad"], b.main_grad.cpu())
        assert torch.equal(r["parameter"], b.parameter.detach().cpu())
        assert r["optimizer_parameter"].dtype == torch.float32
        assert r["optimizer_state"]["step"].item() == 1.0
        assert set(r["optimizer_hyperparameters"]) == {"beta1", "beta2", "epsilon", "weight_decay"}


def test_post_sync_evidence_holds_the_loss_scaled_gradients(cuda, tmp_path):
    """fp16 first+last stage with loss scale 2^16 and the unscale fused into
    the sync's unpack: the post_sync snapshot records the main grads as the
    reference does before optimizer.step() -- still loss-scaled -- so each
    equals its pre_sync value times the normalization scale, and the tied
    word embedding the (scaled) sum of its two copies', bit for bit; the
    clock carries the loss scale."""
    announce("post_sync evidence under loss scaling")
    from eth_amd.loss import global_normalization_scale

    cfg = GPTConfig(hidden_size=H, num_attention_heads=HEADS, ffn_hidden_size=FFN, num_layers=2, seq_length=SEQ,
                    micro_batch_size=MB, padded_vocab_size=50304, params_dtype=torch.float16, device="cuda", seed=17)
    tr = FirstLastStageTrainer(cfg, initial_loss_scale=2.0**16)
    assert tr.optimizer.grads_unscaled_by_sync
    tr.ddp.zero_grad_buffer()
    _, lo = tr.forward_backward([3, 8])
    pre = load_rank_snapshot(tr.record_evidence(tmp_path, "pre_sync", 1))
    ns = np.float32(global_normalization_scale(tr.nominal, lo.local_loss_weight).item())
    assert ns != 1.0
    tr.grad_sync.execute(float(ns))
    tr.tie_gradients()
    post = load_rank_snapshot(tr.record_evidence(tmp_path, "post_sync", 1))
    torch.cuda.synchronize()
    assert post["clock"]["loss_scale"] == 2.0**16
    by_ptr = {b.main_grad.data_ptr(): b.logical_param_id for b in tr.bindings}
    word = by_ptr[tr.embedding.word_embeddings.weight.main_grad.data_ptr()]
    head = by_ptr[tr.post.word_embeddings.weight.main_grad.data_ptr()]
    pre_g = {r["descriptor"]["logical_param_id"]: r["main_grad"] for r in pre["records"]}
    nst = torch.tensor(ns)
    for r in post["records"]:
        lid = r["descriptor"]["logical_param_id"]
        if lid in (word, head):
            expect = pre_g[word] * nst + pre_g[head] * nst
        else:
            expect = pre_g[lid] * nst
        assert torch.equal(r["main_grad"], expect), lid
    # the trainer's own main grads stay unscaled for the step
    g = tr.embedding.position_embeddings.weight.main_grad
    assert torch.equal(g.cpu() * 2.0**16, pre_g[by_ptr[g.data_ptr()]] * nst)


def test_snapshot_after_an_overlapped_update_sees_the_updated_parameters(cuda, tmp_path):
    """With the update overlapped, a step leaves the later layers' AdamW
    launches to the next forward; a post_step snapshot taken before that
    forward issues and waits for them, so it records the parameters, fp32
    masters and AdamW moments of the in-line update bit for bit."""
    announce("snapshot after an overlapped update")
    gen = torch.Generator().manual_seed(31)
    plain = MiddleStageTrainer(_cfg(layers=3))
    over = MiddleStageTrainer(_cfg(layers=3), overlap_optimizer=True)
    _randomize(plain, gen)
    _copy_weights(plain, over)
    x, dy = _inputs(gen)
    plain.train_step(x, dy)
    over.train_step(x, dy)
    snaps = [load_rank_snapshot(tr.record_evidence(tmp_path / name, "post_step", 1))
             for name, tr in (("plain", plain), ("over", over))]
    torch.cuda.synchronize()
    assert len(snaps[0]["records"]) == len(snaps[1]["records"]) > 0
    for r0, r1 in zip(snaps[0]["records"], snaps[1]["records"]):
        assert r0["descriptor"]["logical_param_id"] == r1["descriptor"]["logical_param_id"]
        for key in ("parameter", "optimizer_parameter"):
            assert torch.equal(r0[key], r1[key]), (key, r0["descriptor"]["logical_param_id"])
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(r0["optimizer_state"][key], r1["optimizer_state"][key]), key


def test_a_sync_and_step_without_a_forward_issue_the_pending_update_first(cuda):
    """A step leaves its last layers' AdamW parts for the next forward.  If
    a gradient sync and another step follow without a forward (the sync
    resets the found-inf flag and the step rewrites the clip coefficient the
    pending parts read), the parts are issued and waited for before the
    statistics are reused: the parameters match the in-line update's."""
    announce("sync and step without a forward after an overlapped update")
    gen = torch.Generator().manual_seed(37)
    plain = MiddleStageTrainer(_cfg(layers=3))
    over = MiddleStageTrainer(_cfg(layers=3), overlap_optimizer=True)
    assert over.optimizer.eager_update_parts < len(over.optimizer._overlap[1])
    _randomize(plain, gen)
    _copy_weights(plain, over)
    x, dy = _inputs(gen)
    for tr in (plain, over):
        tr.train_step(x, dy)
    for tr in (plain, over):
        tr.grad_sync.execute(0.5)
        ok, _, _ = tr.optimizer.step()
        assert ok
    over.optimizer.join_overlapped_update()
    torch.cuda.synchronize()
    for (n1, p1), (_, p2) in zip(plain.model.named_parameters(), over.model.named_parameters()):
        assert torch.equal(p1, p2), n1


@pytest.mark.parametrize("mode", ["recompute", "microbatches"])
def test_overlapped_update_with_recompute_and_microbatches(cuda, mode):
    """The overlapped update under activation recompute (each checkpointed
    segment waits for its parameters, in the forward and again in its
    replay) and under two microbatches per step (the first microbatch's
    forward waits for every part): three steps match the in-line update of
    the same trainer bit for bit."""
    announce(f"overlapped update with {mode}")
    gen = torch.Generator().manual_seed(41)
    kw = {"recompute_ops": ([0] + [1] * 6 + [0] * 3) * 3} if mode == "recompute" else {}
    plain = MiddleStageTrainer(_cfg(layers=3), **kw)
    over = MiddleStageTrainer(_cfg(layers=3), overlap_optimizer=True, **kw)
    _randomize(plain, gen)
    _copy_weights(plain, over)
    for _ in range(3):
        if mode == "recompute":
            x, dy = _inputs(gen)
            out_p, dx_p, ok_p, n_p = plain.train_step(x, dy)
            out_o, dx_o, ok_o, n_o = over.train_step(x, dy)
            assert torch.equal(out_p, out_o) and torch.equal(dx_p, dx_o)
        else:
            mbs = [{"input_tensors": {"hidden_states": x}, "output_grads": {"hidden_states": dy}}
                   for x, dy in (_inputs(gen) for _ in range(2))]
            res_p, ok_p, n_p = plain.train_step_microbatches(mbs)
            res_o, ok_o, n_o = over.train_step_microbatches(mbs)
            for rp, ro in zip(res_p, res_o):
                assert torch.equal(rp[0]["hidden_states"], ro[0]["hidden_states"])
                assert torch.equal(rp[2]["hidden_states"], ro[2]["hidden_states"])
        assert ok_p and ok_o and n_p == n_o
    over.optimizer.join_overlapped_update()
    torch.cuda.synchronize()
    for (n1, p1), (_, p2) in zip(plain.model.named_parameters(), over.model.named_parameters()):
        assert torch.equal(p1, p2), n1


def test_update_overlapped_with_the_next_forward_is_bit_identical(cuda):
    """AdamW on a side stream, one launch per part (a layer; the first
    layer in two halves), the later parts issued by the next forward a few
    ops before their first use and every op waiting only for its own
    weights: three steps give the outputs, input gradients, norms and
    parameters of the in-line update bit for bit."""
    announce("optimizer update overlapped with the next forward")
    gen = torch.Generator().manual_seed(12)
    plain = MiddleStageTrainer(_cfg(layers=3))
    over = MiddleStageTrainer(_cfg(layers=3), overlap_optimizer=True)
    _randomize(plain, gen)
    _copy_weights(plain, over)
    steps = [_inputs(gen) for _ in range(3)]
    for x, dy in steps:
        out_p, dx_p, ok_p, n_p = plain.train_step(x, dy)
        out_o, dx_o, ok_o, n_o = over.train_step(x, dy)
        assert ok_p and ok_o and n_p == n_o
        assert torch.equal(out_p, out_o) and torch.equal(dx_p, dx_o)
    # the later layers' updates are launched by the next forward; a reader
    # of the parameters before it joins the update
    over.optimizer.join_overlapped_update()
    torch.cuda.synchronize()
    for (n1, p1), (n2, p2) in zip(plain.model.named_parameters(), over.model.named_parameters()):
        assert torch.equal(p1, p2), n1


def test_forward_waits_once_per_update_part(cuda, monkeypatch):
    """The next forward waits for each overlapped update part once, at the
    first op that reads one of its parameters (every later op of the part is
    behind that wait on the same stream), and for every part."""
    announce("forward waits once per overlapped update part")
    gen = torch.Generator().manual_seed(43)
    over = MiddleStageTrainer(_cfg(layers=3), overlap_optimizer=True)
    _randomize(over, gen)
    x, dy = _inputs(gen)
    over.train_step(x, dy)  # leaves its parts' events on the parameters
    part_events = {id(e) for e in over.optimizer.optimizer.part_events}
    assert len(part_events) == len(over.optimizer._overlap[1]) > 1
    waits = []
    wait_event = torch.cuda.Stream.wait_event

    def counting(self, event):
        if id(event) in part_events:
            waits.append(id(event))
        return wait_event(self, event)

    monkeypatch.setattr(torch.cuda.Stream, "wait_event", counting)
    over.train_step(x, dy)
    torch.cuda.synchronize()
    assert sorted(waits) == sorted(part_events)
