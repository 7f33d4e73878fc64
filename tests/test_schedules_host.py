"""Host logic of the 1F1B pipeline schedule (schedules.py:595-713) over
in-process stages, with small fp64 CPU stages standing in for the GPU ones:
the per-rank action order against the published 1F1B order and its
invariants, the pipeline clock's makespan and activation memory, and the
results against plain autograd through the chained stages."""

import pytest
import torch

from eth_amd import schedules as sch


def _f(order):
    return " ".join(f"{k}{i}" for k, i in order)


def test_order_is_the_published_1f1b_order():
    """p = 4, m = 8: the worker rows of the non-interleaved 1F1B figure
    (Narayanan et al., SC'21, Fig. 4 top), 0-based."""
    assert _f(sch.one_f_one_b_order(4, 0, 8)) == "F0 F1 F2 F3 B0 F4 B1 F5 B2 F6 B3 F7 B4 B5 B6 B7"
    assert _f(sch.one_f_one_b_order(4, 1, 8)) == "F0 F1 F2 B0 F3 B1 F4 B2 F5 B3 F6 B4 F7 B5 B6 B7"
    assert _f(sch.one_f_one_b_order(4, 2, 8)) == "F0 F1 B0 F2 B1 F3 B2 F4 B3 F5 B4 F6 B5 F7 B6 B7"
    assert _f(sch.one_f_one_b_order(4, 3, 8)) == "F0 B0 F1 B1 F2 B2 F3 B3 F4 B4 F5 B5 F6 B6 F7 B7"
    # fewer microbatches than warm-up slots: all forwards, then all backwards
    assert _f(sch.one_f_one_b_order(4, 0, 2)) == "F0 F1 B0 B1"
    assert _f(sch.one_f_one_b_order(4, 0, 8, forward_only=True)) == " ".join(f"F{i}" for i in range(8))
    assert sch.one_f_one_b_order(3, 1, 0) == []
    with pytest.raises(ValueError):
        sch.get_num_warmup_microbatches(2, 2, 4)


@pytest.mark.parametrize("p", [1, 2, 3, 5])
@pytest.mark.parametrize("m", [1, 2, 4, 7])
def test_order_invariants(p, m):
    for r in range(p):
        order = sch.one_f_one_b_order(p, r, m)
        assert sorted(order) == sorted([("F", i) for i in range(m)] + [("B", i) for i in range(m)])
        fwd = [i for k, i in order if k == "F"]
        bwd = [i for k, i in order if k == "B"]
        assert fwd == list(range(m)) and bwd == list(range(m))
        held = peak = 0
        for k, i in order:
            held += 1 if k == "F" else -1
            assert held >= 0
            peak = max(peak, held)
        # a rank holds at most p - r forwards' activations
        assert peak == min(p - r, m)
        warm = sch.get_num_warmup_microbatches(p, r, m)
        assert order[:warm] == [("F", i) for i in range(warm)]


class _TanhStage:
    """y = tanh(x W) (+ a side-channel `skip` tensor received from the stage
    before); optionally emits `skip` = 0.5 y for the next stage.  The same
    forward_step / backward_step contract as the GPU stage trainers."""

    def __init__(self, w, emit):
        self.w = w
        self.emit = emit

    def forward_step(self, input_tensors, input_extra_tensors=None):
        x = input_tensors["hidden_states"].detach().requires_grad_(True)
        ex = {k: v.detach().requires_grad_(True) for k, v in (input_extra_tensors or {}).items()}
        h = torch.tanh(x @ self.w)
        if "skip" in ex:
            h = h + ex["skip"]
        out_extra = {"skip": h * 0.5} if self.emit else {}
        return {"hidden_states": h}, out_extra, ({"hidden_states": x}, ex)

    def backward_step(self, outputs, output_grads, output_extra_tensors=None, output_extra_grads=None, leaves=None):
        ts, gs = [outputs["hidden_states"]], [output_grads["hidden_states"]]
        for k in sorted(output_extra_tensors or {}):
            g = (output_extra_grads or {}).get(k)
            if g is not None:
                ts.append(output_extra_tensors[k])
                gs.append(g)
        torch.autograd.backward(ts, gs)
        ins, ex = leaves
        z = lambda t: t.grad if t.grad is not None else torch.zeros_like(t)  # noqa: E731
        return {k: z(t) for k, t in ins.items()}, {k: z(t) for k, t in ex.items()}


def _stages(p, gen, d=6):
    ws = [(torch.randn(d, d, generator=gen, dtype=torch.float64) / d**0.5).requires_grad_(True) for _ in range(p)]
    return [_TanhStage(w, emit=r < p - 1 and r % 2 == 0) for r, w in enumerate(ws)], ws


def _microbatches(m, gen, d=6):
    return [{"input_tensors": {"hidden_states": torch.randn(3, d, generator=gen, dtype=torch.float64)},
             "output_grads": {"hidden_states": torch.randn(3, d, generator=gen, dtype=torch.float64)}}
            for _ in range(m)]


def _direct(ws, mbs):
    """Plain autograd through the chained stages, one microbatch at a time."""
    p = len(ws)
    outs, dxs = [], []
    for mb in mbs:
        x = mb["input_tensors"]["hidden_states"].clone().requires_grad_(True)
        h, skip = x, None
        for r, w in enumerate(ws):
            y = torch.tanh(h @ w)
            if skip is not None:
                y = y + skip
            skip = y * 0.5 if (r < p - 1 and r % 2 == 0) else None
            h = y
        torch.autograd.backward(h, mb["output_grads"]["hidden_states"])
        outs.append(h.detach())
        dxs.append(x.grad)
    return outs, dxs


@pytest.mark.parametrize("p,m", [(1, 3), (2, 4), (3, 2), (4, 8), (5, 5)])
def test_pipelined_results_equal_autograd_and_the_sequential_order(p, m):
    gen = torch.Generator().manual_seed(10 * p + m)
    stages, ws = _stages(p, gen)
    mbs = _microbatches(m, gen)
    ref_out, ref_dx = _direct(ws, mbs)
    ref_w = [w.grad.clone() for w in ws]
    runs = {}
    for schedule in ("1f1b", "sequential"):
        for w in ws:
            w.grad = None
        res, tl = sch.forward_backward_pipelining_without_interleaving(stages, mbs, schedule=schedule)
        runs[schedule] = (res, [w.grad.clone() for w in ws], tl)
    for schedule, (res, wg, tl) in runs.items():
        for i, (out, extra, in_g, extra_g) in enumerate(res):
            assert extra == {} and extra_g == {}
            assert torch.equal(out["hidden_states"], ref_out[i])
            assert torch.equal(in_g["hidden_states"], ref_dx[i])
        # each stage's weight gradient accumulates in microbatch order in
        # every schedule
        for g, r in zip(wg, ref_w):
            assert torch.equal(g, r)
    # the pipeline clock: 1F1B finishes in 2 (m + p - 1) unit ticks and holds
    # at most min(p - r, m) forwards on rank r; one microbatch at a time takes
    # 2 p m ticks and holds one
    tl = runs["1f1b"][2]
    assert tl["ticks"] == 2 * (m + p - 1)
    assert tl["peak_in_flight"] == [min(p - r, m) for r in range(p)]
    seq = runs["sequential"][2]
    assert seq["ticks"] == 2 * p * m and seq["peak_in_flight"] == [1] * p
    # every rank's events are its order, and a forward / backward never runs
    # before its input was sent in an earlier tick
    done = {}
    for tick, r, kind, i in tl["events"]:
        if kind == "F" and r > 0:
            assert done[(r - 1, "F", i)] < tick
        if kind == "B" and r < p - 1:
            assert done[(r + 1, "B", i)] < tick
        done[(r, kind, i)] = tick
    for r in range(p):
        mine = [(k, i) for _, rr, k, i in tl["events"] if rr == r]
        assert mine == sch.one_f_one_b_order(p, r, m)


def test_forward_only_runs_no_backward():
    gen = torch.Generator().manual_seed(2)
    stages, ws = _stages(3, gen)
    mbs = _microbatches(4, gen)
    ref_out, _ = _direct(ws, mbs)
    for w in ws:
        w.grad = None
    res, tl = sch.forward_backward_pipelining_without_interleaving(stages, mbs, forward_only=True)
    assert all(w.grad is None for w in ws)
    assert tl["peak_in_flight"] == [0, 0, 0] and tl["ticks"] == 4 + 3 - 1
    for (out, _e, in_g, _eg), r in zip(res, ref_out):
        assert torch.equal(out["hidden_states"], r) and in_g == {}


def test_a_schedule_that_cannot_progress_is_reported(monkeypatch):
    """A rank whose order wants a backward before the forward that feeds it
    stalls the clock: the driver raises instead of spinning."""
    gen = torch.Generator().manual_seed(3)
    stages, _ = _stages(2, gen)
    mbs = _microbatches(2, gen)

    def backwards_first(p, r, m, forward_only=False):
        order = sch.one_f_one_b_order(p, r, m)
        return order[::-1] if r == 0 else order

    monkeypatch.setitem(sch.SCHEDULES, "bad", backwards_first)
    with pytest.raises(RuntimeError, match="stalled"):
        sch.forward_backward_pipelining_without_interleaving(stages, mbs, schedule="bad")
    with pytest.raises(ValueError, match="unknown schedule"):
        sch.forward_backward_pipelining_without_interleaving(stages, mbs, schedule="interleaved")


def test_gpt_pipeline_cuts_must_cover_the_manifest_in_order():
    """build_gpt_pipeline refuses cuts that leave a gap, overlap, or do not
    run from the embedding (op 0) to the loss (op 10 L + 2) before it builds
    any stage."""
    from eth_amd.model.flex_ops import GPTConfig

    cfg = GPTConfig(hidden_size=64, num_attention_heads=2, ffn_hidden_size=256, num_layers=2, seq_length=16,
                    micro_batch_size=1, device="cpu")
    for cuts in ([(1, 23)], [(0, 11), (12, 23)], [(0, 11), (10, 23)], [(0, 11), (11, 22)], [], [(0, 0), (0, 23)]):
        with pytest.raises(ValueError, match="consecutive stages"):
            sch.build_gpt_pipeline(cfg, cuts)
