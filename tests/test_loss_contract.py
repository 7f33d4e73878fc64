"""CPU tests of the loss contract, sample ownership, synthetic batch and
training clock (eth_amd/loss.py) against the reference tests' known
answers (tests/golden/known_answers.json)."""

from types import SimpleNamespace

import pytest
import torch

from eth_amd import loss as L
from tests.helpers import known_answers

KA = known_answers()


def test_loss_contract_gives_the_global_masked_mean_gradient():
    rec = KA["loss_contract_global_mean"]
    nominal = rec["nominal_global_loss_scale"]
    leaves, outs = [], []
    for mb in rec["microbatches"]:
        x = torch.tensor(mb["losses"], requires_grad=True)
        leaves.append(x)
        outs.append(L.gpt_loss_output(x, torch.tensor(mb["mask"]), nominal_global_loss_scale=nominal))
    assert [o.local_loss_sum.item() for o in outs] == rec["expected_local_loss_sum"]
    assert [o.local_loss_weight.item() for o in outs] == rec["expected_local_loss_weight"]
    numerator, weight = L.sum_loss_outputs(outs)
    (numerator / nominal).backward()
    scale = L.global_normalization_scale(nominal, weight)
    for x, expected in zip(leaves, rec["expected_normalized_grads"]):
        assert torch.equal(x.grad * scale, torch.tensor(expected))


def test_loss_contract_rejects_bad_scales_and_sizes():
    with pytest.raises(ValueError, match="nominal_global_loss_scale"):
        L.gpt_loss_output(torch.ones(1), torch.ones(1), 0.0)
    with pytest.raises(ValueError, match="global_loss_weight"):
        L.global_normalization_scale(4.0, torch.tensor(0.0))
    with pytest.raises(ValueError, match="loss_mask"):
        L.gpt_loss_output(torch.ones(3), torch.ones(2), 1.0)
    with pytest.raises(ValueError):
        L.sum_loss_outputs([])


def test_loss_outputs_aggregate_before_dividing():
    rec = KA["loss_aggregation"]
    outs = [L.LossOutput(torch.tensor(a), torch.tensor(b), 8.0, {}) for a, b in rec["outputs"]]
    numerator, weight = L.sum_loss_outputs(outs)
    assert numerator.item() == rec["expected_numerator"]
    assert weight.item() == rec["expected_weight"]
    assert (numerator / weight).item() == rec["expected_mean"]


def test_training_clock_counts_attempts_and_successes():
    rec = KA["training_clock"]
    clock = L.TrainingClock(rec["total_gbs"], rec["global_data_cursor"], rec["successful_optimizer_steps"])
    assert [clock.after_attempt(ok) for ok in rec["attempts"]] == rec["expected_returns"]
    assert clock.global_data_cursor == rec["expected_cursor"]
    assert clock.successful_optimizer_steps == rec["expected_steps"]
    with pytest.raises(ValueError):
        L.TrainingClock(0)


def test_training_clock_restore_and_cross_rank_check():
    rec = KA["training_clock_restore"]
    assert L.restore_training_clock(SimpleNamespace(**rec["checkpoint"]), rec["iteration"]) == tuple(rec["expected"])
    assert L.restore_training_clock(SimpleNamespace(**rec["legacy_checkpoint"]), rec["iteration"]) == tuple(
        rec["expected_legacy"]
    )
    L.validate_training_clock_states([(30, 4, 0.1, 1024.0)] * 2)
    with pytest.raises(ValueError, match="training clock mismatch"):
        L.validate_training_clock_states([(30, 4, 0.1, 1024.0), (40, 4, 0.1, 1024.0)])


def test_sample_slots_known_answers_and_partition():
    rec = KA["sample_slots"]
    seqs = tuple(tuple(tuple(e) for e in s) for s in rec["mbs_sequences"])
    offsets = tuple(rec["pipeline_sample_offsets"])
    for (pid, mb, dp, rank, cursor), expected in rec["cases"]:
        assert L.local_sample_slots(pid, mb, dp, rank, seqs, offsets, cursor) == tuple(expected)
    # every sample of the first iteration is owned exactly once, and the
    # second iteration's samples are new ones
    first = [
        s
        for pid, seq in enumerate(seqs)
        for mb in range(len(seq))
        for rank in range(2)
        for s in L.local_sample_slots(pid, mb, 2, rank, seqs, offsets, 0)
    ]
    assert sorted(first) == list(range(rec["total_gbs"]))
    second = L.local_sample_slots(0, 0, 1, 0, seqs, offsets, rec["total_gbs"])
    assert set(first).isdisjoint(second)
    for bad in ((2, 0, 1, 0), (0, 2, 1, 0), (0, 0, 0, 0), (0, 0, 3, 0)):
        with pytest.raises(ValueError):
            L.local_sample_slots(*bad, seqs, offsets, 0)


def test_synthetic_batch_hand_computed_values():
    for case in KA["synthetic_gpt_batch"]["cases"]:
        tokens, mask, positions, attn = L.synthetic_gpt_batch(case["ids"], case["seq"], case["vocab"], "cpu")
        assert tokens.tolist() == case["tokens"]
        assert mask.tolist() == case["mask"]
        assert mask.dtype == torch.float32 and tokens.dtype == torch.int64
        b, s = len(case["ids"]), case["seq"]
        assert positions.tolist() == [list(range(s))] * b
        assert attn.shape == (b, 1, s, s) and attn.dtype == torch.bool
        for i in range(s):
            assert attn[0, 0, i].tolist() == [j > i for j in range(s)]
        # the stages ask for no attention mask (the causal kernels imply it)
        t2, m2, p2, none = L.synthetic_gpt_batch(case["ids"], case["seq"], case["vocab"], "cpu", attention_mask=False)
        assert none is None and torch.equal(t2, tokens) and torch.equal(m2, mask) and torch.equal(p2, positions)
