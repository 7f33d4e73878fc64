"""CPU tests of host-side optimizer and DDP logic against the reference's
known answers: the dynamic loss scaler's growth / hysteresis rule
(optimizer/grad_scaler.py:99-119) and the local-DDP main-grad contract
(model/distributed.py:69-127, tests/test_local_ddp_runtime.py:48-72)."""

import pytest
import torch

from eth_amd.model.distributed import DistributedDataParallel
from eth_amd.optimizer.grad_scaler import ConstantGradScaler, DynamicGradScaler
from tests.helpers import known_answers

KA = known_answers()


def _scaler(rec):
    return DynamicGradScaler(
        initial_scale=rec["initial_scale"],
        min_scale=rec["min_scale"],
        growth_factor=rec["growth_factor"],
        backoff_factor=rec["backoff_factor"],
        growth_interval=rec["growth_interval"],
        hysteresis=rec["hysteresis"],
        device="cpu",
    )


def test_dynamic_scaler_grows_after_the_window_and_backs_off_after_hysteresis():
    rec = KA["dynamic_loss_scale"]
    sc = _scaler(rec)
    seen = []
    for found in rec["found_inf"]:
        sc.update(found)
        seen.append(sc.host_scale)
    assert seen == rec["expected_scale"]
    # the device copy follows the host mirror; inv_scale is fp32(1/scale)
    assert sc.scale.item() == seen[-1]
    assert sc.inv_scale_value == pytest.approx(1.0 / seen[-1], rel=0)


def test_dynamic_scaler_one_overflow_does_not_back_off_with_hysteresis_2():
    rec = dict(KA["dynamic_loss_scale"], growth_interval=1000)
    sc = _scaler(rec)
    sc.update(True)
    assert sc.host_scale == rec["initial_scale"]
    sc.update(False)  # a clean step in between does not restore the hysteresis
    sc.update(True)
    assert sc.host_scale == rec["initial_scale"] / 2


def test_dynamic_scaler_state_round_trip_and_validation():
    rec = KA["dynamic_loss_scale"]
    sc = _scaler(rec)
    for found in rec["found_inf"][:5]:
        sc.update(found)
    other = _scaler(rec)
    other.load_state_dict(sc.state_dict())
    for found in rec["found_inf"][5:]:
        sc.update(found)
        other.update(found)
        assert other.host_scale == sc.host_scale
    for bad in (dict(min_scale=2 * rec["initial_scale"]), dict(growth_factor=1.0), dict(backoff_factor=1.0),
                dict(growth_interval=0), dict(hysteresis=0)):
        with pytest.raises(ValueError):
            _scaler(dict(rec, **bad))
    const = ConstantGradScaler(1024.0, device="cpu")
    const.update(True)
    assert const.host_scale == 1024.0


class _UsedAndUnused(torch.nn.Module):
    def __init__(self, used):
        super().__init__()
        self.used = torch.nn.Parameter(torch.tensor(used))
        self.unused = torch.nn.Parameter(torch.tensor([3.0]))

    def forward(self, value):
        return (self.used * value).sum()


def test_main_grad_accumulates_and_keeps_unused_zero():
    rec = KA["main_grad_accumulation"]
    module = _UsedAndUnused(rec["param"])
    ddp = DistributedDataParallel(module, accumulate_allreduce_grads_in_fp32=False, use_contiguous_buffers=False)
    assert module.used.main_grad.dtype == module.used.dtype
    for value, expected in zip(rec["inputs"], rec["expected_main_grad_after"]):
        ddp(torch.tensor(value)).backward()
        assert torch.equal(module.used.main_grad, torch.tensor(expected))
        assert torch.equal(module.unused.main_grad, torch.tensor(rec["expected_unused_main_grad"]))
        assert module.used.grad is None
    ddp.zero_grad_buffer()
    assert torch.equal(module.used.main_grad, torch.zeros(2))
    # params are carved from the end of one buffer, in parameters() order
    (buf,) = ddp.grad_buffers.values()
    assert module.unused.main_grad.data_ptr() == buf.data.data_ptr()
    assert module.used.main_grad.data_ptr() == buf.data.data_ptr() + 4


def test_deferred_zeroing_stores_the_first_gradient():
    module = _UsedAndUnused([1.0, 2.0])
    ddp = DistributedDataParallel(module, accumulate_allreduce_grads_in_fp32=True)
    (buf,) = ddp.grad_buffers.values()
    buf.data.fill_(-7.0)
    ddp.zero_grad_buffer(defer=True)
    ddp(torch.tensor([2.0, 4.0])).backward()
    ddp.settle_grad_buffer()
    assert module.used.main_grad.tolist() == [2.0, 4.0]
    assert module.unused.main_grad.tolist() == [0.0]
