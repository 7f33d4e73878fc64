"""Host-side bookkeeping of the Megatron optimizer wrapper (no GPU launch):
a tied copy sharing its root's storage, and FusedAdamW dropping a
parameter.  The update arithmetic itself is covered by the GPU tests."""

import pytest
import torch

from eth_amd.optimizer.fused_adam import FusedAdamW
from eth_amd.optimizer.optimizer import Float16OptimizerWithFloat16Params


def _params(gen, n=3, shape=(8, 4)):
    return [torch.nn.Parameter(torch.randn(shape, generator=gen).to(torch.bfloat16)) for _ in range(n)]


def _optimizer(groups):
    return Float16OptimizerWithFloat16Params(groups, 1e-3, (0.9, 0.99), 1e-8, 0.1, 1.0, bf16=True)


def test_shared_tied_copy_drops_the_copy_from_every_table():
    gen = torch.Generator().manual_seed(3)
    root, other, copy = _params(gen)
    with torch.no_grad():
        copy.copy_(root)
    opt = _optimizer([{"params": [root, other, copy]}])
    r = opt.optimizer_parameter_for_model_parameter(root)
    c = opt.optimizer_parameter_for_model_parameter(copy)
    assert r is not c and len(opt.get_parameters()) == 3
    opt.share_tied_copy(root, copy)
    # the copy's weight is a view of the root's; its master, moments and
    # model-copy entry are gone, and it maps to the root's master and state
    assert copy.data_ptr() == root.data_ptr()
    assert [id(p) for p in opt.get_parameters()] == [id(r), id(opt.optimizer_parameter_for_model_parameter(other))]
    assert c not in opt.optimizer.state and c not in opt.optimizer._model_copies
    assert opt.optimizer_parameter_for_model_parameter(copy) is r
    assert opt.state_for_model_parameter(copy) is opt.state_for_model_parameter(root)
    assert all(p is not copy for g in opt.float16_groups for p in g)
    assert all(m is not c for g in opt.fp32_from_float16_groups for m in g)
    assert opt._shared_copies == [copy]
    # sharing again is a no-op
    opt.share_tied_copy(root, copy)
    assert opt._shared_copies == [copy] and len(opt.get_parameters()) == 2


def test_shared_tied_copy_refuses_copies_that_would_not_update_alike():
    gen = torch.Generator().manual_seed(4)
    root, copy = _params(gen, 2)
    # unequal values
    opt = _optimizer([{"params": [root, copy]}])
    with pytest.raises(ValueError, match="equal values"):
        opt.share_tied_copy(root, copy)
    # equal values, different weight decay
    with torch.no_grad():
        copy.copy_(root)
    opt = _optimizer([{"params": [root]}, {"params": [copy], "weight_decay": 0.0}])
    with pytest.raises(ValueError, match="hyper-parameters"):
        opt.share_tied_copy(root, copy)
    # different shapes
    odd = torch.nn.Parameter(torch.zeros(4, 8, dtype=torch.bfloat16))
    opt = _optimizer([{"params": [root, odd]}])
    with pytest.raises(ValueError, match="shape"):
        opt.share_tied_copy(root, odd)
    # a parameter the optimizer does not own
    stranger = torch.nn.Parameter(root.detach().clone())
    opt = _optimizer([{"params": [root]}])
    with pytest.raises(ValueError, match="not owned"):
        opt.share_tied_copy(root, stranger)


def test_fused_adamw_remove_param_leaves_group_state_copies_and_partition():
    gen = torch.Generator().manual_seed(5)
    a, b, c = (torch.nn.Parameter(torch.randn(6, generator=gen)) for _ in range(3))
    opt = FusedAdamW([{"params": [a, b]}, {"params": [c], "weight_decay": 0.0}])
    models = {p: torch.nn.Parameter(p.detach().to(torch.bfloat16)) for p in (a, b, c)}
    opt.set_model_copies(models, torch.bfloat16)
    opt.set_partition([[a], [b, c]])
    opt.remove_param(b)
    assert [len(g["params"]) for g in opt.param_groups] == [1, 1]
    assert b not in opt.state and a in opt.state and c in opt.state
    assert b not in opt._model_copies and opt._model_copies[a] is models[a]
    assert opt._partition == [[a], [c]]
    assert opt._table_key is None
