"""The allocation-free embedding backward (eth_embedding_bwd_noalloc, whose
sort keys live in a static device array) against the entry point that takes
a caller workspace (eth_embedding_bwd), through the C-ABI: bit-identical on
two calls in a row, the second smaller, and a clear error past the array's
capacity."""

import pytest
import torch

from eth_amd import _native as nat
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _call(name, tok, pid, dout, dw, dp, ws=None):
    b, s = tok.shape
    args = [nat.ptr(tok), nat.ptr(pid), nat.ptr(dout), nat.ptr(dw), nat.ptr(dp)]
    if ws is not None:
        args.append(nat.ptr(ws))
    args += [b, s, dout.shape[2], dw.shape[0], dp.shape[0], nat.dtype_code(dout.dtype), nat.stream_ptr(dout.device)]
    nat.call(name, *args)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_embedding_backward_matches_the_workspace_entry_point(cuda, dtype):
    gen = torch.Generator().manual_seed(31)
    V = 50304
    for b, s, h in ((4, 2048, 256), (2, 96, 64)):  # the second call is smaller
        announce(f"noalloc embedding backward {dtype} b {b} s {s} h {h}")
        tok = torch.randint(0, 9, (b, s), generator=gen)
        tok[:, ::5] = torch.randint(0, V, (b, (s + 4) // 5), generator=gen)
        tok, pid = tok.to(cuda), torch.arange(s).expand(b, s).contiguous().to(cuda)
        dout = torch.randn(s, b, h, generator=gen).to(dtype).to(cuda)
        start = (torch.randn(V, h, generator=gen) * 0.01).to(cuda)
        ws = torch.empty(nat.value("eth_embedding_bwd_workspace", b, s) // 4, dtype=torch.float32, device=cuda)
        dw_ref, dp_ref = start.clone(), torch.zeros(s, h, device=cuda)
        _call("eth_embedding_bwd", tok, pid, dout, dw_ref, dp_ref, ws)
        dw, dp = start.clone(), torch.zeros(s, h, device=cuda)
        _call("eth_embedding_bwd_noalloc", tok, pid, dout, dw, dp)
        torch.cuda.synchronize()
        assert torch.equal(dw, dw_ref)
        assert torch.equal(dp, dp_ref)


def test_noalloc_embedding_backward_rejects_sizes_past_its_scratch(cuda):
    announce("noalloc embedding backward size limit")
    big = torch.zeros(2, 16385, dtype=torch.int64, device=cuda)
    dout = torch.zeros(16385, 2, 8, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="static scratch"):
        _call("eth_embedding_bwd_noalloc", big, big, dout, torch.zeros(4, 8, device=cuda),
              torch.zeros(4, 8, device=cuda))
