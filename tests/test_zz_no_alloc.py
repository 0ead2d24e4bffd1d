"""fd_gated_delta_fwd_noalloc (static device scratch, no allocation) against fd_gated_delta_fwd.

Both run the same kernels; only the workspace differs (the library's static
scratch vs a caller-allocated buffer), so out and the final state must be
bit-identical.  Two calls in a row, the second smaller than the first (the
scratch keeps the first call's contents), then a packed varlen call.  Every
call goes through the C ABI.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


def _inputs(B, T, hk, hv, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((B, T, hk, 128), generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn((B, T, hk, 128), generator=gen).to(torch.bfloat16).cuda()
    v = torch.randn((B, T, hv, 128), generator=gen).to(torch.bfloat16).cuda()
    g = (-torch.exp(torch.empty((B, T, hv)).uniform_(-3.0, 0.5, generator=gen))).cuda()
    beta = torch.rand((B, T, hv), generator=gen).to(torch.bfloat16).cuda()
    n = B
    s0 = (0.1 * torch.randn((n, hv, 128, 128), generator=gen)).cuda()
    return q, k, v, g, beta, s0


def _run(noalloc, q, k, v, g, beta, s0, cu=None):
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    B, T, hk, _ = q.shape
    hv = v.shape[2]
    n_seqs = 0 if cu is None else cu.numel() - 1
    n_states = B if cu is None else n_seqs
    out = torch.empty((B, T, hv, 128), dtype=torch.bfloat16, device="cuda")
    final = torch.empty((n_states, hv, 128, 128), dtype=torch.float32, device="cuda")
    cu_ptr = None if cu is None else ctypes.c_void_p(cu.data_ptr())
    s0p = None if s0 is None else ctypes.c_void_p(s0.data_ptr())
    stream = _lib.stream_handle(q.device)
    common = (B, T, hk, hv, 128, 128, ctypes.c_float(128 ** -0.5), _lib.FD_DTYPE_BF16, 1, cu_ptr, n_seqs, stream)
    ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), out.data_ptr(), s0p,
            final.data_ptr())
    if noalloc:
        rc = lib.fd_gated_delta_fwd_noalloc(*ptrs, *common)
        _lib.check("fd_gated_delta_fwd_noalloc", rc)
    else:
        nbytes = lib.fd_gated_delta_workspace_bytes(B, T, hv, 128, 128, n_seqs)
        work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        rc = lib.fd_gated_delta_fwd(*ptrs, work.data_ptr(), nbytes, *common)
        _lib.check("fd_gated_delta_fwd", rc)
    torch.cuda.synchronize()
    return out, final


@pytest.mark.parametrize("case", [
    ("decider B=1 T=2048 16/16 heads", 1, 2048, 16, 16, None),
    ("smaller B=2 T=333 4/8 heads", 2, 333, 4, 8, None),
    ("packed varlen 5 requests 16 heads", 1, 1500, 16, 16, [0, 1, 300, 300, 1111, 1500]),
])
def test_noalloc_equals_the_workspace_entry_point(case):
    what, B, T, hk, hv, cu = case
    announce(f"gated delta noalloc {what}")
    q, k, v, g, beta, s0 = _inputs(B, T, hk, hv, seed=T + hv)
    cu_t = None
    if cu is not None:
        cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda")
        gen = torch.Generator().manual_seed(5)
        s0 = (0.1 * torch.randn((len(cu) - 1, hv, 128, 128), generator=gen)).cuda()
    got_o, got_s = _run(True, q, k, v, g, beta, s0, cu_t)
    want_o, want_s = _run(False, q, k, v, g, beta, s0, cu_t)
    assert torch.equal(got_o.view(torch.int16), want_o.view(torch.int16)), what
    assert torch.equal(got_s.view(torch.int32), want_s.view(torch.int32)), what
    # the same call again on the scratch the previous call left behind
    again_o, again_s = _run(True, q, k, v, g, beta, s0, cu_t)
    assert torch.equal(again_o.view(torch.int16), want_o.view(torch.int16)), what
    assert torch.equal(again_s.view(torch.int32), want_s.view(torch.int32)), what
