"""GPU parity of the fused conv + gate-projection launch (fd_packed_conv_gate_fwd).

The launch runs fd_packed_conv_strided_fwd's blocks and fd_gate_proj_fwd's
blocks side by side.  Bar: every output bit-identical to those two entry points
called one after the other; they are pinned on their own (the conv bit-exact to
the CPU oracle, the projection within the fp32-summation bound of float64).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


def _inputs(B, T, key_dim, value_dim, hidden, heads, param_dtype, wide, seed):
    g = torch.Generator().manual_seed(seed)
    C = 2 * key_dim + value_dim
    cols = C + 256 if wide else C  # wide: the conv input is the first C columns of a wider projection
    proj = torch.randn((B, T, cols), generator=g).to(torch.bfloat16).cuda()
    x = proj[..., :C]
    w = (0.25 * torch.randn((C, 1, 4), generator=g)).to(torch.bfloat16).cuda()
    hs = torch.randn((B, T, hidden), generator=g).to(torch.bfloat16).cuda()
    gw = (0.02 * torch.randn((2 * heads, hidden), generator=g)).to(torch.bfloat16).cuda()
    a_log = torch.log(torch.rand(heads, generator=g) * 15 + 1).to(param_dtype).cuda()
    dt_bias = (1 + 0.1 * torch.randn(heads, generator=g)).to(param_dtype).cuda()
    return x, w, hs, gw, a_log, dt_bias


CASES = [
    # B, T, key_dim, value_dim, hidden, heads, param dtype, wide input, varlen bounds
    (1, 2048, 2048, 2048, 2048, 16, torch.float32, True, None),
    (1, 2048, 2048, 2048, 2048, 16, torch.bfloat16, False, None),
    (2, 37, 1024, 1024, 1024, 8, torch.float32, False, None),
    (1, 300, 1024, 2048, 3072, 32, torch.bfloat16, True, [0, 100, 170, 300]),
    (1, 129, 512, 512, 2048, 24, torch.float32, False, [0, 1, 64, 129]),
    (1, 77, 512, 512, 896, 16, torch.bfloat16, False, None),  # hidden 7 x 128: a partial group of blocks
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}T{c[1]}H{c[5]}{'v' if c[8] else ''}" for c in CASES])
def test_bit_identical_to_separate_launches(case):
    from fastdecisions_amd.packed_conv_kernel import prep_qkv, prep_qkv_gates
    from fastdecisions_amd.unpack_gate_transform_kernel import gate_projection
    B, T, kd, vd, hidden, heads, pdt, wide, bounds = case
    announce(f"conv+gates B={B} T={T} key_dim={kd} value_dim={vd} hidden={hidden} heads={heads} {pdt} "
             f"wide={wide} varlen={bounds}")
    x, w, hs, gw, a_log, dt_bias = _inputs(B, T, kd, vd, hidden, heads, pdt, wide, seed=T + heads)
    cu = None if bounds is None else torch.tensor(bounds, dtype=torch.int32, device="cuda")
    q, k, v, decay, beta = prep_qkv_gates(x, w, hs, gw, a_log, dt_bias, key_dim=kd, value_dim=vd, cu_seqlens=cu)
    q0, k0, v0 = prep_qkv(x, w, key_dim=kd, value_dim=vd, cu_seqlens=cu)
    decay0, beta0 = gate_projection(hs, gw, a_log, dt_bias)
    torch.cuda.synchronize()
    for name, got, want in (("q", q, q0), ("k", k, k0), ("v", v, v0), ("beta", beta, beta0)):
        assert got.shape == want.shape and got.dtype == want.dtype, name
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), name
    assert decay.shape == decay0.shape
    assert torch.equal(decay.view(torch.int32), decay0.view(torch.int32))


def test_packed_conv_gates_op_matches_the_layer_path():
    from fastdecisions_amd.packed_conv import packed_conv, packed_conv_gates
    from fastdecisions_amd.combined_gates import gate_proj_op
    announce("conv+gates torch op, B=1 T=512")
    x, w, hs, gw, a_log, dt_bias = _inputs(1, 512, 2048, 2048, 2048, 16, torch.float32, True, seed=5)
    out = packed_conv_gates(x, w, hs, gw, a_log, dt_bias, None)
    ref = (*packed_conv(x, w), *gate_proj_op(hs, gw, a_log, dt_bias))
    torch.cuda.synchronize()
    for got, want in zip(out, ref):
        assert torch.equal(got, want)


def test_rejects_bad_inputs():
    from fastdecisions_amd.packed_conv_kernel import prep_qkv_gates
    x, w, hs, gw, a_log, dt_bias = _inputs(1, 64, 1024, 1024, 2048, 16, torch.float32, False, seed=1)
    with pytest.raises(ValueError, match="hidden_states must be"):
        prep_qkv_gates(x, w, hs[:, :32].clone(), gw, a_log, dt_bias)
    with pytest.raises(ValueError, match="weight \\[2H, hidden\\]"):
        prep_qkv_gates(x, w, hs, gw[:, :1024], a_log, dt_bias)
    with pytest.raises(ValueError, match="Expected weight shape"):
        prep_qkv_gates(x, w[:100], hs, gw, a_log, dt_bias)
    with pytest.raises(RuntimeError, match="heads must be"):
        prep_qkv_gates(x, w, hs, gw[:20].contiguous(), a_log[:10].contiguous(), dt_bias[:10].contiguous())
