"""GPU parity of the Gated-DeltaNet gate transform (fd_gate_transform_fwd).

Bar: the fp32 decay g within 4 fp32 ulps of the float64 oracle (the eager fp32
expression itself is within 3), beta = bf16(sigmoid(b)) within one bf16 ulp;
against PyTorch's own eager kernels on the same GPU, the share of bit-identical
results is reported and both outputs stay within 2 ulps.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import announce, from_bits, to_bits, ulp_diff

pytestmark = pytest.mark.gpu


def _f32_ulps(got, want):
    want = np.asarray(want, np.float64)
    return np.abs(np.asarray(got, np.float64) - want) / np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)


def _unpack():
    from fastdecisions_amd.unpack_gate_transform_kernel import unpack_gate
    return unpack_gate


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_golden_fixture(oracle, golden, tag):
    d = golden("gates")
    announce(f"gate transform golden {tag}")
    dt = torch.bfloat16 if tag == "bf16" else torch.float32
    a, b = from_bits(d["a"]), from_bits(d["b"])
    a_log = torch.from_numpy(d[f"{tag}_a_log"]).to(dt).cuda()
    bias = torch.from_numpy(d[f"{tag}_dt_bias"]).to(dt).cuda()
    combined = torch.cat([a, b], dim=-1).contiguous()
    g, beta = _unpack()(combined, a_log, bias)
    torch.cuda.synchronize()
    ref_g, ref_beta = oracle.gate_transform(d["a"], d["b"], d[f"{tag}_a_log"], d[f"{tag}_dt_bias"])
    assert _f32_ulps(g.cpu().numpy(), ref_g).max() < 4
    assert _f32_ulps(g.cpu().numpy(), d[f"{tag}_g"]).max() < 4
    assert ulp_diff(to_bits(beta), d["beta"]).max() <= 1
    assert ulp_diff(to_bits(beta), oracle.f32_to_bf16(ref_beta.astype(np.float32))).max() <= 1


def test_decider_rows_vs_oracle_and_eager_on_gpu(oracle):
    """B=1, T=2048, 16 heads, bf16 parameters as in the decider (a_log = log U(1,16), dt_bias = 1)."""
    gen = torch.Generator().manual_seed(3)
    a = (torch.randn((1, 2048, 16), generator=gen) * 3).to(torch.bfloat16)
    b = (torch.randn((1, 2048, 16), generator=gen) * 3).to(torch.bfloat16)
    a_log = torch.log(torch.empty(16).uniform_(1, 16, generator=gen)).to(torch.bfloat16)
    bias = torch.ones(16, dtype=torch.bfloat16)
    announce("gate transform T=2048 H=16")
    ac, bc, lc, dc = (t.cuda() for t in (a, b, a_log, bias))
    combined = torch.cat([ac, bc], dim=-1).contiguous()
    g, beta = _unpack()(combined, lc, dc)
    eager_g = -lc.float().exp() * F.softplus(ac.float() + dc)
    eager_beta = bc.sigmoid()
    torch.cuda.synchronize()
    ref_g, ref_beta = oracle.gate_transform(to_bits(a), to_bits(b), a_log.float().numpy(), bias.float().numpy())
    gh = g.cpu().numpy()
    assert _f32_ulps(gh, ref_g).max() < 4
    assert ulp_diff(to_bits(beta), oracle.f32_to_bf16(ref_beta.astype(np.float32))).max() <= 1
    same_g = (gh == eager_g.cpu().numpy()).mean()
    same_b = (to_bits(beta) == to_bits(eager_beta)).mean()
    print(f"bit-identical to PyTorch eager: g {same_g:.5f}, beta {same_b:.5f}")
    assert _f32_ulps(gh, eager_g.cpu().numpy()).max() <= 2
    assert ulp_diff(to_bits(beta), to_bits(eager_beta)).max() <= 1


def test_separate_strided_views_and_fp32_params(oracle):
    from fastdecisions_amd.unpack_gate_transform_kernel import gate_transform
    gen = torch.Generator().manual_seed(4)
    big = (torch.randn((2, 37, 100), generator=gen) * 5).to(torch.bfloat16).cuda()
    a, b = big[..., 10:18], big[..., 50:58]   # row stride 100, 8 heads
    a_log = torch.randn(8, generator=gen).cuda()
    bias = torch.randn(8, generator=gen).cuda()
    announce("gate transform strided views")
    g, beta = gate_transform(a, b, a_log, bias)
    torch.cuda.synchronize()
    ref_g, ref_beta = oracle.gate_transform(to_bits(a), to_bits(b), a_log.cpu().numpy(), bias.cpu().numpy())
    assert g.shape == (2, 37, 8) and beta.shape == (2, 37, 8)
    assert _f32_ulps(g.cpu().numpy(), ref_g).max() < 4
    assert ulp_diff(to_bits(beta), oracle.f32_to_bf16(ref_beta.astype(np.float32))).max() <= 1


def test_wrapper_rejects_bad_inputs():
    unpack = _unpack()
    c = torch.zeros((1, 8, 32), dtype=torch.bfloat16, device="cuda")
    p = torch.zeros(16, device="cuda")
    with pytest.raises(ValueError, match="shape \\[B, T, 2H\\]"):
        unpack(torch.zeros((1, 8, 31), dtype=torch.bfloat16, device="cuda"), p, p)
    with pytest.raises(ValueError, match="CUDA BF16"):
        unpack(c.float(), p, p)
    with pytest.raises(ValueError, match="a_log must have shape"):
        unpack(c, torch.zeros(8, device="cuda"), p)
    with pytest.raises(ValueError, match="BF16 or FP32"):
        unpack(c, p.double(), p)
