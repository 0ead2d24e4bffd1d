"""GPU parity of the Gated-DeltaNet gate transform (fd_gate_transform_fwd).

Bar: the fp32 decay g within 4 fp32 ulps of the float64 oracle (the eager fp32
expression itself is within 3), beta = bf16(sigmoid(b)) within one bf16 ulp;
against PyTorch's own eager kernels on the same GPU both are bit-identical
(the kernel calls the same library exp / log1p).  The fused a|b projection
(fd_gate_proj_fwd) sums in the order hipBLASLt uses for the eager 16-output
in_proj_a / in_proj_b GEMMs, so for the decider's layer a, b, g and beta equal
the eager layer's bit for bit at any token count.
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
    assert same_g == 1.0 and same_b == 1.0


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


@pytest.mark.parametrize("B,T,H,hidden,pdt", [
    (1, 2048, 16, 2048, torch.bfloat16),   # the decider's layer
    (2, 37, 8, 1024, torch.float32),       # ragged token count (tail workgroup), fp32 parameters
    (1, 100, 32, 3072, torch.bfloat16),
    (1, 50, 16, 640, torch.bfloat16),      # 5 blocks of 128: the last group of four is partial
])
def test_fused_projection_vs_float64_and_hipblaslt(oracle, B, T, H, hidden, pdt):
    """fd_gate_proj_fwd: the a|b projection against the float64 dot product, under the bound any
    fp32 summation order meets, |a - a64| <= (n - 1) 2^-24 sum|x_k w_k| + one bf16 ulp of a64,
    which hipBLASLt's bf16 GEMM (F.linear) meets too, and with > 99 % bit-exact; the transform of
    the a|b it used (returned through `ab`) at the gate-transform bar against the float64 oracle."""
    from fastdecisions_amd.unpack_gate_transform_kernel import gate_projection
    gen = torch.Generator().manual_seed(5 + T)
    x = torch.randn((B, T, hidden), generator=gen).to(torch.bfloat16)
    w = (torch.randn((2 * H, hidden), generator=gen) * 0.03).to(torch.bfloat16)
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen)).to(pdt)
    bias = torch.randn(H, generator=gen).to(pdt)
    announce(f"fused gate projection B={B} T={T} H={H} hidden={hidden}")
    xc, wc, lc, dc = (t.cuda() for t in (x, w, a_log, bias))
    ab = torch.empty((B, T, 2 * H), dtype=torch.bfloat16, device="cuda")
    g, beta = gate_projection(xc, wc, lc, dc, ab=ab)
    lin = F.linear(xc, wc)
    g2, beta2 = gate_projection(xc, wc, lc, dc)
    torch.cuda.synchronize()
    want = x.double().numpy() @ w.double().numpy().T
    scale = np.abs(x.double().numpy()) @ np.abs(w.double().numpy()).T
    bf16_ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) * 2.0 ** 16
    bound = (hidden - 1) * 2.0 ** -24 * scale + bf16_ulp
    want_bits = oracle.f32_to_bf16(want.astype(np.float32))
    exact = (to_bits(ab) == want_bits).mean()
    print(f"a|b vs float64: exact {exact:.5f}, max |err|/bound "
          f"{(np.abs(ab.float().cpu().numpy() - want) / bound).max():.3f}; "
          f"F.linear vs float64 exact {(to_bits(lin) == want_bits).mean():.5f}")
    assert (np.abs(ab.float().cpu().numpy() - want) <= bound).all() and exact > 0.99
    assert (np.abs(lin.float().cpu().numpy() - want) <= bound).all()
    ab_bits = to_bits(ab)
    ref_g, ref_beta = oracle.gate_transform(ab_bits[..., :H], ab_bits[..., H:], a_log.float().numpy(),
                                            bias.float().numpy())
    assert _f32_ulps(g.cpu().numpy(), ref_g).max() < 4
    assert ulp_diff(to_bits(beta), oracle.f32_to_bf16(ref_beta.astype(np.float32))).max() <= 1
    # the optional ab output changes nothing; the result is deterministic
    assert torch.equal(g, g2) and torch.equal(beta, beta2)


@pytest.mark.parametrize("T", [2048, 777, 5008])
def test_fused_projection_equals_the_eager_layer(T):
    """The decider's layer (16 heads, hidden 2048, bf16 parameters): a and b equal the eager
    in_proj_a / in_proj_b GEMMs (two 16-output F.linear calls) bit for bit, and so do g and beta
    the eager gate expressions (transformers Qwen3_5GatedDeltaNet)."""
    from fastdecisions_amd.unpack_gate_transform_kernel import gate_projection
    gen = torch.Generator().manual_seed(40 + T)
    H, hidden = 16, 2048
    x = torch.randn((1, T, hidden), generator=gen).to(torch.bfloat16).cuda()
    wa = (torch.randn((H, hidden), generator=gen) * 0.02).to(torch.bfloat16).cuda()
    wb = (torch.randn((H, hidden), generator=gen) * 0.02).to(torch.bfloat16).cuda()
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=gen)).to(torch.bfloat16).cuda()
    dt_bias = torch.ones(H, dtype=torch.bfloat16, device="cuda")
    announce(f"fused gate projection vs the eager layer T={T}")
    ab = torch.empty((1, T, 2 * H), dtype=torch.bfloat16, device="cuda")
    g, beta = gate_projection(x, torch.cat([wa, wb]).contiguous(), a_log, dt_bias, ab=ab)
    a, b = F.linear(x, wa), F.linear(x, wb)
    eager_beta = b.sigmoid()
    eager_g = -a_log.float().exp() * F.softplus(a.float() + dt_bias)
    torch.cuda.synchronize()
    assert torch.equal(ab[..., :H].view(torch.int16), a.view(torch.int16))
    assert torch.equal(ab[..., H:].view(torch.int16), b.view(torch.int16))
    assert torch.equal(g.view(torch.int32), eager_g.reshape(g.shape).view(torch.int32))
    assert torch.equal(beta.view(torch.int16), eager_beta.reshape(beta.shape).view(torch.int16))


def test_fused_projection_rejects_bad_inputs():
    from fastdecisions_amd import _lib
    from fastdecisions_amd.unpack_gate_transform_kernel import gate_projection
    x = torch.zeros((1, 8, 2048), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((32, 2048), dtype=torch.bfloat16, device="cuda")
    p = torch.zeros(16, device="cuda")
    with pytest.raises(ValueError, match="weight \\[2H, hidden\\]"):
        gate_projection(x, w[:, :1024], p, p)
    with pytest.raises(ValueError, match="a_log must have shape"):
        gate_projection(x, w, torch.zeros(8, device="cuda"), p)
    with pytest.raises(RuntimeError, match="heads must be"):
        gate_projection(x, torch.zeros((20, 2048), dtype=torch.bfloat16, device="cuda"),
                        torch.zeros(10, device="cuda"), torch.zeros(10, device="cuda"))
    with pytest.raises(RuntimeError, match="multiple of 128"):
        gate_projection(x[..., :1000].contiguous(), w[:, :1000].contiguous(), p, p)
