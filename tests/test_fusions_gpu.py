"""GPU parity of the gated RMSNorm (fd_gated_rmsnorm_fwd) and the MLP's SiLU gate
(fd_silu_mul_fwd).

Bar: within one bf16 ulp of the float64 oracle (which follows the eager bf16
roundings) and of transformers' eager modules on the golden fixture, with more
than 99 % identical; on this GPU, where the eager norm sums in another order,
within two ulps for the gated norm and one for the SiLU gate, with more than
99.9 % identical.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, from_bits, to_bits, ulp_diff

pytestmark = pytest.mark.gpu


def test_gated_rmsnorm_golden(oracle, golden):
    from fastdecisions_amd.gated_norm_kernel import gated_rms_norm
    d = golden("fusions")
    announce("gated rmsnorm golden")
    x, z = from_bits(d["x"]), from_bits(d["z"])
    for tag, w in (("bf16", from_bits(d["w_bf16"])), ("f32", torch.from_numpy(d["w_f32"]).cuda())):
        y = to_bits(gated_rms_norm(x, z, w, 1e-6))
        ref = oracle.f32_to_bf16(oracle.gated_rmsnorm(d["x"], d["z"], d[f"w_{tag}"]).astype(np.float32))
        assert ulp_diff(y, ref).max() <= 1, tag
        u = ulp_diff(y, d[f"y_{tag}"])
        assert u.max() <= 1 and (u == 0).mean() > 0.99, tag


def test_silu_mul_golden(oracle, golden):
    from fastdecisions_amd.gated_norm_kernel import silu_mul
    d = golden("fusions")
    announce("silu_mul golden")
    y = to_bits(silu_mul(from_bits(d["gu"])))
    assert ulp_diff(y, oracle.f32_to_bf16(oracle.silu_mul(d["gu"]).astype(np.float32))).max() <= 1
    u = ulp_diff(y, d["mlp"])
    assert u.max() <= 1 and (u == 0).mean() > 0.99


def test_decider_sizes_vs_eager_on_gpu():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from fastdecisions_amd.gated_norm_kernel import gated_rms_norm, silu_mul
    gen = torch.Generator().manual_seed(31)
    x = (torch.randn((2048 * 16, 128), generator=gen) * 0.2).to(torch.bfloat16).cuda()
    zfull = (torch.randn((2048, 16, 2 * 128), generator=gen)).to(torch.bfloat16).cuda()
    z = zfull[..., :128]   # a strided [tokens, heads, 128] gate view (no copy)
    norm = mq.Qwen3_5RMSNormGated(128, eps=1e-6).cuda()
    with torch.no_grad():
        norm.weight.copy_(1 + 0.02 * torch.randn(128, generator=gen).cuda())
    norm = norm.to(torch.bfloat16)
    announce("gated rmsnorm rows=32768, silu_mul 2048x6144")
    with torch.no_grad():
        ours, eager = gated_rms_norm(x, z, norm.weight.data, 1e-6), norm(x, z.reshape(-1, 128))
        gu = (torch.randn((2048, 2 * 6144), generator=gen) * 2).to(torch.bfloat16).cuda()
        m_ours = silu_mul(gu)
        m_eager = torch.nn.functional.silu(gu[:, :6144]) * gu[:, 6144:]
    torch.cuda.synchronize()
    for name, a, b in (("gated norm", ours, eager), ("silu_mul", m_ours, m_eager)):
        u = ulp_diff(to_bits(a), to_bits(b))
        print(f"{name} vs eager on GPU: max ulp {u.max()}, identical {(u == 0).mean():.5f}")
        # the gated norm rounds three times after the reduction: a normalised value one ulp
        # apart (another fp32 summation order) can end two ulps apart
        assert u.max() <= (2 if name == "gated norm" else 1) and (u == 0).mean() > 0.999, name
