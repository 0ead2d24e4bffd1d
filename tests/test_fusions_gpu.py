"""GPU parity of the gated RMSNorm (fd_gated_rmsnorm_fwd) and the MLP's SiLU gate
(fd_silu_mul_fwd).

Bar: within one bf16 ulp of the float64 oracle (which follows the eager bf16
roundings) and of transformers' eager modules on the golden fixture, with more
than 99 % identical; on this GPU, bit-exact against the eager modules at the
decider's sizes (the gated norm sums the squares in the order PyTorch's GPU row
mean uses at width 128 and rounds the inverse root once, as torch.rsqrt does).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, from_bits, to_bits, ulp_diff

pytestmark = pytest.mark.gpu


def test_gated_silu_fast_path_rounds_like_the_exact_product_for_every_bf16_pair():
    """With a bf16 weight the gated norm's last product bf16(y2 * silu(z)) takes y2 and z as bf16
    values and uses the hardware exp2 and reciprocal wherever they round to the same bf16 as
    y2 * (z / (1 + expf(-z))), the eager expression, and that expression elsewhere.
    fd_gated_silu_check compares the two bf16 roundings on the GPU; this runs it over all 2^32
    (y2, z) pairs of bf16 bit patterns."""
    import ctypes
    from fastdecisions_amd import _lib
    announce("gated SiLU product fast path over every bf16 pair")
    lib = _lib.lib()
    count = torch.zeros(1, dtype=torch.int64, device="cuda")
    # one launch over 2^32 - 1 pairs (the largest count: its grid-stride index must not wrap), then the last
    for begin, n in ((0, (1 << 32) - 1), ((1 << 32) - 1, 1)):
        _lib.check("fd_gated_silu_check", lib.fd_gated_silu_check(
            ctypes.c_uint32(begin), ctypes.c_uint32(n), count.data_ptr(), _lib.stream_handle(count.device)))
    torch.cuda.synchronize()
    print(f"gated SiLU fast path: {int(count.item())} of 2^32 (y2, z) pairs round differently")
    assert int(count.item()) == 0


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
        assert u.max() == 0, name


@pytest.mark.parametrize("rows,i1,i2", [(2048, 4096, 2048), (37, 24, 8), (5, 64, 0)])
def test_silu_mul_split_equals_one_projection(rows, i1, i2):
    """fd_silu_mul_split_fwd on two gate|up halves gives silu_mul's bits on the joined projection
    (an empty second projection is the single-projection case)."""
    from fastdecisions_amd.gated_norm_kernel import silu_mul, silu_mul_split
    announce(f"silu_mul_split rows={rows} widths {i1}+{i2}")
    gen = torch.Generator().manual_seed(rows + i1)
    g1, u1 = (torch.randn((2, rows, i1), generator=gen) * 3).to(torch.bfloat16).cuda()
    g2, u2 = (torch.randn((2, rows, i2), generator=gen) * 3).to(torch.bfloat16).cuda()
    split = silu_mul_split(torch.cat((g1, u1), -1), torch.cat((g2, u2), -1))
    joined = silu_mul(torch.cat((g1, g2, u1, u2), -1))
    torch.cuda.synchronize()
    assert split.shape == (rows, i1 + i2)
    assert torch.equal(split.view(torch.int16), joined.view(torch.int16))


def test_split_mlp_matches_eager_mlp():
    """The installed MLP (two gate|up GEMMs + fd_silu_mul_split_fwd) against the eager Qwen3_5MLP."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from fastdecisions_amd.layer_fusions import install_mlp_fusion
    announce("split MLP 2048 tokens, hidden 2048, intermediate 6144")
    torch.manual_seed(3)
    cfg = Qwen3_5TextConfig(hidden_size=2048, intermediate_size=6144, hidden_act="silu")
    mlp = mq.Qwen3_5MLP(cfg, 6144).to(torch.bfloat16).cuda()
    with torch.no_grad():
        for p in mlp.parameters():
            p.normal_(0, 0.02)
    x = torch.randn((1, 2048, 2048), dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        eager = mlp(x)
        assert install_mlp_fusion(torch.nn.ModuleList([mlp])) == 1
        assert mlp._fd_gate_up_weight.shape == (8192, 2048) and mlp._fd_gate_up_weight2.shape == (4096, 2048)
        ours = mlp(x)
        # float64 evaluation of the same bf16 weights and input
        x64 = x.double()
        g64 = x64 @ mlp.gate_proj.weight.double().t()
        u64 = x64 @ mlp.up_proj.weight.double().t()
        ref = (g64 * torch.sigmoid(g64) * u64) @ mlp.down_proj.weight.double().t()
    torch.cuda.synchronize()
    # the GEMMs sum in another order than the eager gate and up GEMMs, so the bits differ;
    # the bar is accuracy: no worse than the eager module against float64
    e_ours, e_eager = (ours.double() - ref).abs(), (eager.double() - ref).abs()
    print(f"split MLP vs float64: max {e_ours.max().item():.3e} rms {e_ours.pow(2).mean().sqrt().item():.3e}; "
          f"eager max {e_eager.max().item():.3e} rms {e_eager.pow(2).mean().sqrt().item():.3e}")
    assert e_ours.max() <= 1.5 * e_eager.max()
    assert e_ours.pow(2).mean() <= 1.1 ** 2 * e_eager.pow(2).mean()


@pytest.mark.parametrize("width", [64, 256])
def test_gated_rmsnorm_other_widths_vs_eager_on_gpu(width):
    """Widths 64 and 256 run 8 and 32 lanes per row (the 32-lane butterfly crosses
    16-lane rows); both sum in PyTorch's order for the width, so the rows equal
    eager Qwen3_5RMSNormGated bit for bit, as at 128."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from fastdecisions_amd.gated_norm_kernel import gated_rms_norm
    gen = torch.Generator().manual_seed(40 + width)
    rows, heads = 4096, 8
    x = (torch.randn((rows, width), generator=gen) * 0.3).to(torch.bfloat16).cuda()
    zfull = torch.randn((rows // heads, heads, 2 * width), generator=gen).to(torch.bfloat16).cuda()
    z = zfull[..., :width]
    norm = mq.Qwen3_5RMSNormGated(width, eps=1e-6).cuda()
    with torch.no_grad():
        norm.weight.copy_(1 + 0.02 * torch.randn(width, generator=gen).cuda())
    norm = norm.to(torch.bfloat16)
    announce(f"gated rmsnorm width {width} vs eager")
    with torch.no_grad():
        ours, eager = gated_rms_norm(x, z, norm.weight.data, 1e-6), norm(x, z.reshape(-1, width))
    torch.cuda.synchronize()
    u = ulp_diff(to_bits(ours), to_bits(eager))
    print(f"gated norm width {width} vs eager: max ulp {u.max()}, identical {(u == 0).mean():.5f}")
    assert u.max() == 0
