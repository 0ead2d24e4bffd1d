"""GPU parity of the attention prologue (fd_attn_prologue_fwd) and of the gated
attention store (fd_gqa_gated_fwd).

Bars: the prologue is bit-exact against the C restatement of its fp32 sequence
(oracle/fd_oracle.c), bit-exact against transformers' eager q_norm / k_norm /
apply_rotary_pos_emb on this GPU (the kernel sums the squares in the order
PyTorch's GPU row mean uses at width 128 and rounds the inverse root once, as
torch.rsqrt does), and within one bf16 ulp of the CPU-eager golden fixture,
whose reduction order differs;
the gated store is bit-exact against the eager ``out * sigmoid(gate)`` on the
kernel's own ungated output.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, from_bits, to_bits, ulp_diff

pytestmark = pytest.mark.gpu


def test_prologue_golden(oracle, golden):
    from fastdecisions_amd.attention_prologue_kernel import attention_prologue
    d = golden("prologue")
    announce("attention prologue golden")
    q, k = from_bits(d["q"]), from_bits(d["k"])
    qw, kw = from_bits(d["q_w"]), from_bits(d["k_w"])
    cos, sin = from_bits(d["cos"]), from_bits(d["sin"])
    qo, ko = attention_prologue(q, k, qw, kw, cos, sin, 1e-6)
    torch.cuda.synchronize()
    for name, got, inp, w in (("q", qo, d["q"], d["q_w"]), ("k", ko, d["k"], d["k_w"])):
        assert np.array_equal(to_bits(got), oracle.attn_prologue(inp, w, d["cos"], d["sin"])), name
        assert ulp_diff(to_bits(got), d[f"{name}_out"]).max() <= 1, name


def test_prologue_decider_shape_from_qproj_view(oracle):
    """q is the query half of the q_proj output [B, T, 16, 256] (no copy), k [B, T, 4, 128];
    bit-exact vs the oracle and vs the eager ops on this GPU."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from fastdecisions_amd.attention_prologue_kernel import attention_prologue
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, make_config
    gen = torch.Generator().manual_seed(12)
    T = 2048
    qg = (torch.randn((1, T, 16, 256), generator=gen) * 2).to(torch.bfloat16).cuda()
    kp = torch.randn((1, T, 4, 128), generator=gen).to(torch.bfloat16).cuda()
    rope = mq.Qwen3_5TextRotaryEmbedding(make_config(DECIDER_2B_SHAPED)).cuda()
    cos, sin = rope(qg, torch.arange(T, device="cuda")[None])
    qn = mq.Qwen3_5RMSNorm(128).cuda()
    kn = mq.Qwen3_5RMSNorm(128).cuda()
    with torch.no_grad():
        qn.weight.copy_(torch.randn(128, generator=gen).cuda() * 0.05)
        kn.weight.copy_(torch.randn(128, generator=gen).cuda() * 0.05)
    qn, kn = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    announce("attention prologue T=2048 16/4 heads")
    q_view = qg[..., :128]
    qo, ko = attention_prologue(q_view, kp, qn.weight.data, kn.weight.data, cos, sin, 1e-6)
    with torch.no_grad():
        qe, ke = mq.apply_rotary_pos_emb(qn(q_view).transpose(1, 2), kn(kp).transpose(1, 2), cos, sin)
    torch.cuda.synchronize()
    cb, sb = to_bits(cos), to_bits(sin)
    assert np.array_equal(to_bits(qo), oracle.attn_prologue(to_bits(q_view), to_bits(qn.weight.data), cb, sb))
    assert np.array_equal(to_bits(ko), oracle.attn_prologue(to_bits(kp), to_bits(kn.weight.data), cb, sb))
    uq = ulp_diff(to_bits(qo), to_bits(qe.transpose(1, 2)))
    uk = ulp_diff(to_bits(ko), to_bits(ke.transpose(1, 2)))
    print(f"prologue vs eager on GPU: max ulp q {uq.max()} k {uk.max()}, identical {(uq == 0).mean():.5f}")
    assert uq.max() == 0 and uk.max() == 0


@pytest.mark.parametrize("varlen", [False, True])
def test_gated_store_equals_eager_gate(varlen):
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    gen = torch.Generator().manual_seed(21)
    T = 700
    qg = torch.randn((1, T, 16, 256), generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn((1, T, 4, 128), generator=gen).to(torch.bfloat16).cuda()
    v = torch.randn((1, T, 4, 128), generator=gen).to(torch.bfloat16).cuda()
    q, gate = qg[..., :128].transpose(1, 2), qg[..., 128:].transpose(1, 2)
    kw = {}
    if varlen:
        kw = dict(cu_seqlens=torch.tensor([0, 100, 100, 450, 700], dtype=torch.int32, device="cuda"), max_seqlen=350)
    announce(f"gated GQA store varlen={varlen}")
    plain = native_gqa_attention(q, k.transpose(1, 2), v.transpose(1, 2), **kw)
    gated = native_gqa_attention(q, k.transpose(1, 2), v.transpose(1, 2), gate=gate, **kw)
    eager = plain * torch.sigmoid(gate)
    torch.cuda.synchronize()
    assert gated.stride() == plain.stride()
    assert torch.equal(gated, eager)


@pytest.mark.parametrize("rot", [16, 64, 128])
def test_prologue_other_rotary_dims(oracle, rot):
    """Rotary dims 16, 64 and 128 put a row's rotation partner 1, 4 and 8 lanes
    away (the decider's 32: 2); bit-exact vs the oracle and the eager ops."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from fastdecisions_amd.attention_prologue_kernel import attention_prologue
    gen = torch.Generator().manual_seed(60 + rot)
    T = 96
    q = torch.randn((1, T, 16, 128), generator=gen).to(torch.bfloat16).cuda()
    k = torch.randn((1, T, 4, 128), generator=gen).to(torch.bfloat16).cuda()
    cos = (torch.rand((1, T, rot), generator=gen) * 2 - 1).to(torch.bfloat16).cuda()
    sin = (torch.rand((1, T, rot), generator=gen) * 2 - 1).to(torch.bfloat16).cuda()
    qn = mq.Qwen3_5RMSNorm(128).cuda()
    kn = mq.Qwen3_5RMSNorm(128).cuda()
    with torch.no_grad():
        qn.weight.copy_(torch.randn(128, generator=gen).cuda() * 0.05)
        kn.weight.copy_(torch.randn(128, generator=gen).cuda() * 0.05)
    qn, kn = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    announce(f"attention prologue rotary dim {rot}")
    qo, ko = attention_prologue(q, k, qn.weight.data, kn.weight.data, cos, sin, 1e-6)
    with torch.no_grad():
        qe, ke = mq.apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    torch.cuda.synchronize()
    cb, sb = to_bits(cos), to_bits(sin)
    assert np.array_equal(to_bits(qo), oracle.attn_prologue(to_bits(q), to_bits(qn.weight.data), cb, sb))
    assert np.array_equal(to_bits(ko), oracle.attn_prologue(to_bits(k), to_bits(kn.weight.data), cb, sb))
    assert torch.equal(qo, qe.transpose(1, 2)) and torch.equal(ko, ke.transpose(1, 2))
