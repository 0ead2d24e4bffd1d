"""GPU parity of the packed causal conv1d + SiLU kernel (fd_packed_conv_fwd).

Bar: bit-exact vs the oracle's documented fp32 sequence everywhere; against
fp32 torch ``conv1d`` + SiLU then cast the mismatch count
is reported and every mismatch is <= 1 bf16 ulp (or an absolute error below
2^-20 where the tap sum cancels to ~0).  The reference's four unit tests
(ref: experiments/packed_conv/check_packed_output_conv.py:48-95) run at full size.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import announce, from_bits, seeded, to_bits, ulp_diff

pytestmark = pytest.mark.gpu


def cat_bits(q, k, v):
    B, T = q.shape[:2]
    return np.concatenate([to_bits(t).reshape(B, T, -1) for t in (q, k, v)], axis=-1)


def torch_fp32_conv(x, w):
    C = x.shape[-1]
    W = w.reshape(C, -1).shape[1]
    y = F.conv1d(x.float().transpose(1, 2), w.reshape(C, 1, W).float(), padding=W - 1, groups=C)[..., :x.shape[1]]
    return F.silu(y).transpose(1, 2).to(torch.bfloat16)


def test_golden_fixtures(golden, oracle):
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    d = golden("conv")
    announce("conv golden batch")
    q, k, v = prep_qkv(from_bits(d["batch_x"]), from_bits(d["batch_w"]), head_k_dim=8, head_v_dim=8)
    torch.cuda.synchronize()
    assert np.array_equal(cat_bits(q, k, v), d["batch_y_fp32"])
    announce("conv golden bias")
    q, k, v = prep_qkv(from_bits(d["batch_x"]), from_bits(d["batch_w"]), from_bits(d["bias_b"]),
                       head_k_dim=8, head_v_dim=8)
    assert np.array_equal(cat_bits(q, k, v), d["bias_y_fp32"])
    announce("conv golden varlen")
    cu = torch.from_numpy(d["var_cu"]).cuda()
    q, k, v = prep_qkv(from_bits(d["var_x"]), from_bits(d["batch_w"]), cu_seqlens=cu, head_k_dim=8, head_v_dim=8)
    assert np.array_equal(cat_bits(q, k, v), d["var_y_fp32"])
    announce("conv golden decider split")
    q, k, v = prep_qkv(from_bits(d["dec_x"]), from_bits(d["dec_w"]))
    assert q.shape == (1, 8, 16, 128)
    assert np.array_equal(cat_bits(q, k, v), d["dec_y_fp32"])


def test_config2_full_size(oracle):
    """B=1, T=2048, C=6144, W=4, x ~ N(0,1), w ~ N(0, 0.25), bias 0, bf16."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce("conv config2 [1,2048,6144]")
    x = seeded((1, 2048, 6144), 100).cuda()
    w = seeded((6144, 4), 101, 0.25).cuda()
    q, k, v = prep_qkv(x, w)
    torch.cuda.synchronize()
    got = cat_bits(q, k, v)
    want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w)), axis=-1)
    assert np.array_equal(got, want)
    ref = to_bits(torch_fp32_conv(x, w))
    diff = ulp_diff(got, ref)
    tiny = np.abs(oracle.bf16_to_f32(got) - oracle.bf16_to_f32(ref)) < 2.0 ** -20
    print(f"config2: vs torch fp32 conv1d+SiLU: {int((diff != 0).sum())} of {diff.size} differ; "
          f"max {int(diff.max())} ulp")
    assert ((diff <= 1) | tiny).all()
    assert (diff != 0).mean() < 1e-4


@pytest.mark.parametrize("batch", [1, 2, 4])
@pytest.mark.parametrize("weight_shape", [(6144, 4), (6144, 1, 4)])
def test_reference_random_batches_and_weight_shapes(oracle, batch, weight_shape):
    """ref: check_packed_output_conv.py:48-57 (x = 0.5 N, w = 0.25 N), at the reference size T=2048."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce(f"conv ref random batch={batch} weight={weight_shape}")
    x = seeded((batch, 2048, 6144), 200 + batch, 0.5).cuda()
    w = seeded(weight_shape, 210 + len(weight_shape), 0.25).cuda()
    q, k, v = prep_qkv(x, w)
    torch.cuda.synchronize()
    for t in (q, k, v):
        assert t.shape == (batch, 2048, 16, 128) and t.is_contiguous() and t.dtype == torch.bfloat16
    want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w)), axis=-1)
    assert np.array_equal(cat_bits(q, k, v), want)
    # the reference's own tolerance vs its fp64 oracle
    exact = torch.from_numpy(oracle.bf16_to_f32(oracle.packed_conv_f64(to_bits(x), to_bits(w))))
    got = torch.from_numpy(oracle.bf16_to_f32(cat_bits(q, k, v)))
    torch.testing.assert_close(got, exact, rtol=0.008, atol=0.002)


def test_reference_each_tap_and_batch_boundaries(oracle):
    """ref: check_packed_output_conv.py:59-71 at full size."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    x = torch.empty((2, 2048, 6144), dtype=torch.bfloat16)
    for b in range(2):
        for region in range(3):
            x[b, :, region * 2048:(region + 1) * 2048] = (b * 3 + region + 1) / 8
    x[0, -3:, :] = 3
    x = x.cuda()
    for tap in range(4):
        announce(f"conv one-hot tap {tap}")
        w = torch.zeros((6144, 4), dtype=torch.bfloat16)
        w[:, tap] = 1
        w = w.cuda()
        q, k, v = prep_qkv(x, w)
        torch.cuda.synchronize()
        want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w)), axis=-1)
        got = cat_bits(q, k, v)
        assert np.array_equal(got, want)
        assert not (oracle.bf16_to_f32(got[1]) > 1.0).any()


def test_reference_zero_input():
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce("conv zero input")
    x = torch.zeros((1, 2048, 6144), dtype=torch.bfloat16, device="cuda")
    w = seeded((6144, 4), 300).cuda()
    for t in prep_qkv(x, w):
        assert torch.count_nonzero(t).item() == 0


def test_reference_graph_replay_with_changed_input(oracle):
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce("conv graph replay")
    x = seeded((1, 2048, 6144), 400, 0.5).cuda()
    w = seeded((6144, 4), 401, 0.25).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            prep_qkv(x, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = prep_qkv(x, w)
    for seed in (402, 403):
        x.copy_(seeded((1, 2048, 6144), seed, 0.5).cuda())
        graph.replay()
        torch.cuda.synchronize()
        want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w)), axis=-1)
        assert np.array_equal(cat_bits(*outputs), want)


def test_varlen_requests_never_leak(oracle):
    """Packed requests (BASELINE config 5 style): each output equals the request run alone."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    rng = np.random.default_rng(7)
    lengths = [int(round(np.exp(rng.uniform(np.log(256), np.log(8192))))) for _ in range(4)] + [0, 1, 2, 17]
    rng.shuffle(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    T = int(cu[-1])
    announce(f"conv varlen lengths={lengths}")
    x = seeded((1, T, 6144), 500).cuda()
    w = seeded((6144, 4), 501, 0.25).cuda()
    q, k, v = prep_qkv(x, w, cu_seqlens=torch.from_numpy(cu).cuda())
    torch.cuda.synchronize()
    got = cat_bits(q, k, v)
    want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w), cu_seqlens=cu), axis=-1)
    assert np.array_equal(got, want)
    for a, b in zip(cu[:-1], cu[1:]):
        if b > a:
            qa, ka, va = prep_qkv(x[:, a:b].contiguous(), w)
            assert np.array_equal(got[:, a:b], cat_bits(qa, ka, va))


@pytest.mark.parametrize("width", [1, 2, 3])
@pytest.mark.parametrize("act", ["silu", None])
def test_widths_bias_activation_and_ragged_T(oracle, width, act):
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce(f"conv width={width} act={act}")
    B, T, kd, vd = 3, 37, 64, 128
    C = 2 * kd + vd
    x = seeded((B, T, C), 600 + width).cuda()
    w = seeded((C, width), 610 + width, 0.3).cuda()
    bias = seeded((C,), 620 + width, 0.1).cuda()
    q, k, v = prep_qkv(x, w, bias, key_dim=kd, value_dim=vd, head_k_dim=32, head_v_dim=64, activation=act)
    torch.cuda.synchronize()
    assert q.shape == (B, T, 2, 32) and v.shape == (B, T, 2, 64)
    want = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w), to_bits(bias), key_dim=kd, value_dim=vd,
                                             activation=act), axis=-1)
    assert np.array_equal(cat_bits(q, k, v), want)


def test_wrapper_rejects_bad_inputs():
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    x = torch.zeros((1, 16, 6144), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((6144, 4), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="contiguous BF16"):
        prep_qkv(x.float(), w)
    with pytest.raises(ValueError, match="weight shape"):
        prep_qkv(x, w[:, :3].contiguous().reshape(6144, 3)[:100])
    with pytest.raises(ValueError, match="aligned"):
        prep_qkv(torch.zeros(16 * 6144 + 1, dtype=torch.bfloat16, device="cuda")[1:].view(1, 16, 6144), w)
    with pytest.raises(ValueError, match="batch size 1"):
        prep_qkv(torch.zeros((2, 16, 6144), dtype=torch.bfloat16, device="cuda"), w,
                 cu_seqlens=torch.tensor([0, 16], dtype=torch.int32, device="cuda"))


def test_strided_input_from_a_wider_projection(oracle):
    """The q|k|v columns read as a view of a wider [B, T, 8224] projection output give the
    bit-identical result of the contiguous input."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    g = torch.Generator().manual_seed(44)
    wide = torch.randn((2, 300, 8224), generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn((6144, 4), generator=g) * 0.25).to(torch.bfloat16).cuda()
    announce("conv strided input B=2 T=300 row stride 8224")
    got = prep_qkv(wide[..., :6144], w)
    want = prep_qkv(wide[..., :6144].contiguous(), w)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got, want))
