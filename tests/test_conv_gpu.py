"""GPU parity of the packed causal conv1d + SiLU kernel (fd_packed_conv_fwd).

Bar: bit-exact against PyTorch's own fp32 GPU path,
``silu(conv1d(x.float(), w.float(), bias.float()))`` then one bf16 cast, run per
request for varlen inputs, on every case below.  The CPU oracle is the semantic
pin: it computes the same exact tap sum but the C library's expf, so it agrees
to within one bf16 ulp, on all but a few elements per million.  The reference's
four unit tests (ref: experiments/packed_conv/check_packed_output_conv.py:48-95)
run at full size.
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


def torch_gpu_conv(x, w, bias=None, cu=None, act="silu"):
    """PyTorch's fp32 GPU conv1d (+ SiLU), one bf16 cast; each request of a varlen batch alone.
    Returns bf16 bits [B, T, C]."""
    C = x.shape[-1]
    W = w.reshape(C, -1).shape[1]

    def one(xs):
        y = F.conv1d(xs.float().transpose(1, 2), w.reshape(C, 1, W).float(),
                     None if bias is None else bias.float(), padding=W - 1, groups=C)[..., :xs.shape[1]]
        return (F.silu(y) if act == "silu" else y).transpose(1, 2).to(torch.bfloat16)

    if cu is None:
        out = one(x)
    else:
        cu = [int(c) for c in cu]
        out = torch.cat([one(x[:, a:b]) for a, b in zip(cu[:-1], cu[1:]) if b > a], dim=1)
    return to_bits(out)


def check(got, x, w, oracle, bias=None, cu=None, act="silu", key_dim=None, value_dim=None):
    """got == torch's GPU result bit for bit; within one bf16 ulp of the CPU oracle."""
    want = torch_gpu_conv(x, w, bias, cu, act)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} differ from torch"
    orc = np.concatenate(oracle.packed_conv(to_bits(x), to_bits(w), None if bias is None else to_bits(bias),
                                            key_dim=key_dim, value_dim=value_dim,
                                            cu_seqlens=None if cu is None else np.asarray(cu, np.int32),
                                            activation=act), axis=-1)
    d = ulp_diff(got, orc)
    assert d.max() <= 1 and (d != 0).sum() <= max(4, got.size // 200_000), int((d != 0).sum())
    return int((d != 0).sum())


def test_golden_fixtures(golden, oracle):
    """The CPU-torch golden vectors (tests/golden/conv.npz); small shapes, so exact everywhere."""
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


def test_torch_gpu_golden(golden):
    """tests/golden/conv_torch_gpu.npz (torch's fp32 GPU conv + SiLU at config 2, written on an
    MI355X): each fixture element, rebuilt as a 4-row window of its own channel, comes out as
    torch's bf16, without and with a bias."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    d = golden("conv_torch_gpu")
    for tag, bias in (("conv", None), ("bias", "bias_bias")):
        announce(f"conv torch-gpu golden {tag}")
        n = d[f"{tag}_x"].shape[0]
        C = -(-n // 24) * 24
        x = np.zeros((1, 4, C), np.uint16)
        x[0, :, :n] = d[f"{tag}_x"].T
        w = np.zeros((C, 4), np.uint16)
        w[:n] = d[f"{tag}_w"]
        b = None
        if bias is not None:
            b = np.zeros(C, np.uint16)
            b[:n] = d[bias]
        q, k, v = prep_qkv(from_bits(x), from_bits(w), None if b is None else from_bits(b),
                           head_k_dim=8, head_v_dim=8)
        torch.cuda.synchronize()
        got = cat_bits(q, k, v)[0, 3, :n]
        assert np.array_equal(got, d[f"{tag}_out"]), int((got != d[f"{tag}_out"]).sum())


def test_config2_full_size(oracle):
    """B=1, T=2048, C=6144, W=4, x ~ N(0,1), w ~ N(0, 0.25), bias 0, bf16:
    bit-exact against fp32 torch conv1d + SiLU on the GPU, then cast."""
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    announce("conv config2 [1,2048,6144]")
    x = seeded((1, 2048, 6144), 100).cuda()
    w = seeded((6144, 4), 101, 0.25).cuda()
    q, k, v = prep_qkv(x, w)
    torch.cuda.synchronize()
    n = check(cat_bits(q, k, v), x, w, oracle)
    print(f"config2: 0 of {x.numel()} differ from torch fp32 conv1d+SiLU; {n} differ from the CPU oracle by 1 ulp")


def test_silu_fast_path_rounds_like_torch_for_every_fp32_input():
    """The conv's SiLU uses the hardware exp2 and reciprocal wherever they round to the same bf16 as
    y / (1 + expf(-y)), PyTorch's fp32 SiLU expression, and that expression elsewhere.  fd_silu_check
    compares the two bf16 roundings on the GPU; this runs it over all 2^32 fp32 bit patterns."""
    import ctypes
    from fastdecisions_amd import _lib
    announce("conv SiLU fast path over every fp32 bit pattern")
    lib = _lib.lib()
    count = torch.zeros(1, dtype=torch.int64, device="cuda")
    # one launch over 2^32 - 1 patterns (the largest count: its grid-stride index must not wrap), then the last
    for begin, n in ((0, (1 << 32) - 1), ((1 << 32) - 1, 1)):
        _lib.check("fd_silu_check", lib.fd_silu_check(ctypes.c_uint32(begin), ctypes.c_uint32(n),
                                                      count.data_ptr(), _lib.stream_handle(count.device)))
    torch.cuda.synchronize()
    print(f"SiLU fast path: {int(count.item())} of 2^32 fp32 inputs round differently")
    assert int(count.item()) == 0


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
    check(cat_bits(q, k, v), x, w, oracle)
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
        got = cat_bits(q, k, v)
        check(got, x, w, oracle)
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
        check(cat_bits(*outputs), x, w, oracle)


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
    check(got, x, w, oracle, cu=cu)
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
    check(cat_bits(q, k, v), x, w, oracle, bias=bias, act=act, key_dim=kd, value_dim=vd)


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
