"""GPU parity of the native GQA causal attention kernel (fd_gqa_fwd).

Bar (north_star): max abs error <= 2e-2 vs fp32 SDPA on the same bf16 inputs
(the reference's oracle, ref: experiments/native_gqa/bench_native_gqa.py:46-61);
exact identities where the mathematics fixes the answer (row 0 = V[0],
constant V); varlen equal to per-request attention.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from helpers import announce, from_bits, seeded

pytestmark = pytest.mark.gpu

ATOL = 2e-2


def sdpa_fp32(q, k, v):
    """fp32 MATH SDPA with repeated KV heads and a causal mask (q [B,Hq,T,D])."""
    group = q.shape[1] // k.shape[1]
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q.float(), k.float().repeat_interleave(group, 1),
                                              v.float().repeat_interleave(group, 1), is_causal=True)


def model_layout(B, Hq, Hkv, T, D, seed, scale=1.0):
    """Q and V as permuted views of token-major [B, T, H, D] (as the decider feeds them), K head-major."""
    q = seeded((B, T, Hq, D), seed, scale).cuda().permute(0, 2, 1, 3)
    k = seeded((B, Hkv, T, D), seed + 1, scale).cuda()
    v = seeded((B, T, Hkv, D), seed + 2, scale).cuda().permute(0, 2, 1, 3)
    return q, k, v


def test_golden_fixtures(golden, oracle):
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    d = golden("gqa")
    announce("gqa golden bf16 B=2 Hq=4 Hkv=2 T=70 D=128")
    o = native_gqa_attention(from_bits(d["bf16_q"]), from_bits(d["bf16_k"]), from_bits(d["bf16_v"]))
    torch.cuda.synchronize()
    assert (o.float().cpu().numpy() - d["bf16_o"]).__abs__().max() <= ATOL
    announce("gqa golden varlen")
    cu = torch.from_numpy(d["var_cu"]).cuda()
    o = native_gqa_attention(from_bits(d["var_q"]), from_bits(d["var_k"]), from_bits(d["var_v"]),
                             cu_seqlens=cu, max_seqlen=int(np.diff(d["var_cu"]).max()))
    torch.cuda.synchronize()
    assert np.abs(o.float().cpu().numpy() - d["var_o"]).max() <= ATOL
    announce("gqa golden fp32 recipe (inputs cast to bf16)")
    f = lambda a: torch.from_numpy(a).to(torch.bfloat16).cuda()
    qb, kb, vb = f(d["f32_q"]), f(d["f32_k"]), f(d["f32_v"])
    o = native_gqa_attention(qb, kb, vb)
    want = oracle.gqa_attention(qb.float().cpu().numpy(), kb.float().cpu().numpy(), vb.float().cpu().numpy())
    assert np.abs(o.float().cpu().numpy() - want).max() <= ATOL


def config1_inputs():
    """q [1,16,1024,128], k and v [1,4,1024,128], fp32 N(0,1)/sqrt(128) drawn in the
    order q, k, v from one generator seeded 0 (as oracle/reference_cpu.py:gqa_config1 times it)."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 16, 1024, 128), generator=g) / 128 ** 0.5
    k = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5
    v = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5
    return q, k, v


def test_config1_recipe_through_the_kernel(oracle):
    """BASELINE config 1's exact inputs, cast to bf16, through native_gqa_attention: within 2e-2 of fp32
    MATH SDPA on the bf16 inputs and of the fp64 oracle; and within the bf16 input-rounding error of
    the fp32 reference path itself (SDPA on the fp32 inputs, the CPU baseline's computation)."""
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce("gqa config1 B=1 T=1024 16/4x128 seed 0")
    q32, k32, v32 = config1_inputs()
    q, k, v = (t.to(torch.bfloat16).cuda() for t in (q32, k32, v32))
    o = native_gqa_attention(q, k, v)
    torch.cuda.synchronize()
    err_sdpa = (o.float() - sdpa_fp32(q, k, v)).abs().max().item()
    want = oracle.gqa_attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy())
    err_oracle = float(np.abs(o.float().cpu().numpy() - want).max())
    ref32 = sdpa_fp32(q32.cuda(), k32.cuda(), v32.cuda())
    err_fp32_path = (o.float() - ref32).abs().max().item()
    print(f"gqa config1: max abs err vs fp32 SDPA (bf16 inputs) {err_sdpa:.3e}, vs fp64 oracle {err_oracle:.3e}, "
          f"vs the fp32-input reference {err_fp32_path:.3e}")
    assert err_sdpa <= ATOL and err_oracle <= ATOL and err_fp32_path <= ATOL


@pytest.mark.parametrize("recipe", ["config1_scaled", "reference_bench_unscaled"])
def test_decider_shape_T2048(recipe, oracle):
    """B=1, T=2048, 16 q / 4 kv heads, D=128 bf16 (the BASELINE GQA kernel config)."""
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    scale = 128 ** -0.5 if recipe == "config1_scaled" else 1.0
    announce(f"gqa decider shape {recipe}")
    q, k, v = model_layout(1, 16, 4, 2048, 128, 700, scale)
    o = native_gqa_attention(q, k, v)
    ref = sdpa_fp32(q, k, v)
    torch.cuda.synchronize()
    assert o.shape == (1, 16, 2048, 128) and o.stride() == (2048 * 16 * 128, 128, 16 * 128, 1)
    err = (o.float() - ref).abs().max().item()
    print(f"gqa {recipe}: max abs err vs fp32 SDPA = {err:.3e}")
    assert err <= ATOL
    # fp64 oracle on two heads (first and last of different KV groups)
    for h in (0, 15):
        want = oracle.gqa_attention(q[:, h:h + 1].float().cpu().numpy(), k[:, h // 4:h // 4 + 1].float().cpu().numpy(),
                                    v[:, h // 4:h // 4 + 1].float().cpu().numpy())
        assert np.abs(o[:, h:h + 1].float().cpu().numpy() - want).max() <= ATOL


@pytest.mark.parametrize("B,Hq,Hkv,T,D", [
    (1, 8, 2, 2048, 256),   # real decider-2b attention shape
    (4, 16, 4, 2048, 128),  # more than two work items per CU
    (2, 8, 2, 333, 256),
    (2, 16, 4, 1000, 128),
    (1, 4, 4, 257, 128),    # MHA (group 1)
    (3, 6, 3, 129, 64),     # group 2
    (1, 16, 2, 190, 64),    # group 8
    (1, 4, 1, 1, 128),      # single token
    (2, 12, 4, 95, 128),    # group 3
])
def test_shapes_groups_and_head_dims(B, Hq, Hkv, T, D):
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce(f"gqa B={B} Hq={Hq} Hkv={Hkv} T={T} D={D}")
    q, k, v = model_layout(B, Hq, Hkv, T, D, 800 + T + D)
    o = native_gqa_attention(q, k, v)
    ref = sdpa_fp32(q, k, v)
    torch.cuda.synchronize()
    err = (o.float() - ref).abs().max().item()
    assert err <= ATOL, err


def test_exact_identities():
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce("gqa identities")
    q, k, v = model_layout(1, 16, 4, 300, 128, 900)
    o = native_gqa_attention(q, k, v)
    torch.cuda.synchronize()
    # query 0 sees key 0 only: output row 0 is V[0] exactly
    assert torch.equal(o[:, :, 0], v[:, torch.arange(16, device="cuda") // 4, 0])
    # constant V gives that constant, up to the bf16 rounding of P in the P·V product
    # (the denominator sums the unrounded P, as ref: src/decider/native_gqa_kernel.py:98-103)
    vc = torch.full_like(v, 0.6875)
    oc = native_gqa_attention(q, k, vc)
    torch.cuda.synchronize()
    assert (oc.float() - 0.6875).abs().max().item() <= 0.6875 * 2.0 ** -7
    # permuting query heads within KV groups permutes the output heads
    perm = torch.tensor([3, 1, 2, 0, 4, 5, 6, 7, 11, 10, 9, 8, 12, 14, 13, 15], device="cuda")
    op = native_gqa_attention(q[:, perm], k, v)
    torch.cuda.synchronize()
    assert torch.equal(op, o[:, perm])


def test_gate_sigmoid_is_exact_for_every_bf16_value():
    """The gated store's bf16(sigmoid(gate)) equals torch's bf16 sigmoid bit for bit for each of
    the 65536 bf16 gate values.  K = 0 makes every score equal and V = 1 every output row exactly
    1.0 (the P·V sum and the denominator both count the visible keys), so the gated output is the
    rounded sigmoid itself."""
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce("gqa gate sigmoid over every bf16 value")
    T, Hq, Hkv, D = 512, 16, 4, 128
    bits = torch.arange(T * Hq * D, dtype=torch.int64) % 65536  # every bf16 pattern, 16 times
    bits = torch.where(bits >= 32768, bits - 65536, bits).to(torch.int16)
    gate = bits.view(torch.bfloat16).reshape(1, T, Hq, D).cuda().transpose(1, 2)
    q = seeded((1, T, Hq, D), 1300).cuda().transpose(1, 2)
    k = torch.zeros((1, Hkv, T, D), dtype=torch.bfloat16, device="cuda")
    v = torch.ones((1, T, Hkv, D), dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    plain = native_gqa_attention(q, k, v)
    gated = native_gqa_attention(q, k, v, gate=gate)
    expect = torch.sigmoid(gate)
    torch.cuda.synchronize()
    assert torch.equal(plain, torch.ones_like(plain))
    gated, expect = gated.contiguous(), expect.contiguous()
    nan = torch.isnan(expect)
    assert torch.equal(torch.isnan(gated), nan)
    differ = (gated.view(torch.int16) != expect.view(torch.int16)) & ~nan
    print(f"gate sigmoid: {int(differ.sum())} of {differ.numel()} outputs differ from torch.sigmoid")
    assert not differ.any()


def test_varlen_equals_per_request():
    """BASELINE config 5 style: 4 requests, lengths log-uniform in [256, 8192], packed with cu_seqlens."""
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    rng = np.random.default_rng(11)
    lengths = [int(round(np.exp(rng.uniform(np.log(256), np.log(8192))))) for _ in range(4)]
    lengths = lengths[:2] + [0, 5] + lengths[2:]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    T = int(cu[-1])
    announce(f"gqa varlen lengths={lengths} T={T}")
    q, k, v = model_layout(1, 16, 4, T, 128, 1000)
    o = native_gqa_attention(q, k, v, cu_seqlens=torch.from_numpy(cu).cuda(), max_seqlen=max(lengths))
    torch.cuda.synchronize()
    for a, b in zip(cu[:-1], cu[1:]):
        if b == a:
            continue
        alone = native_gqa_attention(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b])  # default launch, no switches
        ref = sdpa_fp32(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b])
        torch.cuda.synchronize()
        assert torch.equal(o[:, :, a:b], alone)  # head_dim 128: the same loop alone and packed
        assert (o[:, :, a:b].float() - ref).abs().max().item() <= ATOL


@pytest.mark.parametrize("Hq,Hkv,T,D", [(16, 4, 2048, 128), (16, 4, 700, 64), (8, 2, 1024, 256)])
def test_rows_do_not_depend_on_the_batch(Hq, Hkv, T, D):
    """A request's rows are bit-identical alone (B=1) and in padded batches of 2 and 5 sequences
    (different work-item counts per CU).  head_dim 256 with the key split off (its split tiles round
    differently); head_dim 64 and 128 with the default launch, which has no switch."""
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce(f"gqa batch invariance {Hq}/{Hkv}x{D} T={T}")
    split = D != 256
    q, k, v = model_layout(5, Hq, Hkv, T, D, 1300 + D, D ** -0.5)
    alone = native_gqa_attention(q[2:3], k[2:3], v[2:3], key_split=split)
    for lo, hi in ((1, 3), (0, 5)):
        batch = native_gqa_attention(q[lo:hi], k[lo:hi], v[lo:hi], key_split=split)
        torch.cuda.synchronize()
        assert torch.equal(batch[2 - lo:3 - lo], alone), (lo, hi)


def test_graph_replay_with_changed_input():
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    announce("gqa graph replay")
    q, k, v = model_layout(1, 16, 4, 512, 128, 1100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            native_gqa_attention(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = native_gqa_attention(q, k, v)
    for seed in (1101, 1102):
        k.copy_(seeded(tuple(k.shape), seed).cuda())
        graph.replay()
        torch.cuda.synchronize()
        eager = native_gqa_attention(q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_wrapper_rejects_bad_inputs():
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    q = torch.zeros((1, 4, 16, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 2, 16, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="four-dimensional"):
        native_gqa_attention(q[0], k, k)
    with pytest.raises(ValueError, match="divisible"):
        native_gqa_attention(q[:, :3], k, k)
    with pytest.raises(ValueError, match="head dimension"):
        native_gqa_attention(q[..., :96], k[..., :96], k[..., :96])
    with pytest.raises(ValueError, match="BF16"):
        native_gqa_attention(q.float(), k.float(), k.float())
    qt = torch.zeros((1, 4, 128, 16), dtype=torch.bfloat16, device="cuda").transpose(2, 3)
    kt = torch.zeros((1, 2, 128, 16), dtype=torch.bfloat16, device="cuda").transpose(2, 3)
    with pytest.raises(ValueError, match="contiguous"):
        native_gqa_attention(qt, kt, kt)


@pytest.mark.parametrize("Hq,Hkv,T,D,gated", [(8, 2, 2048, 256, False), (8, 2, 2048, 256, True),
                                               (4, 4, 1024, 256, False),   # MHA: one head x 4 query blocks
                                               (6, 3, 600, 256, True)])    # group 2: 2 heads x 2 query blocks
def test_key_split_equals_the_unsplit_kernel(Hq, Hkv, T, D, gated, oracle):
    """head_dim 256 with fewer work items than CUs: with the workspace fd_gqa_workspace_bytes asks
    for, the long query tiles run as two halves merged by a second launch; without it every tile runs
    whole.  Both must agree to bf16 rounding (the merge order differs) and stay within the 2e-2 bar of
    fp32 SDPA.  Groups below 4 heads per KV head cover the split's several-query-blocks indexing."""
    import ctypes
    from fastdecisions_amd import _lib
    announce(f"gqa key split vs whole tiles B=1 T={T} {Hq}/{Hkv}x{D} gated={gated}")
    lib = _lib.lib()
    q, k, v = model_layout(1, Hq, Hkv, T, D, 1100 + D, D ** -0.5)
    gate = seeded((1, T, Hq, D), 1200).cuda().permute(0, 2, 1, 3) if gated else None
    nbytes = lib.fd_gqa_workspace_bytes(1, Hq, Hkv, T, D, 0, 0)
    assert nbytes > 0
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    outs = []
    for ws, wb in ((work.data_ptr(), nbytes), (None, 0)):
        o = torch.empty((1, T, Hq, D), dtype=torch.bfloat16, device="cuda").permute(0, 2, 1, 3)
        common = (1, Hq, Hkv, T, D, ctypes.c_float(D ** -0.5), None, 0, T, ws, wb,
                  _lib.stream_handle(q.device))
        if gated:
            rc = lib.fd_gqa_gated_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), gate.data_ptr(), o.data_ptr(),
                                      _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(gate),
                                      _lib.strides4(o), *common)
        else:
            rc = lib.fd_gqa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), _lib.strides4(q),
                                _lib.strides4(k), _lib.strides4(v), _lib.strides4(o), *common)
        _lib.check("fd_gqa_fwd", rc)
        torch.cuda.synchronize()
        outs.append(o.float())
    split, whole = outs
    diff = (split - whole).abs()
    ulp = (whole.abs() * 2.0 ** -7).clamp_min(2.0 ** -14)  # one bf16 ulp of the value (and a floor)
    print(f"split vs whole: max|diff| {diff.max().item():.3e}, {int((diff > 0).sum())} of {diff.numel()} differ")
    assert (diff <= ulp).all()
    if not gated:
        assert (split - sdpa_fp32(q, k, v)).abs().max().item() <= ATOL
