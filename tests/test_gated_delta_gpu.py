"""GPU parity of the chunked gated delta rule (fd_gated_delta_fwd) against the CPU oracle.

The oracle (oracle/gated_delta.py) runs in float64 and is pinned against
transformers' fp32 torch_chunk_gated_delta_rule (golden fixtures) and against
the token-by-token recurrence.  The kernel runs in fp32 with its own reduction
orders and rounds the output to bf16 once, so the bar is a bf16-level one:
every element within 2^-7 of its reference value plus 1e-3 of the largest
reference magnitude, and more than 99 % of the elements within one bf16 ulp.
The l2norm's bf16 sum can land on the other side of a rounding boundary when
its fp32 order differs, which moves a whole q/k row by one bf16 ulp of the
norm; the bound above covers such a row.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, from_bits, to_bits, ulp_diff

pytestmark = pytest.mark.gpu

REL, FLOOR = 2 ** -7, 1e-3


@pytest.fixture(scope="module")
def gd():
    from oracle import gated_delta
    return gated_delta


def _rule():
    from fastdecisions_amd.gated_delta_kernel import chunk_gated_delta_rule
    return chunk_gated_delta_rule


def _check(oracle, got_bits, ref, what):
    ref = np.asarray(ref, dtype=np.float64)
    got = oracle.bf16_to_f32(got_bits).astype(np.float64)
    err = np.abs(got - ref)
    bound = REL * np.abs(ref) + FLOOR * max(np.abs(ref).max(), 1e-30)
    ref_bits = oracle.f32_to_bf16(ref.astype(np.float32))
    within_ulp = (ulp_diff(got_bits, ref_bits) <= 1).mean()
    print(f"{what}: max|err|={err.max():.3e} max|ref|={np.abs(ref).max():.3e} <=1ulp={within_ulp:.5f}")
    assert np.isfinite(got).all()
    assert (err <= bound).all(), f"{what}: {(err > bound).sum()} elements out of bounds, worst {err.max():.3e}"
    assert within_ulp > 0.99, what


def _inputs(T, hk, hv, seed, g_lo=-3.0, g_hi=0.5, beta_f32=False, B=1):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((B, T, hk, 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((B, T, hk, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((B, T, hv, 128), generator=gen).to(torch.bfloat16)
    g = -torch.exp(torch.empty((B, T, hv)).uniform_(g_lo, g_hi, generator=gen))
    beta = torch.rand((B, T, hv), generator=gen)
    if not beta_f32:
        beta = beta.to(torch.bfloat16)
    return q, k, v, g, beta


def _np(t):
    return to_bits(t) if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("case", ["d", "s", "v"])
def test_golden_fixtures(oracle, golden, case):
    """transformers' own output (q/k already normalised, so l2norm off)."""
    d = golden("gated_delta")
    announce(f"gated delta golden case {case}")
    q, k, v = (from_bits(d[f"{case}_{n}"]) for n in ("q", "k", "v"))
    g = torch.from_numpy(d[f"{case}_g"]).cuda()
    beta = from_bits(d[f"{case}_beta"])
    kw = {}
    if case == "s":
        kw["initial_state"] = torch.from_numpy(d["s_init"]).cuda()
    if case == "v":
        kw["cu_seqlens"] = torch.from_numpy(d["v_cu"]).cuda()
    out, final = _rule()(q, k, v, g, beta, output_final_state=True, use_qk_l2norm_in_kernel=False, **kw)
    torch.cuda.synchronize()
    _check(oracle, to_bits(out), oracle.bf16_to_f32(d[f"{case}_o"]), f"golden {case}")
    if f"{case}_final" in d:
        want = d[f"{case}_final"]
        assert np.abs(final.cpu().numpy() - want).max() <= 1e-4 * max(1.0, np.abs(want).max())


def test_decider_shape_T2048(oracle, gd):
    """B=1, T=2048, 16 heads, l2norm in the kernel, decider-like decay; also vs
    transformers' torch form on the same GPU."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    q, k, v, g, beta = _inputs(2048, 16, 16, seed=7, g_lo=-1.0, g_hi=2.5)
    announce("gated delta B=1 T=2048 H=16")
    qc, kc, vc, gcu, bc = (t.cuda() for t in (q, k, v, g, beta))
    out, final = _rule()(qc, kc, vc, gcu, bc, output_final_state=True, use_qk_l2norm_in_kernel=True)
    eager, eager_final = mq.torch_chunk_gated_delta_rule(qc, kc, vc, g=gcu, beta=bc, output_final_state=True,
                                                         use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    ref, ref_final = gd.chunked(_np(q), _np(k), _np(v), g.numpy(), _np(beta))
    _check(oracle, to_bits(out), ref, "T2048 vs fp64 oracle")
    _check(oracle, to_bits(eager), ref, "transformers torch form (GPU) vs fp64 oracle")
    assert np.abs(final.cpu().numpy() - ref_final).max() < 1e-3 * max(1.0, np.abs(ref_final).max())
    diff = (out.float() - eager.float()).abs().max().item()
    print(f"max |hip - transformers GPU| = {diff:.3e}")


@pytest.mark.parametrize("T,hk,hv,beta_f32,l2", [
    (1, 1, 1, False, True), (63, 2, 2, True, True), (64, 1, 2, False, False), (65, 2, 4, False, True),
    (200, 1, 1, True, False), (333, 2, 2, False, True)])
def test_ragged_lengths_heads_and_dtypes(oracle, gd, T, hk, hv, beta_f32, l2):
    q, k, v, g, beta = _inputs(T, hk, hv, seed=T + hk + hv, beta_f32=beta_f32)
    if not l2:  # unnormalised keys make the solve harder; keep them at unit scale
        q, k = ((x.float() / 11.3).to(torch.bfloat16) for x in (q, k))
    announce(f"gated delta T={T} hk={hk} hv={hv} beta_f32={beta_f32} l2norm={l2}")
    out, _ = _rule()(*(t.cuda() for t in (q, k, v, g, beta)), use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    ref, _ = gd.chunked(_np(q), _np(k), _np(v), g.numpy(), beta.numpy() if beta_f32 else _np(beta), l2norm=l2)
    _check(oracle, to_bits(out), ref, f"T={T}")


def test_padded_batch_initial_and_final_state(oracle, gd):
    q, k, v, g, beta = _inputs(100, 2, 2, seed=31, B=3)
    s0 = torch.randn((3, 2, 128, 128), generator=torch.Generator().manual_seed(2)) * 0.1
    announce("gated delta B=3 T=100 with states")
    out, final = _rule()(*(t.cuda() for t in (q, k, v, g, beta)), initial_state=s0.cuda(), output_final_state=True,
                         use_qk_l2norm_in_kernel=True, scale=0.05)
    torch.cuda.synchronize()
    ref, ref_final = gd.chunked(_np(q), _np(k), _np(v), g.numpy(), _np(beta), scale=0.05, initial_state=s0.numpy())
    _check(oracle, to_bits(out), ref, "B=3")
    assert np.abs(final.cpu().numpy() - ref_final).max() < 1e-4 * max(1.0, np.abs(ref_final).max())


def test_varlen_requests_never_leak(oracle, gd):
    """Packed requests (one empty, one of a single token) equal each request run alone."""
    cu = [0, 1, 1, 130, 131, 300]
    q, k, v, g, beta = _inputs(300, 2, 2, seed=5)
    announce(f"gated delta varlen cu={cu}")
    cu_t = torch.tensor(cu, dtype=torch.int32).cuda()
    rule = _rule()
    out, final = rule(*(t.cuda() for t in (q, k, v, g, beta)), cu_seqlens=cu_t, output_final_state=True,
                      use_qk_l2norm_in_kernel=True)
    parts = []
    for a, b in zip(cu[:-1], cu[1:]):
        if b > a:
            o, f = rule(*(t[:, a:b].contiguous().cuda() for t in (q, k, v, g, beta)), output_final_state=True,
                        use_qk_l2norm_in_kernel=True)
            parts.append(o)
    alone = torch.cat(parts, dim=1)
    torch.cuda.synchronize()
    assert torch.equal(out, alone)  # same chunks, same arithmetic
    ref, ref_final = gd.chunked(_np(q), _np(k), _np(v), g.numpy(), _np(beta), cu_seqlens=np.array(cu))
    _check(oracle, to_bits(out), ref, "varlen")
    assert final.shape == (5, 2, 128, 128)
    assert torch.count_nonzero(final[1]) == 0  # the empty request keeps a zero state
    assert np.abs(final.cpu().numpy() - ref_final).max() < 1e-4 * max(1.0, np.abs(ref_final).max())


def test_graph_replay_with_changed_input(oracle, gd):
    q, k, v, g, beta = (t.cuda() for t in _inputs(256, 4, 4, seed=9))
    rule = _rule()
    announce("gated delta graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _ = rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True)
    for seed in (9, 10, 11):
        nq, nk, nv, ng, nb = _inputs(256, 4, 4, seed=seed)
        q.copy_(nq.cuda()); k.copy_(nk.cuda()); v.copy_(nv.cuda()); g.copy_(ng.cuda()); beta.copy_(nb.cuda())
        graph.replay()
        eager, _ = rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), seed
    ref, _ = gd.chunked(_np(nq), _np(nk), _np(nv), ng.numpy(), _np(nb))
    _check(oracle, to_bits(out), ref, "graph replay")


def test_wrapper_rejects_bad_inputs():
    rule = _rule()
    q, k, v, g, beta = (t.cuda() for t in _inputs(64, 2, 2, seed=1))
    with pytest.raises(ValueError, match="head dims"):
        rule(q[..., :64].contiguous(), k[..., :64].contiguous(), v, g, beta)
    with pytest.raises(ValueError, match="chunk_size"):
        rule(q, k, v, g, beta, chunk_size=32)
    with pytest.raises(ValueError, match="g must be"):
        rule(q, k, v, g.to(torch.bfloat16), beta)
    with pytest.raises(ValueError, match="multiple of key heads"):
        rule(q, k, v[:, :, :1].contiguous().expand(1, 64, 3, 128).contiguous(), g[..., :1].expand(1, 64, 3).contiguous(),
             beta[..., :1].expand(1, 64, 3).contiguous())
    with pytest.raises(ValueError, match="cu_seqlens requires batch size 1"):
        rule(*(torch.cat([t, t]) for t in (q, k, v, g, beta)), cu_seqlens=torch.tensor([0, 64], dtype=torch.int32,
                                                                                          device="cuda"))
    with pytest.raises(ValueError, match="initial_state"):
        rule(q, k, v, g, beta, initial_state=torch.zeros((1, 2, 128, 64), device="cuda"))


def test_norm_epilogue_equals_delta_rule_then_gated_norm():
    """fd_gated_delta_norm_fwd: the delta rule with the gated RMSNorm in one call gives the
    values of fd_gated_delta_fwd followed by fd_gated_rmsnorm_fwd, bit for bit (a ragged
    tail, grouped heads, the decider shape, packed requests with an empty one, bf16 and
    fp32 norm weights; the gate is a strided view as in the combined projection)."""
    from fastdecisions_amd.gated_norm_kernel import gated_rms_norm
    rule = _rule()
    cases = ((300, 2, 4, None, torch.bfloat16), (2048, 16, 16, None, torch.bfloat16),
             (200, 2, 2, [0, 37, 37, 150, 200], torch.float32))
    for T, hk, hv, cu, wdtype in cases:
        announce(f"gated delta + norm epilogue T={T} hk={hk} hv={hv} cu={cu} w={wdtype}")
        q, k, v, g, beta = (t.cuda() for t in _inputs(T, hk, hv, seed=21))
        gen = torch.Generator().manual_seed(5)
        zbig = torch.randn((1, T, hv * 128 + 64), generator=gen).to(torch.bfloat16).cuda()
        z = zbig[..., :hv * 128].view(1, T, hv, 128)
        w = (1.0 + 0.02 * torch.randn(128, generator=gen)).to(wdtype).cuda()
        cu_t = torch.tensor(cu, dtype=torch.int32).cuda() if cu else None
        plain, _ = rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
        ref = gated_rms_norm(plain.reshape(-1, 128), z, w, 1e-6).reshape(plain.shape)
        fused, _ = rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t, norm=(z, w, 1e-6))
        torch.cuda.synchronize()
        assert torch.equal(fused, ref), (T, hk, hv, cu)



@pytest.mark.parametrize("T,hk,hv,B", [(2048, 16, 16, 1), (1000, 16, 16, 1), (640, 4, 8, 2)])
def test_rows_do_not_depend_on_the_batch(oracle, gd, T, hk, hv, B):
    """The same sequences alone and inside a larger padded batch give the same outputs and final
    states bit for bit (same chunks, same arithmetic), with and without an initial state."""
    big = B + 6
    q, k, v, g, beta = _inputs(T, hk, hv, seed=T + hv, B=big)
    s0 = torch.randn((big, hv, 128, 128), generator=torch.Generator().manual_seed(3)) * 0.1
    rule = _rule()
    for init in (None, s0):
        announce(f"gated delta alone vs in a batch: B={B} (+{big - B}) T={T} hk={hk} hv={hv} init={init is not None}")
        args = [t.cuda() for t in (q, k, v, g, beta)]
        out_big, fin_big = rule(*args, initial_state=None if init is None else init.cuda(), output_final_state=True,
                                use_qk_l2norm_in_kernel=True)
        out, fin = rule(*(t[:B].contiguous() for t in args),
                        initial_state=None if init is None else init[:B].contiguous().cuda(), output_final_state=True,
                        use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
        assert torch.equal(out, out_big[:B])
        assert torch.equal(fin, fin_big[:B])
    ref, _ = gd.chunked(_np(q[:B]), _np(k[:B]), _np(v[:B]), g[:B].numpy(), _np(beta[:B]),
                        initial_state=s0[:B].numpy())
    _check(oracle, to_bits(out), ref, f"B={B} T={T} hv={hv}")
