"""CPU tests that pin the oracle before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against (a) the golden fixtures produced by the
reference's PyTorch path (tests/golden/make_golden.py), (b) closed forms and
brute force in fp64, and (c) special cases — chosen so that a plausible slip
(a dropped or reordered tap, a wrong sign, eps outside the rsqrt, an unrounded
residual, a wrong KV-head mapping, a leak across requests) fails at least one
of them; the ``planted`` tests show that it does.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def concat_qkv(q, k, v):
    return np.concatenate([q, k, v], axis=-1)


# ------------------------------------------------------------------ SiLU

def test_silu_special_values(oracle):
    assert oracle.silu(0.0) == 0.0 and not np.signbit(oracle.silu(0.0))
    assert oracle.silu(100.0) == 100.0             # 1 + e^-100 == 1
    assert oracle.silu(-100.0) == 0.0 and np.signbit(oracle.silu(-100.0))  # y / (1 + inf) = -0
    assert np.isnan(oracle.silu(float("nan")))
    # against fp64 on a dense grid: within 2 fp32 ulp (expf, 1 + e and the division each
    # round once; the reference formula itself performs those three roundings)
    # (below -88.72, expf(-y) overflows to inf and the formula gives -0, as torch's does)
    assert all(oracle.silu(y) == 0.0 for y in (-88.8, -89.0, -95.0))
    ys = np.concatenate([np.linspace(-88.7, 30, 24001), np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    got = np.array([oracle.silu(float(y)) for y in ys], np.float64)
    ref = ys.astype(np.float64) / (1 + np.exp(-ys.astype(np.float64)))
    ok = np.abs(got - ref) <= 2 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + 1e-45
    assert ok.all()


# ------------------------------------------------------------------ packed conv

@pytest.mark.parametrize("case,expected", [("batch", "batch_y_fp32"), ("batch", "batch_y_fp64")])
def test_conv_matches_golden(oracle, golden, case, expected):
    d = golden("conv")
    got = concat_qkv(*oracle.packed_conv(d[f"{case}_x"], d[f"{case}_w"]))
    assert np.array_equal(got, d[expected])


def test_conv_bias_and_decider_split_match_golden(oracle, golden):
    d = golden("conv")
    got = concat_qkv(*oracle.packed_conv(d["batch_x"], d["batch_w"], d["bias_b"]))
    assert np.array_equal(got, d["bias_y_fp32"])
    q, k, v = oracle.packed_conv(d["dec_x"], d["dec_w"])
    assert q.shape == (1, 8, 2048) and v.shape == (1, 8, 2048)
    assert np.array_equal(concat_qkv(q, k, v), d["dec_y_fp32"])


def test_conv_varlen_matches_golden(oracle, golden):
    d = golden("conv")
    got = concat_qkv(*oracle.packed_conv(d["var_x"], d["batch_w"], cu_seqlens=d["var_cu"]))
    assert np.array_equal(got, d["var_y_fp32"])


def test_conv_vs_fp64_and_torch_at_decider_size(oracle):
    """Config-2 recipe (x ~ N(0,1), w ~ 0.25 N(0,1), bf16) on a T=256 slice."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn((1, 256, 6144), generator=g).to(torch.bfloat16)
    w = (torch.randn((6144, 4), generator=g) * 0.25).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    got = concat_qkv(*oracle.packed_conv(xb, wb))
    exact = oracle.packed_conv_f64(xb, wb)
    ref = F.silu(F.conv1d(x.float().transpose(1, 2), w.float()[:, None], padding=3, groups=6144)[..., :256])
    ref = ref.transpose(1, 2).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    for other in (exact, ref):
        # <= 1 bf16 ulp, except where the conv cancels to ~0 and a 1-ulp fp32 difference of
        # the tap sum is many ulps of a tiny result (then the absolute error is < 2^-20)
        diff = np.abs(got.astype(np.int32) - other.astype(np.int32))
        tiny = np.abs(oracle.bf16_to_f32(got) - oracle.bf16_to_f32(other)) < 2.0 ** -20
        assert ((diff <= 1) | tiny).all()
        assert (diff != 0).mean() < 1e-4


def test_conv_matches_torch_gpu_golden(oracle, golden):
    """tests/golden/conv_torch_gpu.npz: PyTorch's fp32 GPU conv1d + SiLU at config 2, written on the
    MI355X by tests/golden/make_golden_gpu.py.  The pre-activation is bit-exact (without and with a
    bias), including on the elements where an fp32 tap sum in any order rounds differently; the SiLU
    differs from torch's only through expf (libm vs the device's), which moves the bf16 result by at
    most one ulp on rare elements."""
    d = golden("conv_torch_gpu")
    for tag, bias in (("conv", None), ("bias", "bias_bias")):
        y = oracle.conv_taps(d[f"{tag}_x"], d[f"{tag}_w"], None if bias is None else d[bias])
        assert np.array_equal(y.view(np.uint32), d[f"{tag}_y_f32"]), tag
        assert d[f"{tag}_hard"].sum() >= 1000  # the fixture holds order-sensitive cases
        s = np.array([oracle.silu(float(v)) for v in y], np.float32)
        out = oracle.f32_to_bf16(s)
        diff = np.abs(out.astype(np.int32) - d[f"{tag}_out"].astype(np.int32))
        assert diff.max() <= 1 and (diff != 0).sum() <= 4, (tag, int((diff != 0).sum()))
        # the SiLU formula itself: y / (1 + exp(-y)) with a correctly rounded exp equals torch's
        # fp32 SiLU on all but a few percent of elements, all within two fp32 ulps
        sd = np.abs(s.view(np.int32).astype(np.int64) - d[f"{tag}_silu_f32"].view(np.int32).astype(np.int64))
        assert sd.max() <= 2 and (sd != 0).mean() < 0.1


def test_planted_conv_order_slip_fails_the_torch_gpu_golden(oracle, golden):
    """An fp32 tap sum in the reference Triton kernel's order (w3 x3 first, then w0..w2 by fma) misses
    the torch GPU pre-activation on most of the fixture's order-sensitive elements."""
    d = golden("conv_torch_gpu")
    x = oracle.bf16_to_f32(d["conv_x"])
    w = oracle.bf16_to_f32(d["conv_w"])
    acc = (w[:, 3] * x[:, 3]).astype(np.float32)
    for j in range(3):
        acc = (acc + (w[:, j] * x[:, j]).astype(np.float32)).astype(np.float32)  # products are exact
    miss = acc.view(np.uint32) != d["conv_y_f32"]
    assert miss[d["conv_hard"]].mean() > 0.3 and not miss[~d["conv_hard"]].any()


def test_conv_reference_unit_cases(oracle):
    """The reference's own conv unit cases (ref: experiments/packed_conv/check_packed_output_conv.py:59-77),
    at the decider channel count with T shortened to 16."""
    T = 16
    x = np.zeros((2, T, 6144), np.float32)
    for b in range(2):
        for region in range(3):
            x[b, :, region * 2048:(region + 1) * 2048] = (b * 3 + region + 1) / 8
    x[0, -3:, :] = 3  # must never reach batch 1
    xb = oracle.f32_to_bf16(x)
    for tap in range(4):
        w = np.zeros((6144, 4), np.float32)
        w[:, tap] = 1
        wb = oracle.f32_to_bf16(w)
        got = concat_qkv(*oracle.packed_conv(xb, wb))
        # one-hot tap `tap` copies x[t - (3 - tap)] (zero before the start), then SiLU
        lag = 3 - tap
        src = np.zeros_like(x)
        src[:, lag:] = x[:, :T - lag] if lag else x
        want = oracle._f64_to_bf16(src / (1 + np.exp(-src.astype(np.float64))))
        assert np.array_equal(got, want), tap
        assert not np.any(oracle.bf16_to_f32(got[1]) > 1.0)  # the 3s of batch 0 never leak
    zero = oracle.packed_conv(np.zeros((1, 8, 6144), np.uint16), oracle.f32_to_bf16(np.random.randn(6144, 4)))
    assert all((oracle.bf16_to_f32(t) == 0).all() for t in zero)  # +0 or -0, as count_nonzero


def test_conv_varlen_equals_per_request(oracle):
    rng = np.random.default_rng(3)
    x = oracle.f32_to_bf16(rng.standard_normal((1, 61, 24)).astype(np.float32))
    w = oracle.f32_to_bf16((0.25 * rng.standard_normal((24, 4))).astype(np.float32))
    cu = np.array([0, 1, 20, 20, 61], np.int32)
    got = concat_qkv(*oracle.packed_conv(x, w, cu_seqlens=cu))
    for a, b in zip(cu[:-1], cu[1:]):
        if b > a:
            alone = concat_qkv(*oracle.packed_conv(x[:, a:b], w))
            assert np.array_equal(got[:, a:b], alone)


def test_planted_conv_slips_fail_the_golden(oracle, golden):
    d = golden("conv")
    x, w, want = d["batch_x"], d["batch_w"], d["batch_y_fp32"]
    # reversed taps
    assert not np.array_equal(concat_qkv(*oracle.packed_conv(x, w[:, ::-1].copy())), want)
    # dropped term (tap 0 zeroed)
    w0 = w.copy()
    w0[:, 0] = 0
    assert not np.array_equal(concat_qkv(*oracle.packed_conv(x, w0)), want)
    # wrong sign inside SiLU: silu(-y) != silu(y)
    neg = oracle.f32_to_bf16(-oracle.bf16_to_f32(w))
    assert not np.array_equal(concat_qkv(*oracle.packed_conv(x, neg)), want)
    # batch boundary ignored: treat the two batches as one sequence
    joined = concat_qkv(*oracle.packed_conv(x.reshape(1, -1, x.shape[-1]), w)).reshape(want.shape)
    assert not np.array_equal(joined, want)


# ------------------------------------------------------------------ RMSNorm

@pytest.mark.parametrize("case,wkey,ykey", [("small", "small_w", "small_y"), ("wide", "wide_w_bf16", "wide_y"),
                                            ("wide", "wide_w_f32", "wide_y_f32w")])
def test_rmsnorm_matches_eager_golden(oracle, golden, case, wkey, ykey):
    d = golden("rmsnorm")
    out, res = oracle.add_rmsnorm(d[f"{case}_x"], d[f"{case}_r"], d[wkey])
    assert np.array_equal(res, d[f"{case}_h"])  # updated residual: bit-exact
    diff = np.abs(out.astype(np.int32) - d[ykey].astype(np.int32))
    assert diff.max() <= 1  # normed: <= 1 bf16 ulp of eager (observed: equal)


def test_rmsnorm_vs_fp64_closed_form(oracle):
    rng = np.random.default_rng(0)
    x = oracle.f32_to_bf16(rng.standard_normal((64, 2048)).astype(np.float32))
    r = oracle.f32_to_bf16(rng.standard_normal((64, 2048)).astype(np.float32))
    w = oracle.f32_to_bf16((0.02 * rng.standard_normal(2048)).astype(np.float32))
    out, _ = oracle.add_rmsnorm(x, r, w)
    exact = oracle.add_rmsnorm_f64(x, r, w)
    diff = np.abs(out.astype(np.int32) - exact.astype(np.int32))
    assert diff.max() <= 1 and (diff != 0).mean() < 5e-3


def test_rmsnorm_special_cases(oracle):
    rng = np.random.default_rng(1)
    x = oracle.f32_to_bf16(rng.standard_normal((8, 512)).astype(np.float32))
    zero_w = np.zeros(512, np.uint16)
    out, _ = oracle.add_rmsnorm(x, None, zero_w)  # gain 1 + 0: unit-rms rows
    y = oracle.bf16_to_f32(out).astype(np.float64)
    assert np.allclose(np.sqrt((y * y).mean(axis=1)), 1.0, atol=4e-3)
    # scale invariance: norm(4x) == norm(x) bit for bit (power-of-two scale is exact)
    x4 = oracle.f32_to_bf16(4 * oracle.bf16_to_f32(x))
    assert np.array_equal(oracle.add_rmsnorm(x4, None, zero_w, eps=0.0)[0], oracle.add_rmsnorm(x, None, zero_w, eps=0.0)[0])
    # plain-gain form (gain_offset=False) with w = 1 equals the offset form with w = 0
    one_w = oracle.f32_to_bf16(np.ones(512, np.float32))
    assert np.array_equal(oracle.add_rmsnorm(x, None, one_w, gain_offset=False)[0], out)


def test_planted_rmsnorm_slips_fail_the_golden(oracle, golden):
    d = golden("rmsnorm")
    x, r, w, want = d["wide_x"], d["wide_r"], d["wide_w_bf16"], d["wide_y"]
    # eps outside / much larger than eager's
    assert not np.array_equal(oracle.add_rmsnorm(x, r, w, eps=1.0)[0], want)
    # gain without the +1 offset
    assert not np.array_equal(oracle.add_rmsnorm(x, r, w, gain_offset=False)[0], want)
    # residual dropped
    assert not np.array_equal(oracle.add_rmsnorm(x, None, w)[0], want)


# ------------------------------------------------------------------ GQA

def test_gqa_matches_golden(oracle, golden):
    d = golden("gqa")
    o = oracle.gqa_attention(d["f32_q"], d["f32_k"], d["f32_v"])
    assert np.abs(o - d["f32_o"]).max() < 1e-6
    f = oracle.bf16_to_f32
    o = oracle.gqa_attention(f(d["bf16_q"]), f(d["bf16_k"]), f(d["bf16_v"]))
    assert np.abs(o - d["bf16_o"]).max() < 1e-5
    o = oracle.gqa_attention(f(d["var_q"]), f(d["var_k"]), f(d["var_v"]), cu_seqlens=d["var_cu"])
    assert np.abs(o - d["var_o"]).max() < 1e-5


def test_gqa_config1_vs_torch_sdpa(oracle):
    """B=1, T=1024, 16 q / 4 kv heads, D=128, fp32, N(0,1)/sqrt(128), seed 0, order q, k, v."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 16, 1024, 128), generator=g) / 128 ** 0.5
    k = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5
    v = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5
    with sdpa_kernel(SDPBackend.MATH):
        ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), is_causal=True)
    o = oracle.gqa_attention(q.numpy(), k.numpy(), v.numpy())
    assert np.abs(o - ref.numpy()).max() < 1e-5


def test_gqa_invariants(oracle):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 8, 33, 16))
    k = rng.standard_normal((1, 2, 33, 16))
    v = rng.standard_normal((1, 2, 33, 16))
    o = oracle.gqa_attention(q, k, v)
    # row 0 attends only to key 0
    assert np.allclose(o[:, :, 0], v[:, np.arange(8) // 4, 0])
    # Hkv == Hq reduces to MHA on the repeated heads
    mha = oracle.gqa_attention(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1))
    assert np.allclose(o, mha)
    # constant V gives constant output
    oc = oracle.gqa_attention(q, k, np.full_like(v, 0.75))
    assert np.allclose(oc, 0.75)
    # permuting query heads inside a group permutes the output
    perm = np.array([3, 2, 1, 0, 4, 5, 7, 6])
    assert np.allclose(oracle.gqa_attention(q[:, perm], k, v), o[:, perm])
    # brute force on a tiny case: explicit softmax per query
    s = 1 / np.sqrt(16)
    for h in (0, 5):
        for i in (0, 7, 32):
            logits = np.array([q[0, h, i] @ k[0, h // 4, j] * s for j in range(i + 1)])
            p = np.exp(logits - logits.max())
            p /= p.sum()
            assert np.allclose(o[0, h, i], p @ v[0, h // 4, :i + 1])


def test_planted_gqa_slips_fail_the_golden(oracle, golden):
    d = golden("gqa")
    q, k, v, want = d["f32_q"], d["f32_k"], d["f32_v"], d["f32_o"]
    # wrong KV-head mapping (h % Hkv instead of h // group)
    wrong = np.stack([oracle.gqa_attention(q[:, h:h + 1], k[:, h % 2:h % 2 + 1], v[:, h % 2:h % 2 + 1])[:, 0]
                      for h in range(4)], axis=1)
    assert np.abs(wrong - want).max() > 1e-2
    # missing scale
    assert np.abs(oracle.gqa_attention(q, k, v, scale=1.0) - want).max() > 1e-2
    # transposed operand (V used as K)
    assert np.abs(oracle.gqa_attention(q, v, k) - want).max() > 1e-2


# ------------------------------------------------------------------ readout

def test_readout_matches_golden(oracle, golden):
    d = golden("readout")
    choice, p = oracle.decide(d["logits"], d["nopts"])
    assert np.array_equal(choice, d["choice"])
    assert np.allclose(p.sum(axis=1), 1.0)
    assert all((p[i, n:] == 0).all() for i, n in enumerate(d["nopts"]))


# ------------------------------------------------------------------ gated delta rule

@pytest.fixture(scope="module")
def gd():
    from oracle import gated_delta
    return gated_delta


def _bf16_out(oracle, o):
    return oracle.f32_to_bf16(o.astype(np.float32))


def _close_to_bf16_golden(oracle, o, want_bits, rel=2 ** -7, floor=1e-3):
    """fp64 result vs a bf16 golden: within a bf16 rounding of fp32 work (abs bound
    scaled by the output's magnitude)."""
    want = oracle.bf16_to_f32(want_bits).astype(np.float64)
    err = np.abs(o - want)
    return bool((err <= rel * np.abs(want) + floor * np.abs(want).max()).all())


def test_gated_delta_l2norm_matches_transformers_bitexact(oracle, gd, golden):
    d = golden("gated_delta")
    assert np.array_equal(gd.l2norm_bf16(d["l2_x"]), d["l2_y"])


def test_gated_delta_l2norm_rounds_every_step_to_bf16(oracle, gd):
    """A row whose fp32 sum of squares is not a bf16 value: the sum, the rsqrt and
    the product are each rounded (transformers' l2norm on bf16 tensors)."""
    x = oracle.f32_to_bf16(np.array([[3.0, 4.0, 0.1] + [0.0] * 5], np.float32))
    y = oracle.bf16_to_f32(gd.l2norm_bf16(x))[0]
    sq = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.bf16_to_f32(x)[0] ** 2))
    s = oracle.bf16_to_f32(oracle.f32_to_bf16(np.float32(sq.sum(dtype=np.float32))))
    inv = oracle.bf16_to_f32(oracle.f32_to_bf16(np.float32(1 / np.sqrt(np.float32(s + np.float32(1e-6))))))
    assert np.array_equal(y[:3], oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.bf16_to_f32(x)[0][:3] * inv)))
    assert y[3:].tolist() == [0.0] * 5


@pytest.mark.parametrize("case", ["d", "s", "v"])
def test_gated_delta_matches_transformers_golden(oracle, gd, golden, case):
    d = golden("gated_delta")
    kw = dict(l2norm=False)
    if case == "s":
        kw["initial_state"] = d["s_init"]
    if case == "v":
        kw["cu_seqlens"] = d["v_cu"]
    o, final = gd.chunked(d[f"{case}_q"], d[f"{case}_k"], d[f"{case}_v"], d[f"{case}_g"], d[f"{case}_beta"], **kw)
    assert _close_to_bf16_golden(oracle, o, d[f"{case}_o"])
    if f"{case}_final" in d:
        want = d[f"{case}_final"]
        assert np.abs(final - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


def test_gated_delta_chunked_equals_recurrent(oracle, gd):
    """Two independent algorithms for the same recurrence: dense, ragged, varlen,
    shared key heads and an initial state."""
    rng = np.random.default_rng(11)
    T, hk, hv = 150, 1, 2
    q = oracle.f32_to_bf16(rng.standard_normal((1, T, hk, 128)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((1, T, hk, 128)).astype(np.float32))
    v = oracle.f32_to_bf16(rng.standard_normal((1, T, hv, 128)).astype(np.float32))
    g = -np.exp(rng.uniform(-3, 1, (1, T, hv))).astype(np.float32)
    beta = rng.uniform(0, 1, (1, T, hv)).astype(np.float32)
    s0 = rng.standard_normal((3, hv, 128, 128)) * 0.1
    cu = np.array([0, 65, 65, 150], np.int32)
    for kw in (dict(), dict(cu_seqlens=cu, initial_state=s0)):
        a, fa = gd.chunked(q, k, v, g, beta, **kw)
        b, fb = gd.recurrent(q, k, v, g, beta, **kw)
        assert np.abs(a - b).max() < 1e-10 and np.abs(fa - fb).max() < 1e-10


def test_gated_delta_closed_forms(oracle, gd):
    rng = np.random.default_rng(3)
    T = 70
    q = oracle.f32_to_bf16(rng.standard_normal((1, T, 1, 128)).astype(np.float32))
    k = oracle.f32_to_bf16(rng.standard_normal((1, T, 1, 128)).astype(np.float32))
    v = oracle.f32_to_bf16(rng.standard_normal((1, T, 1, 128)).astype(np.float32))
    g = -np.exp(rng.uniform(-2, 0, (1, T, 1))).astype(np.float32)
    # beta = 0: nothing is ever written, the output is zero
    o, f = gd.chunked(q, k, v, g, np.zeros((1, T, 1), np.float32))
    assert np.abs(o).max() == 0 and np.abs(f).max() == 0
    # first token: o_0 = beta_0 (scale q_0 . k_0) v_0 on the normalised q/k
    beta = rng.uniform(0.2, 1, (1, T, 1)).astype(np.float32)
    o, _ = gd.chunked(q, k, v, g, beta)
    qn = oracle.bf16_to_f32(gd.l2norm_bf16(q)).astype(np.float64)
    kn = oracle.bf16_to_f32(gd.l2norm_bf16(k)).astype(np.float64)
    vv = oracle.bf16_to_f32(v).astype(np.float64)
    scale = float(np.float32(1 / np.sqrt(128)))
    assert np.allclose(o[0, 0, 0], beta[0, 0, 0] * scale * (qn[0, 0, 0] @ kn[0, 0, 0]) * vv[0, 0, 0])
    # orthonormal keys, no decay, beta = 1: the state stores v_i under k_i exactly
    basis = np.eye(128, dtype=np.float32)[:T]
    kb = oracle.f32_to_bf16(basis[None, :, None, :])
    o, f = gd.chunked(kb, kb, v, np.zeros((1, T, 1), np.float32), np.ones((1, T, 1), np.float32), scale=1.0)
    assert np.allclose(f[0, 0][:T], vv[0, :, 0])
    assert np.allclose(o[0, :, 0], vv[0, :, 0])
    # constant decay e^g per token scales an untouched state: beta = 0 with an initial state
    s0 = rng.standard_normal((1, 1, 128, 128))
    _, f = gd.chunked(q, k, v, np.full((1, T, 1), -0.01, np.float32), np.zeros((1, T, 1), np.float32),
                      initial_state=s0)
    assert np.allclose(f, s0 * np.exp(-0.01 * T))


def test_planted_gated_delta_slips_fail_the_golden(oracle, gd, golden):
    """Slips planted in a copy of the recurrence must fail the transformers golden."""
    d = golden("gated_delta")
    q, k, v, g, beta = (d[f"d_{n}"] for n in ("q", "k", "v", "g", "beta"))
    want = d["d_o"]
    assert _close_to_bf16_golden(oracle, gd.recurrent(q, k, v, g, beta, l2norm=False)[0], want)

    def slipped(slip):
        qq, kk, vv, gg, bb = gd._prepare(q, k, v, g, beta, None, False)
        T, H = vv.shape[1], vv.shape[2]
        S = np.zeros((H, 128, 128))
        o = np.zeros(vv.shape[1:])
        for t in range(T):
            decay = np.exp(gg[0, t]) if slip != "no_decay" else np.ones(H)
            if slip != "decay_after":
                S = S * decay[:, None, None]
            mem = np.einsum("hk,hkv->hv", kk[0, t], S)
            dlt = (vv[0, t] - mem) if slip != "beta_outside" else vv[0, t] - mem * bb[0, t][:, None]
            dlt = dlt * bb[0, t][:, None] if slip != "beta_outside" else dlt
            if slip == "sign":
                dlt = vv[0, t] + mem
            S = S + kk[0, t][:, :, None] * dlt[:, None, :]
            if slip == "decay_after":
                S = S * decay[:, None, None]
            o[t] = np.einsum("hk,hkv->hv", qq[0, t], S if slip != "output_before_write" else S - kk[0, t][:, :, None] * dlt[:, None, :])
        return o[None]

    for slip in ("no_decay", "decay_after", "beta_outside", "sign", "output_before_write"):
        assert not _close_to_bf16_golden(oracle, slipped(slip), want), slip


# ------------------------------------------------------------------ gate transform

def _f32_ulps(got, want):
    want = np.asarray(want, np.float64)
    return np.abs(np.asarray(got, np.float64) - want) / np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_gate_transform_matches_eager_golden(oracle, golden, tag):
    d = golden("gates")
    g, beta = oracle.gate_transform(d["a"], d["b"], d[f"{tag}_a_log"], d[f"{tag}_dt_bias"])
    assert _f32_ulps(g, d[f"{tag}_g"]).max() < 4
    assert np.array_equal(oracle.f32_to_bf16(beta.astype(np.float32)), d["beta"])


def test_gate_transform_closed_forms(oracle):
    a = oracle.f32_to_bf16(np.array([[25.0, 0.0, -30.0]], np.float32))
    b = oracle.f32_to_bf16(np.array([[0.0, 80.0, -80.0]], np.float32))
    g, beta = oracle.gate_transform(a, b, np.zeros(3), np.zeros(3))
    # above the threshold softplus is the identity; softplus(0) = ln 2; softplus(-30) = e^-30 to 1e-13
    assert g[0, 0] == -25.0 and np.isclose(g[0, 1], -np.log(2.0)) and np.isclose(g[0, 2], -np.exp(-30.0))
    assert beta[0, 0] == 0.5 and beta[0, 1] == 1.0 and beta[0, 2] < 1e-34
    # the decay scales with exp(a_log)
    g2, _ = oracle.gate_transform(a, b, np.full(3, np.log(4.0)), np.zeros(3))
    assert np.allclose(g2, 4 * g)


def test_planted_gate_slips_fail_the_golden(oracle, golden):
    d = golden("gates")
    want = d["f32_g"]
    a_log, bias = d["f32_a_log"], d["f32_dt_bias"]
    good, _ = oracle.gate_transform(d["a"], d["b"], a_log, bias)
    assert _f32_ulps(good, want).max() < 4
    x = oracle.bf16_to_f32(d["a"]).astype(np.float64) + bias
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    for slip in (-a_log * sp,                        # log-space decay without the exp
                 -np.exp(a_log) * np.log1p(np.exp(np.minimum(oracle.bf16_to_f32(d["a"]), 20.0))),  # bias dropped
                 np.exp(a_log) * sp):                 # sign
        assert _f32_ulps(slip, want).max() > 100


# ------------------------------------------------------------------ attention prologue

def test_attn_prologue_matches_eager_golden(oracle, golden):
    d = golden("prologue")
    for n in ("q", "k"):
        got = oracle.attn_prologue(d[n], d[f"{n}_w"], d["cos"], d["sin"])
        from helpers import ulp_diff
        ulps = ulp_diff(got, d[f"{n}_out"])
        assert ulps.max() <= 1 and (ulps > 0).mean() < 1e-3, n


def test_attn_prologue_vs_f64_and_special_cases(oracle, golden):
    d = golden("prologue")
    got = oracle.bf16_to_f32(oracle.attn_prologue(d["q"], d["q_w"], d["cos"], d["sin"])).astype(np.float64)
    ref = oracle.attn_prologue_f64(d["q"], d["q_w"], d["cos"], d["sin"])
    # each bf16 rounding is within 2^-9 of what it rounds: the normalised value y,
    # the products y*cos and rot*sin, and their sum
    y = oracle.attn_prologue_f64(d["q"], d["q_w"])
    R = d["cos"].shape[-1]
    c = np.abs(oracle.bf16_to_f32(d["cos"]))[:, :, None, :]
    sn = np.abs(oracle.bf16_to_f32(d["sin"]))[:, :, None, :]
    scale = np.abs(y).copy()
    yr = np.abs(y[..., :R])
    scale[..., :R] = yr * c + np.concatenate([yr[..., R // 2:], yr[..., :R // 2]], axis=-1) * sn + np.abs(ref[..., :R])
    assert (np.abs(got - ref) <= 2.0 ** -7 * scale + 1e-6).all()
    # cos = 1, sin = 0 leaves the normalised row unchanged; rotary_dim 0 is the plain RMSNorm
    one = oracle.f32_to_bf16(np.ones(d["cos"].shape, np.float32))
    zero = oracle.f32_to_bf16(np.zeros(d["sin"].shape, np.float32))
    plain = oracle.attn_prologue(d["q"], d["q_w"], None, None)
    assert np.array_equal(oracle.attn_prologue(d["q"], d["q_w"], one, zero), plain)
    # the plain RMSNorm agrees with the add+RMSNorm oracle (no residual) to one bf16 ulp
    from helpers import ulp_diff
    x = d["q"].reshape(-1, 128)
    w = d["q_w"]
    other, _ = oracle.add_rmsnorm(x, None, w)
    assert ulp_diff(plain.reshape(-1, 128), other).max() <= 1


def test_planted_prologue_slips_fail_the_golden(oracle, golden):
    d = golden("prologue")
    want = oracle.bf16_to_f32(d["q_out"]).astype(np.float64)
    q, w, c, s = d["q"], d["q_w"], d["cos"], d["sin"]
    sin_neg = oracle.f32_to_bf16(-oracle.bf16_to_f32(s))
    for slip in (oracle.attn_prologue(q, w, c, sin_neg),                       # rotation the wrong way
                 oracle.attn_prologue(q, w, c, s, gain_offset=False),           # w instead of 1 + w
                 oracle.attn_prologue(q, w, s, c)):                             # cos and sin swapped
        assert np.abs(oracle.bf16_to_f32(slip) - want).max() > 0.05


# ------------------------------------------------------------------ slot readout

def test_slot_readout_matches_eager_golden(oracle, golden):
    d = golden("readout_slots")
    lg, p = oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], d["nopts"])
    # bf16 logits: the fp64 restatement and the eager fp32 path round to the same or a neighbouring bf16
    assert np.abs(lg - d["logits"]).max() <= 2.0 ** -8 * np.abs(d["logits"]).max()
    assert np.abs(p - d["probs"]).max() < 1e-2
    assert np.array_equal(p.argmax(1), d["probs"].argmax(1))
    _, p2 = oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], d["nopts"],
                                temperature=2.0)
    assert np.abs(p2 - d["probs_t2"]).max() < 1e-2
    assert all((p[i, n:] == 0).all() for i, n in enumerate(d["nopts"]))


def test_slot_readout_closed_forms_and_slips(oracle, golden):
    d = golden("readout_slots")
    lg, p = oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], d["nopts"])
    # one allowed letter: probability 1; softmax rows sum to 1
    _, p1 = oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], np.ones(6, np.int32))
    assert np.allclose(p1[:, 0], 1.0) and np.allclose(p.sum(1), 1.0)
    # slips: the norm's gain without the +1, the wrong slot, a transposed gather
    assert np.abs(oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], d["nopts"],
                                      gain_offset=False)[0] - d["logits"]).max() > 0.05
    assert np.abs(oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"] - 1,
                                      d["nopts"])[0] - d["logits"]).max() > 0.05
    assert np.abs(oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], 1 - d["rows"], d["pos"],
                                      d["nopts"])[0] - d["logits"]).max() > 0.05


# ------------------------------------------------------------------ gated norm and MLP gate

def test_gated_rmsnorm_and_silu_mul_match_eager_golden(oracle, golden):
    from helpers import ulp_diff
    d = golden("fusions")
    for tag in ("bf16", "f32"):
        y = oracle.gated_rmsnorm(d["x"], d["z"], d[f"w_{tag}"])
        u = ulp_diff(oracle.f32_to_bf16(y.astype(np.float32)), d[f"y_{tag}"])
        assert u.max() <= 1 and (u > 0).mean() < 1e-2, tag
    m = oracle.silu_mul(d["gu"])
    u = ulp_diff(oracle.f32_to_bf16(m.astype(np.float32)), d["mlp"])
    assert u.max() <= 1 and (u > 0).mean() < 1e-2


def test_planted_fusion_slips_fail_the_golden(oracle, golden):
    d = golden("fusions")
    want = oracle.bf16_to_f32(d["y_bf16"]).astype(np.float64)
    x, z = oracle.bf16_to_f32(d["x"]).astype(np.float64), oracle.bf16_to_f32(d["z"]).astype(np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    w = oracle.bf16_to_f32(d["w_bf16"])
    for slip in (y * w * z / (1 + np.exp(z)),          # silu sign
                 y * w * (1.0 / (1 + np.exp(-z))),      # sigmoid instead of silu
                 (y * (1 + w)) * z / (1 + np.exp(-z))):  # offset gain
        assert np.abs(slip - want).max() > 0.05
    gu = oracle.bf16_to_f32(d["gu"]).astype(np.float64)
    wrong = gu[:, 512:] / (1 + np.exp(-gu[:, 512:])) * gu[:, :512]    # gate and up swapped
    assert np.abs(wrong - oracle.bf16_to_f32(d["mlp"])).max() > 0.05
