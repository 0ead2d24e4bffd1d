"""Write the golden fixtures of the decider hot path (run: python tests/golden/make_golden.py).

The expected outputs come from the reference's PyTorch path on CPU — the
operations the reference itself uses as ground truth — never from this
repository's oracle or kernels:

* conv: fp32 ``F.conv1d`` (depthwise, padding W-1, sliced to T) + SiLU, one cast
  to bf16 (BASELINE config 2's recipe; the eager op is transformers'
  ``causal_conv1d_fn``), and the reference test's fp64 tap loop
  (ref: experiments/packed_conv/check_packed_output_conv.py:21-32);
* RMSNorm: the eager decoder-layer arithmetic, ``h = residual + x`` in bf16
  then transformers' ``Qwen3_5RMSNorm`` (its ``(1 + w)`` gain, eps inside rsqrt);
* GQA: ``F.scaled_dot_product_attention`` (MATH backend, fp32) on K/V repeated
  per group with a causal mask, the reference oracle
  (ref: experiments/native_gqa/bench_native_gqa.py:46-48), per request for varlen;
* readout: brute-force argmax over the allowed letters;
* gated delta rule: transformers' ``torch_chunk_gated_delta_rule`` (fp32 CPU,
  ``use_qk_l2norm_in_kernel=True`` on bf16 q/k, as the decider's layers call it,
  ref: src/decider/packed_conv.py:55-59), per request for varlen, q/k heads
  expanded by ``repeat_interleave`` as ``Qwen3_5GatedDeltaNet.forward`` does,
  and transformers' ``l2norm`` on bf16 rows;
* attention prologue: transformers' ``Qwen3_5RMSNorm`` (q_norm / k_norm over
  head_dim) and ``apply_rotary_pos_emb`` on bf16, with cos / sin from the
  decider shape's ``Qwen3_5TextRotaryEmbedding`` (partial rotary factor 0.25);
* slot readout: the model's final ``Qwen3_5RMSNorm`` on bf16 hidden states, the
  gather at the slots, ``F.linear`` with the bf16 letter rows, ``.float()`` and
  the masked softmax of the reference readout (ref: src/decider/engine.py:48-56);
* gated norm and MLP gate: transformers' ``Qwen3_5RMSNormGated`` (bf16 weight and
  fp32 weight) and ``act_fn(gate) * up`` of ``Qwen3_5MLP`` on bf16 tensors;
* gate transform: the eager expressions ``-A_log.float().exp() * F.softplus(a.float()
  + dt_bias)`` and ``b.sigmoid()`` (ref: src/decider/packed_conv.py:49-53) on bf16
  a, b and bf16 / fp32 parameters.

bf16 arrays are stored as uint16 bit patterns.  Each fixture is small (< 1 MB).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))  # the repository root, for the decider shape of the rotary table


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def conv_ref_fp32(x: torch.Tensor, w: torch.Tensor, bias=None, segments=None) -> torch.Tensor:
    """fp32 depthwise causal conv1d + SiLU, then one bf16 cast. x [B,T,C] bf16, w [C,W] bf16."""
    B, T, C = x.shape
    W = w.shape[1]

    def one(xs):
        y = F.conv1d(xs.float().transpose(1, 2), w.float()[:, None, :], None if bias is None else bias.float(),
                     padding=W - 1, groups=C)[..., :xs.shape[1]]
        return F.silu(y).transpose(1, 2).to(torch.bfloat16)

    if segments is None:
        return one(x)
    return torch.cat([one(x[:, a:b]) for a, b in segments if b > a], dim=1)


def conv_ref_fp64(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The reference test's fp64 tap loop (ref: experiments/packed_conv/check_packed_output_conv.py:21-32)."""
    T = x.shape[1]
    W = w.shape[1]
    wd = w.double()
    xf = x.double()
    acc = torch.zeros_like(xf)
    for tap in range(W):
        lag = W - 1 - tap
        acc[:, lag:, :] += xf[:, :T - lag, :] * wd[:, tap]
    return (acc * torch.sigmoid(acc)).to(torch.bfloat16)


def rms_eager(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm
    h = residual + x  # bf16 add, as Qwen3_5DecoderLayer
    norm = Qwen3_5RMSNorm(x.shape[-1], eps=eps)
    with torch.no_grad():
        norm.weight.data = weight.clone()
        return norm(h), h


def sdpa_ref(q, k, v, cu=None):
    """fp32 MATH SDPA with repeated KV and causal mask; q [B,Hq,T,D], k/v [B,Hkv,T,D]."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    group = q.shape[1] // k.shape[1]
    kr = k.repeat_interleave(group, dim=1)
    vr = v.repeat_interleave(group, dim=1)
    with sdpa_kernel(SDPBackend.MATH):
        if cu is None:
            return F.scaled_dot_product_attention(q.float(), kr.float(), vr.float(), is_causal=True)
        out = torch.zeros(q.shape, dtype=torch.float32)
        for a, b in zip(cu[:-1], cu[1:]):
            if b > a:
                out[:, :, a:b] = F.scaled_dot_product_attention(q[:, :, a:b].float(), kr[:, :, a:b].float(),
                                                                vr[:, :, a:b].float(), is_causal=True)
        return out


def make_conv(g: torch.Generator) -> dict:
    out = {}
    # padded batch: B=2, T=40, key_dim=value_dim=16 (C=48), W=4
    x = (torch.randn((2, 40, 48), generator=g)).to(torch.bfloat16)
    w = (torch.randn((48, 4), generator=g) * 0.25).to(torch.bfloat16)
    out.update(batch_x=bits(x), batch_w=bits(w), batch_y_fp32=bits(conv_ref_fp32(x, w)),
               batch_y_fp64=bits(conv_ref_fp64(x, w)))
    # with bias
    bias = (torch.randn((48,), generator=g) * 0.1).to(torch.bfloat16)
    out.update(bias_b=bits(bias), bias_y_fp32=bits(conv_ref_fp32(x, w, bias)))
    # varlen: one packed row of 50 tokens, requests [0,7), [7,7) (empty), [7,30), [30,50)
    xv = torch.randn((1, 50, 48), generator=g).to(torch.bfloat16)
    cu = [0, 7, 7, 30, 50]
    out.update(var_x=bits(xv), var_cu=np.array(cu, np.int32),
               var_y_fp32=bits(conv_ref_fp32(xv, w, segments=list(zip(cu[:-1], cu[1:])))))
    # decider-shaped channel split on a short sequence: C = 6144, T = 8
    xd = torch.randn((1, 8, 6144), generator=g).to(torch.bfloat16)
    wd = (torch.randn((6144, 4), generator=g) * 0.25).to(torch.bfloat16)
    out.update(dec_x=bits(xd), dec_w=bits(wd), dec_y_fp32=bits(conv_ref_fp32(xd, wd)))
    return out


def make_rms(g: torch.Generator) -> dict:
    out = {}
    x = torch.randn((3, 5, 256), generator=g).to(torch.bfloat16)
    r = torch.randn((3, 5, 256), generator=g).to(torch.bfloat16)
    w = (torch.randn((256,), generator=g) * 0.02).to(torch.bfloat16)
    y, h = rms_eager(x, r, w, 1e-6)
    out.update(small_x=bits(x), small_r=bits(r), small_w=bits(w), small_y=bits(y), small_h=bits(h))
    # decider width 2048, fp32 weight
    x2 = torch.randn((6, 2048), generator=g).to(torch.bfloat16)
    r2 = (torch.randn((6, 2048), generator=g) * 4).to(torch.bfloat16)
    w2 = torch.randn((2048,), generator=g) * 0.02
    y2, h2 = rms_eager(x2, r2, w2.to(torch.bfloat16), 1e-6)
    out.update(wide_x=bits(x2), wide_r=bits(r2), wide_w_bf16=bits(w2.to(torch.bfloat16)),
               wide_y=bits(y2), wide_h=bits(h2))
    # fp32 weight variant of the same rows (module weight kept in fp32)
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm
    norm = Qwen3_5RMSNorm(2048, eps=1e-6)
    with torch.no_grad():
        norm.weight.data = w2.clone()
        y3 = norm(h2)
    out.update(wide_w_f32=w2.numpy().astype(np.float32), wide_y_f32w=bits(y3))
    return out


def make_gqa(g: torch.Generator) -> dict:
    out = {}
    # config-1 recipe at a small size: fp32, N(0,1)/sqrt(D), drawn in order q, k, v
    D = 64
    q = torch.randn((1, 4, 48, D), generator=g) / D ** 0.5
    k = torch.randn((1, 2, 48, D), generator=g) / D ** 0.5
    v = torch.randn((1, 2, 48, D), generator=g) / D ** 0.5
    out.update(f32_q=q.numpy(), f32_k=k.numpy(), f32_v=v.numpy(), f32_o=sdpa_ref(q, k, v).numpy())
    # bf16 inputs (unscaled N(0,1) as ref: experiments/native_gqa/bench_native_gqa.py:43-45), D = 128
    D = 128
    qb = torch.randn((2, 4, 70, D), generator=g).to(torch.bfloat16)
    kb = torch.randn((2, 2, 70, D), generator=g).to(torch.bfloat16)
    vb = torch.randn((2, 2, 70, D), generator=g).to(torch.bfloat16)
    out.update(bf16_q=bits(qb), bf16_k=bits(kb), bf16_v=bits(vb), bf16_o=sdpa_ref(qb, kb, vb).numpy())
    # varlen bf16: 4 requests packed on T = 90 (one empty), 4 q / 1 kv heads, D = 64
    D = 64
    cu = [0, 13, 13, 64, 90]
    qv = torch.randn((1, 4, 90, D), generator=g).to(torch.bfloat16)
    kv = torch.randn((1, 1, 90, D), generator=g).to(torch.bfloat16)
    vv = torch.randn((1, 1, 90, D), generator=g).to(torch.bfloat16)
    out.update(var_q=bits(qv), var_k=bits(kv), var_v=bits(vv), var_cu=np.array(cu, np.int32),
               var_o=sdpa_ref(qv, kv, vv, cu).numpy())
    return out


def make_readout(g: torch.Generator) -> dict:
    logits = torch.randn((64, 10), generator=g, dtype=torch.float64)
    nopts = torch.randint(2, 11, (64,), generator=g)
    choice = np.array([int(np.argmax(row[:n])) for row, n in zip(logits.numpy(), nopts.numpy())])
    return dict(logits=logits.numpy(), nopts=nopts.numpy(), choice=choice)


def make_gated_delta(g: torch.Generator) -> dict:
    """q/k are stored after transformers' ``l2norm`` (the rule then runs with
    ``use_qk_l2norm_in_kernel=False``, which is the same computation): torch's CPU
    bf16 rsqrt rounds twice on rows its vectorised loop leaves to the scalar tail,
    which the GPU does not, so the normalisation is pinned on its own fixture."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    out = {}

    def inputs(T, hk, hv, g_lo, g_hi):
        q = torch.randn((1, T, hk, 128), generator=g).to(torch.bfloat16)
        k = torch.randn((1, T, hk, 128), generator=g).to(torch.bfloat16)
        v = torch.randn((1, T, hv, 128), generator=g).to(torch.bfloat16)
        # g = -exp(A_log) * softplus(a + dt_bias) spans these ranges in the decider
        gg = -torch.exp(torch.empty((1, T, hv)).uniform_(g_lo, g_hi, generator=g))
        beta = torch.rand((1, T, hv), generator=g).to(torch.bfloat16)
        return mq.l2norm(q, dim=-1, eps=1e-6), mq.l2norm(k, dim=-1, eps=1e-6), v, gg, beta

    def run(q, k, v, gg, beta, state=None, final=False):
        r = v.shape[2] // q.shape[2]
        if r > 1:
            q, k = q.repeat_interleave(r, dim=2), k.repeat_interleave(r, dim=2)
        return mq.torch_chunk_gated_delta_rule(q, k, v, g=gg, beta=beta, initial_state=state,
                                               output_final_state=final, use_qk_l2norm_in_kernel=False)

    # dense: T = 140 (two full chunks and a ragged one), 2 heads, long memory, final state
    q, k, v, gg, beta = inputs(140, 2, 2, -3.0, 0.5)
    o, fs = run(q, k, v, gg, beta, final=True)
    out.update(d_q=bits(q), d_k=bits(k), d_v=bits(v), d_g=gg.numpy(), d_beta=bits(beta), d_o=bits(o),
               d_final=fs.numpy())
    # decider-like decay, 1 key head shared by 2 value heads, an initial state
    q, k, v, gg, beta = inputs(96, 1, 2, 0.0, 2.5)
    s0 = torch.randn((1, 2, 128, 128), generator=g) * 0.05
    o, fs = run(q, k, v, gg, beta, state=s0, final=True)
    out.update(s_q=bits(q), s_k=bits(k), s_v=bits(v), s_g=gg.numpy(), s_beta=bits(beta), s_init=s0.numpy(),
               s_o=bits(o), s_final=fs.numpy())
    # varlen: 4 requests packed on T = 150 (one empty), each run alone with a fresh state
    cu = [0, 70, 71, 71, 150]
    q, k, v, gg, beta = inputs(150, 2, 2, -2.0, 1.0)
    parts = [run(q[:, a:b], k[:, a:b], v[:, a:b], gg[:, a:b], beta[:, a:b])[0]
             for a, b in zip(cu[:-1], cu[1:]) if b > a]
    out.update(v_q=bits(q), v_k=bits(k), v_v=bits(v), v_g=gg.numpy(), v_beta=bits(beta),
               v_cu=np.array(cu, np.int32), v_o=bits(torch.cat(parts, dim=1)))
    # l2norm on 64 bf16 rows of 128 (all in torch's vectorised loop), tiny to large
    x = torch.randn((64, 128), generator=g) * torch.logspace(-3, 3, 64)[:, None]
    xb = x.to(torch.bfloat16)
    out.update(l2_x=bits(xb), l2_y=bits(mq.l2norm(xb, dim=-1, eps=1e-6)))
    return out


def make_gates(g: torch.Generator) -> dict:
    H = 16
    a = (torch.randn((1, 300, H), generator=g) * 4).to(torch.bfloat16)
    b = (torch.randn((1, 300, H), generator=g) * 4).to(torch.bfloat16)
    a[0, :4] = torch.tensor([19.5, 20.0, 20.5, 40.0]).to(torch.bfloat16)[:, None]  # around softplus's threshold
    a_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt_bias = torch.ones(H) + 0.1 * torch.randn(H, generator=g)
    out = dict(a=bits(a), b=bits(b))
    for tag, dt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
        al, db = a_log.to(dt), dt_bias.to(dt)
        gg = -al.float().exp() * F.softplus(a.float() + db)
        out.update({f"{tag}_a_log": al.float().numpy(), f"{tag}_dt_bias": db.float().numpy(), f"{tag}_g": gg.numpy()})
    out["beta"] = bits(b.sigmoid())
    return out


def make_prologue(g: torch.Generator) -> dict:
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, make_config
    cfg = make_config(DECIDER_2B_SHAPED)
    rope = mq.Qwen3_5TextRotaryEmbedding(cfg)
    T = 40
    q = torch.randn((1, T, 4, 128), generator=g).to(torch.bfloat16) * 3
    k = torch.randn((1, T, 2, 128), generator=g).to(torch.bfloat16)
    pos = torch.arange(100, 100 + T)[None]
    cos, sin = rope(q, pos)
    qn = mq.Qwen3_5RMSNorm(128, eps=1e-6)
    kn = mq.Qwen3_5RMSNorm(128, eps=1e-6)
    with torch.no_grad():
        qn.weight.copy_(torch.randn(128, generator=g) * 0.1)
        kn.weight.copy_(torch.randn(128, generator=g) * 0.1)
    qn, kn = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    with torch.no_grad():
        qe, ke = mq.apply_rotary_pos_emb(qn(q).transpose(1, 2), kn(k).transpose(1, 2), cos, sin)
    return dict(q=bits(q), k=bits(k), q_w=bits(qn.weight.data), k_w=bits(kn.weight.data), cos=bits(cos),
                sin=bits(sin), q_out=bits(qe.transpose(1, 2)), k_out=bits(ke.transpose(1, 2)))


def make_readout_slots(g: torch.Generator) -> dict:
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    H, K = 2048, 10
    hidden = (torch.randn((2, 50, H), generator=g) * 2).to(torch.bfloat16)
    norm = mq.Qwen3_5RMSNorm(H, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(H, generator=g) * 0.02)
    norm = norm.to(torch.bfloat16)
    letters = (torch.randn((K, H), generator=g) * 0.02).to(torch.bfloat16)
    rows = torch.tensor([0, 0, 1, 1, 1, 0])
    pos = torch.tensor([49, 3, 0, 25, 49, 17])
    nopts = torch.tensor([4, 10, 2, 7, 10, 3])
    with torch.no_grad():
        lg = F.linear(norm(hidden)[rows, pos], letters).float()
    masked = lg.masked_fill(torch.arange(K)[None, :] >= nopts[:, None], float("-inf"))
    return dict(hidden=bits(hidden), norm_w=norm.weight.data.float().numpy(), letters=bits(letters),
                rows=rows.numpy().astype(np.int32), pos=pos.numpy().astype(np.int32),
                nopts=nopts.numpy().astype(np.int32), logits=lg.numpy(), probs=torch.softmax(masked, -1).numpy(),
                probs_t2=torch.softmax(masked / 2.0, -1).numpy())


def make_fusions(g: torch.Generator) -> dict:
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    x = (torch.randn((300, 128), generator=g) * 0.3).to(torch.bfloat16)
    z = (torch.randn((300, 128), generator=g) * 2).to(torch.bfloat16)
    w = 1.0 + 0.02 * torch.randn(128, generator=g)
    out = dict(x=bits(x), z=bits(z), w_f32=w.numpy())
    for tag, dt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
        norm = mq.Qwen3_5RMSNormGated(128, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(w)
        norm = norm.to(dt)
        with torch.no_grad():
            out[f"y_{tag}"] = bits(norm(x, z))
    out["w_bf16"] = bits(w.to(torch.bfloat16))
    gu = (torch.randn((64, 2 * 512), generator=g) * 3).to(torch.bfloat16)
    act = torch.nn.SiLU()
    out.update(gu=bits(gu), mlp=bits(act(gu[:, :512]) * gu[:, 512:]))
    return out


FIXTURES = (("conv", make_conv), ("rmsnorm", make_rms), ("gqa", make_gqa), ("readout", make_readout),
            ("gated_delta", make_gated_delta), ("gates", make_gates), ("prologue", make_prologue),
            ("readout_slots", make_readout_slots), ("fusions", make_fusions))


def main(names=None) -> None:
    torch.manual_seed(0)
    for name, fn in FIXTURES:
        if names and name not in names:
            continue
        g = torch.Generator().manual_seed(20260101)
        data = fn(g)
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    import sys
    main(sys.argv[1:])
