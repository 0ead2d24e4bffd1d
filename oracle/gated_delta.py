"""TEST INFRASTRUCTURE — CPU oracle of the chunked gated delta rule (numpy).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module.  bf16 tensors travel as numpy uint16 arrays holding the raw bits.

The decider's linear-attention layers call transformers'
``torch_chunk_gated_delta_rule`` with ``use_qk_l2norm_in_kernel=True``
(ref: src/decider/packed_conv.py:55-59).  Its definition, restated here:

* ``l2norm_bf16`` — the q/k normalisation as it runs on the bf16 q/k the conv
  produces (transformers modeling_qwen3_5.py:242-245 applied to bf16 tensors):
  x*x, the row sum, +eps, rsqrt and the final product each rounded to bf16;
* ``recurrent`` — the token-by-token recurrence (modeling_qwen3_5.py:331-378):
  S <- e^{g_t} S;  d = beta_t (v_t - S^T k_t);  S <- S + k_t d^T;  o_t = S^T (scale q_t);
* ``chunked`` — the 64-token chunked form (modeling_qwen3_5.py:249-328):
  within a chunk, g cumsum, decay D_ij = e^{gc_i - gc_j} (j <= i),
  L = strictly-lower(beta_i k_i.k_j D_ij), T = (I + L)^-1,
  u = T (beta v), w = T (beta e^{gc} k); across chunks
  v' = u - w S,  o = (scale q e^{gc}) S + ((scale q k^T) o D) v',
  S <- e^{gc_last} S + (k e^{gc_last - gc})^T v'.

Both run in float64 from the same fp32 inputs; they are two independent
algorithms for the same quantity, so their agreement (tests/test_oracle.py)
pins each of them, and transformers' own fp32 CPU output is a golden fixture.
Packed requests (``cu_seqlens``) are run one request at a time with a fresh
state — what the reference's per-request decisions assume.
"""
from __future__ import annotations

import numpy as np

from .cpu import bf16_to_f32, f32_to_bf16

CHUNK = 64


def _bf16_round(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(np.asarray(x, dtype=np.float32)))


def l2norm_bf16(x_bits: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Row-wise x * rsqrt(sum(x*x) + eps) over the last axis of a bf16 tensor,
    every intermediate rounded to bf16 as torch does for bf16 operands; the row
    sum is accumulated in fp32 in index order.  Returns bf16 bits."""
    x = bf16_to_f32(x_bits)
    sq = _bf16_round(x * x)
    s = np.zeros(x.shape[:-1], dtype=np.float32)
    for i in range(x.shape[-1]):
        s = (s + sq[..., i]).astype(np.float32)
    s = _bf16_round(s)
    e = _bf16_round(s + np.float32(eps))
    inv = _bf16_round((np.float32(1.0) / np.sqrt(e.astype(np.float32))).astype(np.float32))
    return f32_to_bf16((x * inv[..., None]).astype(np.float32))


def _prepare(q_bits, k_bits, v_bits, g, beta, scale, l2norm):
    """Common front end: bf16 bits -> float64 arrays [N, T, H, D] (k/q heads
    expanded to the value heads as transformers' repeat_interleave does)."""
    if l2norm:
        q_bits, k_bits = l2norm_bf16(q_bits), l2norm_bf16(k_bits)
    q = bf16_to_f32(q_bits).astype(np.float64)
    k = bf16_to_f32(k_bits).astype(np.float64)
    v = bf16_to_f32(v_bits).astype(np.float64)
    hv, hk = v.shape[2], k.shape[2]
    if hv != hk:
        q = np.repeat(q, hv // hk, axis=2)
        k = np.repeat(k, hv // hk, axis=2)
    if beta.dtype == np.uint16:
        beta = bf16_to_f32(beta)
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(q.shape[-1])))
    return q * scale, k, v, np.asarray(g, dtype=np.float64), np.asarray(beta, dtype=np.float64)


def _segments(total: int, seq_len: int, batch: int, cu_seqlens):
    if cu_seqlens is None:
        return [(b, 0, seq_len) for b in range(batch)]
    cu = [int(c) for c in cu_seqlens]
    return [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def recurrent(q_bits, k_bits, v_bits, g, beta, *, scale=None, l2norm=True, cu_seqlens=None,
              initial_state=None):
    """Token-by-token gated delta rule in float64.  q/k [B,T,Hk,Dk], v [B,T,Hv,Dv]
    bf16 bits; g [B,T,Hv] fp32; beta [B,T,Hv] (bf16 bits or float).  Returns
    (o float64 [B,T,Hv,Dv], final states float64 [N,Hv,Dk,Dv])."""
    q, k, v, g, beta = _prepare(q_bits, k_bits, v_bits, g, beta, scale, l2norm)
    B, T, H, Dv = v.shape
    Dk = k.shape[-1]
    o = np.zeros((B, T, H, Dv))
    segs = _segments(B * T, T, B, cu_seqlens)
    finals = np.zeros((len(segs), H, Dk, Dv))
    for n, (b, s, e) in enumerate(segs):
        S = np.zeros((H, Dk, Dv)) if initial_state is None else np.array(initial_state[n], dtype=np.float64)
        for t in range(s, e):
            S = S * np.exp(g[b, t])[:, None, None]
            mem = np.einsum("hk,hkv->hv", k[b, t], S)
            d = (v[b, t] - mem) * beta[b, t][:, None]
            S = S + k[b, t][:, :, None] * d[:, None, :]
            o[b, t] = np.einsum("hk,hkv->hv", q[b, t], S)
        finals[n] = S
    return o, finals


def _chunked_one(q, k, v, g, beta, S):
    """One request, arrays [T, H, D] (q already scaled) -> (o [T,H,Dv], S)."""
    T, H, Dv = v.shape
    pad = (-T) % CHUNK
    if pad:
        q, k, v = (np.concatenate([a, np.zeros((pad,) + a.shape[1:])]) for a in (q, k, v))
        g, beta = (np.concatenate([a, np.zeros((pad,) + a.shape[1:])]) for a in (g, beta))
    o = np.zeros_like(v)
    tri_strict = np.tril(np.ones((CHUNK, CHUNK)), -1)
    tri = np.tril(np.ones((CHUNK, CHUNK)))
    eye = np.eye(CHUNK)
    for c0 in range(0, T + pad, CHUNK):
        sl = slice(c0, c0 + CHUNK)
        for h in range(H):
            qc, kc, vc = q[sl, h], k[sl, h], v[sl, h]
            gc = np.cumsum(g[sl, h])
            bc = beta[sl, h]
            D = np.exp((gc[:, None] - gc[None, :]) * tri) * tri
            L = (bc[:, None] * (kc @ kc.T)) * D * tri_strict
            Tm = np.linalg.solve(eye + L, eye)  # (I + L)^-1
            u = Tm @ (bc[:, None] * vc)
            w = Tm @ (bc[:, None] * np.exp(gc)[:, None] * kc)
            vn = u - w @ S[h]
            A = (qc @ kc.T) * D
            o[sl, h] = (qc * np.exp(gc)[:, None]) @ S[h] + A @ vn
            S[h] = S[h] * np.exp(gc[-1]) + (kc * np.exp(gc[-1] - gc)[:, None]).T @ vn
    return o[:T], S


def chunked(q_bits, k_bits, v_bits, g, beta, *, scale=None, l2norm=True, cu_seqlens=None, initial_state=None):
    """The 64-token chunked gated delta rule in float64 (same arguments and
    results as ``recurrent``)."""
    q, k, v, g, beta = _prepare(q_bits, k_bits, v_bits, g, beta, scale, l2norm)
    B, T, H, Dv = v.shape
    Dk = k.shape[-1]
    o = np.zeros((B, T, H, Dv))
    segs = _segments(B * T, T, B, cu_seqlens)
    finals = np.zeros((len(segs), H, Dk, Dv))
    for n, (b, s, e) in enumerate(segs):
        S = np.zeros((H, Dk, Dv)) if initial_state is None else np.array(initial_state[n], dtype=np.float64)
        if e > s:
            o[b, s:e], S = _chunked_one(q[b, s:e], k[b, s:e], v[b, s:e], g[b, s:e], beta[b, s:e], S)
        finals[n] = S
    return o, finals
