"""Attention prologue on the gfx950 HIP kernel ``fd_attn_prologue_fwd``.

Replaces the eager prologue of the reference's patched attention forward
(ref: experiments/native_gqa/bench_native_gqa_model.py:47-53):
``q_norm`` / ``k_norm`` (transformers ``Qwen3_5RMSNorm`` over head_dim, gain
``1 + w``) and ``apply_rotary_pos_emb`` on the first ``rotary_dim`` features,
with every bf16 product and sum rounded as the eager bf16 ops round it.

``attention_prologue(q, k, q_weight, k_weight, cos, sin, eps)`` takes ``q``
``[B, T, Hq, D]`` and ``k`` ``[B, T, Hkv, D]`` as views with a contiguous
feature dimension (the query half of the ``q_proj`` output needs no copy) and
``cos``/``sin`` ``[B, T, R]`` bf16 (the model's position embeddings, R = 0 for
none); it returns contiguous ``[B, T, Hq, D]`` and ``[B, T, Hkv, D]`` tensors.
"""
from __future__ import annotations

import torch

from . import _lib

_W_DTYPES = {torch.bfloat16: _lib.FD_DTYPE_BF16, torch.float32: _lib.FD_DTYPE_F32}


def attention_prologue(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                       cos: torch.Tensor | None, sin: torch.Tensor | None, eps: float = 1e-6, *,
                       gain_offset: bool = True):
    if not q.is_cuda or q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or k.device != q.device:
        raise ValueError("q and k must be CUDA BF16 on one device")
    if q.ndim != 4 or k.ndim != 4 or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise ValueError("Expected q [B, T, Hq, D] and k [B, T, Hkv, D]")
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if D != 128:
        raise ValueError("head_dim must be 128")
    for name, t in (("q", q), ("k", k)):
        if t.stride(3) != 1 or t.stride(0) != T * t.stride(1):
            raise ValueError(f"{name} must have a contiguous feature dimension and packed token rows")
        if t.data_ptr() % 16 or t.stride(1) % 8 or t.stride(2) % 8:
            raise ValueError(f"{name} rows must be 16-byte aligned")
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        if w.shape != (D,) or w.dtype not in _W_DTYPES or w.device != q.device or not w.is_contiguous():
            raise ValueError(f"{name} must be a contiguous BF16 or FP32 vector [{D}] on q's device")
    if q_weight.dtype != k_weight.dtype:
        raise ValueError("q_weight and k_weight must share a dtype")
    rot = 0
    if cos is not None or sin is not None:
        if cos is None or sin is None or cos.shape != sin.shape or cos.ndim != 3 or cos.shape[:2] != (B, T):
            raise ValueError("cos and sin must both be [B, T, R]")
        rot = cos.shape[2]
        for t in (cos, sin):
            if t.dtype != torch.bfloat16 or t.device != q.device or not t.is_contiguous() or t.data_ptr() % 16:
                raise ValueError("cos and sin must be contiguous, 16-byte aligned BF16 on q's device")
    with torch.cuda.device(q.device):
        q_out = torch.empty((B, T, Hq, D), device=q.device, dtype=torch.bfloat16)
        k_out = torch.empty((B, T, Hkv, D), device=q.device, dtype=torch.bfloat16)
        _lib.check("fd_attn_prologue_fwd", _lib.lib().fd_attn_prologue_fwd(
            q.data_ptr(), q.stride(1), q.stride(2), k.data_ptr(), k.stride(1), k.stride(2),
            q_weight.data_ptr(), k_weight.data_ptr(), _W_DTYPES[q_weight.dtype], int(gain_offset), float(eps),
            _lib.ptr(cos), _lib.ptr(sin), rot, q_out.data_ptr(), k_out.data_ptr(), B * T, Hq, Hkv, D,
            _lib.stream_handle(q.device)))
    return q_out, k_out
