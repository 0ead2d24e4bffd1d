"""Chunked gated delta rule on the gfx950 HIP kernels behind ``fd_gated_delta_fwd``.

Drop-in for the call the reference's Gated-DeltaNet forward makes,
``torch_chunk_gated_delta_rule(query, key, value, g=g, beta=beta,
initial_state=None, output_final_state=False, use_qk_l2norm_in_kernel=True,
cu_seqlens=...)`` (ref: src/decider/packed_conv.py:55-59; transformers
modeling_qwen3_5.py:249-328): same positional arguments, keywords and
``(core_attn_out, last_recurrent_state)`` result, tensors ``[B, T, H, D]``.

Differences a caller can see:

* ``cu_seqlens`` (int32 ``[n + 1]`` on the device, B == 1) is honoured: each
  packed request runs from its own state (the torch form ignores it);
  ``initial_state`` / the final state are then ``[n, H, Dk, Dv]``;
* key heads may divide the value heads (value head h reads key head
  h // (Hv / Hk)), so the caller's ``repeat_interleave`` is not needed;
* head dims must be 128 and ``chunk_size`` 64 (the decider's geometry); q/k/v
  must be bf16, g fp32, beta bf16 or fp32; the output is bf16;
* ``norm=(z, weight, eps)`` applies the layer's gated RMSNorm
  (transformers ``Qwen3_5RMSNormGated``, the call after the delta rule at
  ref: src/decider/packed_conv.py:60-61) in the same library call
  (``fd_gated_delta_norm_fwd``: the delta rule's rows pass through the
  workspace): the result equals ``gated_rms_norm`` of the plain output, bit
  for bit; z is a ``[B, T, Hv, Dv]`` bf16 view.
"""
from __future__ import annotations

import torch

from . import _lib


def workspace_bytes(batch: int, seq_len: int, v_heads: int, n_seqs: int = 0) -> int:
    """Device workspace one call needs (n_seqs = packed requests, 0 for a padded batch)."""
    n = _lib.lib().fd_gated_delta_workspace_bytes(batch, seq_len, v_heads, 128, 128, n_seqs)
    if n < 0:
        raise ValueError(f"unsupported gated delta rule sizes (code {n})")
    return int(n)


def chunk_gated_delta_rule(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    chunk_size: int = 64,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    *,
    scale: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
    norm: tuple | None = None,
    **kwargs,
):
    if not value.is_cuda:
        raise ValueError("value must be on CUDA")
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("Expected query/key [B, T, Hk, Dk] and value [B, T, Hv, Dv]")
    B, T, Hk, Dk = key.shape
    Hv, Dv = value.shape[2], value.shape[3]
    if query.shape != key.shape or value.shape[:2] != (B, T):
        raise ValueError("query and key must match, and value must share their [B, T]")
    if Dk != 128 or Dv != 128:
        raise ValueError("head dims must be 128")
    if chunk_size != 64:
        raise ValueError("chunk_size must be 64")
    if Hv % Hk:
        raise ValueError(f"value heads ({Hv}) must be a multiple of key heads ({Hk})")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != value.device:
            raise ValueError(f"{name} must be contiguous BF16 on value's device")
    if g.shape != (B, T, Hv) or g.dtype != torch.float32 or not g.is_contiguous() or g.device != value.device:
        raise ValueError(f"g must be a contiguous float32 tensor [{B}, {T}, {Hv}] on value's device")
    if (beta.shape != (B, T, Hv) or beta.dtype not in (torch.bfloat16, torch.float32) or not beta.is_contiguous()
            or beta.device != value.device):
        raise ValueError(f"beta must be a contiguous BF16 or float32 tensor [{B}, {T}, {Hv}] on value's device")
    if any(t.data_ptr() % 16 for t in (query, key, value)):
        raise ValueError("query, key and value must be aligned to 16 bytes")

    n_seqs = 0
    cu_ptr = None
    n_states = B
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1 (packed requests)")
        if (cu_seqlens.ndim != 1 or cu_seqlens.dtype != torch.int32 or cu_seqlens.device != value.device
                or cu_seqlens.numel() < 2 or not cu_seqlens.is_contiguous()):
            raise ValueError("cu_seqlens must be a contiguous int32 vector [n_seqs + 1] on value's device")
        n_seqs = cu_seqlens.numel() - 1
        cu_ptr = cu_seqlens.data_ptr()
        n_states = n_seqs
    state_shape = (n_states, Hv, Dk, Dv)
    if initial_state is not None:
        if initial_state.shape != state_shape or initial_state.device != value.device:
            raise ValueError(f"initial_state must be {list(state_shape)} on value's device")
        initial_state = initial_state.to(torch.float32).contiguous()
    if scale is None:
        scale = 1.0 / Dk ** 0.5

    norm_args = None
    if norm is not None:
        z, norm_weight, norm_eps = norm
        norm_args = _norm_args(z, norm_weight, B, T, Hv, Dv, value.device)
    with torch.cuda.device(value.device):
        out = torch.empty((B, T, Hv, Dv), device=value.device, dtype=torch.bfloat16)
        final = torch.empty(state_shape, device=value.device, dtype=torch.float32) if output_final_state else None
        nbytes = workspace_bytes(B, T, Hv, n_seqs)
        work = torch.empty(max(nbytes, 16), device=value.device, dtype=torch.uint8)
        beta_dtype = _lib.FD_DTYPE_F32 if beta.dtype == torch.float32 else _lib.FD_DTYPE_BF16
        tail = (_lib.ptr(initial_state), _lib.ptr(final), work.data_ptr(), nbytes,
                B, T, Hk, Hv, Dk, Dv, float(scale), beta_dtype, int(bool(use_qk_l2norm_in_kernel)),
                cu_ptr, n_seqs, _lib.stream_handle(value.device))
        if norm_args is None:
            _lib.check("fd_gated_delta_fwd", _lib.lib().fd_gated_delta_fwd(
                query.data_ptr(), key.data_ptr(), value.data_ptr(), g.data_ptr(), beta.data_ptr(), out.data_ptr(),
                *tail))
        else:
            _lib.check("fd_gated_delta_norm_fwd", _lib.lib().fd_gated_delta_norm_fwd(
                query.data_ptr(), key.data_ptr(), value.data_ptr(), g.data_ptr(), beta.data_ptr(), *norm_args,
                float(norm_eps), out.data_ptr(), *tail))
    return out, final


_NORM_W_DTYPES = {torch.bfloat16: _lib.FD_DTYPE_BF16, torch.float32: _lib.FD_DTYPE_F32}


def _norm_args(z: torch.Tensor, weight: torch.Tensor, B: int, T: int, Hv: int, Dv: int, device):
    """(z pointer, token stride, head stride, weight pointer, weight dtype) for the gated-norm epilogue;
    z is a [B, T, Hv, Dv] bf16 view with unit feature stride and uniformly strided tokens."""
    if z.shape != (B, T, Hv, Dv) or z.dtype != torch.bfloat16 or z.device != device:
        raise ValueError(f"z must be a BF16 [{B}, {T}, {Hv}, {Dv}] tensor on value's device")
    ts, hs = z.stride(1), z.stride(2)
    if z.stride(3) != 1 or (B > 1 and z.stride(0) != T * ts) or ts % 8 or hs % 8 or z.data_ptr() % 16:
        raise ValueError("z rows must be contiguous, 16-byte aligned and uniformly strided over tokens")
    if weight.shape != (Dv,) or weight.dtype not in _NORM_W_DTYPES or weight.device != device \
            or not weight.is_contiguous():
        raise ValueError(f"the norm weight must be a contiguous BF16 or FP32 vector [{Dv}] on value's device")
    return z.data_ptr(), ts, hs, weight.data_ptr(), _NORM_W_DTYPES[weight.dtype]
