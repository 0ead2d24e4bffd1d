"""Packed causal depthwise conv1d + SiLU on the gfx950 HIP kernel ``fd_packed_conv_fwd``.

Drop-in for the reference's ``prep_qkv(input_qkv, weight)``
(ref: src/decider/packed_conv_kernel.py:194-232): input ``[B, T, 6144]`` bf16
contiguous token-major, depthwise weight ``[6144, 4]`` or ``[6144, 1, 4]``,
outputs q, k, v ``[B, T, 16, 128]`` bf16 contiguous, launched on the current
stream.  Validation and messages follow the reference; the fixed
``T == 2048`` (ref: :200-201) is lifted to any ``T >= 1``, and the input may be
a view of the first C columns of a wider projection output (uniform row stride).

Keyword extensions (defaults reproduce the reference exactly): ``bias``,
``head_k_dim``/``head_v_dim`` and ``key_dim``/``value_dim`` for other head
splits, ``activation`` (``"silu"`` or ``None``) and ``cu_seqlens`` for packed
variable-length batches (B == 1), where the causal window restarts at every
request start so no request reads another's tokens.
"""
from __future__ import annotations

import torch

from . import _lib

_ACTIVATIONS = {"silu": _lib.FD_ACT_SILU, None: _lib.FD_ACT_NONE}


def _check_conv(input_qkv, weight, bias, key_dim, value_dim, head_k_dim, head_v_dim, activation, cu_seqlens):
    """prep_qkv's validation; returns (B, T, key_dim, value_dim, row_stride, width, cu_ptr, n_seqs)."""
    if not input_qkv.is_cuda:
        raise ValueError("input_qkv must be on CUDA")
    if input_qkv.ndim != 3:
        raise ValueError("Expected input_qkv shape [B, T, C]")

    B, T, C = input_qkv.shape
    if key_dim is None and value_dim is None:
        if C % 3:
            raise ValueError("C must split into equal q/k/v parts unless key_dim/value_dim are given")
        key_dim = value_dim = C // 3
    elif key_dim is None or value_dim is None:
        raise ValueError("key_dim and value_dim must be given together")
    if B < 1 or T < 1 or C != 2 * key_dim + value_dim:
        raise ValueError("Expected input_qkv shape [B, T, 2*key_dim + value_dim], B >= 1, T >= 1")
    if key_dim % head_k_dim or value_dim % head_v_dim or head_k_dim % 8 or head_v_dim % 8:
        raise ValueError("key_dim/value_dim must be multiples of head dims that are multiples of 8")
    # a view of the first C columns of a wider projection output is accepted too (rows
    # stride(1) elements apart); the reference requires a contiguous tensor
    row_stride = input_qkv.stride(1)
    if (input_qkv.dtype != torch.bfloat16 or input_qkv.stride(2) != 1 or row_stride < C or row_stride % 8
            or (B > 1 and input_qkv.stride(0) != T * row_stride)):
        raise ValueError("input_qkv must be contiguous BF16")
    if weight.device != input_qkv.device:
        raise ValueError("weight and input_qkv must share a device")
    if weight.dtype != torch.bfloat16 or not weight.is_contiguous():
        raise ValueError("weight must be contiguous BF16")
    if weight.ndim == 3:
        if weight.shape[1] != 1:
            raise ValueError(f"Expected weight shape [{C}, W] or [{C}, 1, W]")
        width = weight.shape[2]
    elif weight.ndim == 2:
        width = weight.shape[1]
    else:
        raise ValueError(f"Expected weight shape [{C}, W] or [{C}, 1, W]")
    if weight.shape[0] != C or not 1 <= width <= 4:
        raise ValueError(f"Expected weight shape [{C}, W] or [{C}, 1, W] with 1 <= W <= 4")
    if bias is not None:
        if (bias.device != input_qkv.device or bias.dtype != torch.bfloat16 or bias.shape != (C,)
                or not bias.is_contiguous()):
            raise ValueError(f"bias must be a contiguous BF16 vector [{C}] on input_qkv's device")
    if activation not in _ACTIVATIONS:
        raise ValueError("activation must be 'silu' or None")
    tensors = [input_qkv, weight] + ([bias] if bias is not None else [])
    if any(t.data_ptr() % 16 for t in tensors):
        raise ValueError("Inputs must be aligned to 16 bytes")

    n_seqs = 0
    cu_ptr = None
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1 (packed requests)")
        if (cu_seqlens.ndim != 1 or cu_seqlens.dtype != torch.int32 or cu_seqlens.device != input_qkv.device
                or cu_seqlens.numel() < 2 or not cu_seqlens.is_contiguous()):
            raise ValueError("cu_seqlens must be a contiguous int32 vector [n_seqs + 1] on input_qkv's device")
        n_seqs = cu_seqlens.numel() - 1
        cu_ptr = cu_seqlens.data_ptr()
    return B, T, key_dim, value_dim, row_stride, width, cu_ptr, n_seqs


def _alloc_qkv(input_qkv, B, T, key_dim, value_dim, head_k_dim, head_v_dim):
    q = torch.empty((B, T, key_dim // head_k_dim, head_k_dim), device=input_qkv.device, dtype=input_qkv.dtype)
    k = torch.empty_like(q)
    v = torch.empty((B, T, value_dim // head_v_dim, head_v_dim), device=input_qkv.device, dtype=input_qkv.dtype)
    return q, k, v


def prep_qkv(
    input_qkv: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    key_dim: int | None = None,
    value_dim: int | None = None,
    head_k_dim: int = 128,
    head_v_dim: int = 128,
    activation: str | None = "silu",
    cu_seqlens: torch.Tensor | None = None,
):
    B, T, key_dim, value_dim, row_stride, width, cu_ptr, n_seqs = _check_conv(
        input_qkv, weight, bias, key_dim, value_dim, head_k_dim, head_v_dim, activation, cu_seqlens)
    with torch.cuda.device(input_qkv.device):
        q, k, v = _alloc_qkv(input_qkv, B, T, key_dim, value_dim, head_k_dim, head_v_dim)
        lib = _lib.lib()
        _lib.check("fd_packed_conv_strided_fwd", lib.fd_packed_conv_strided_fwd(
            input_qkv.data_ptr(), row_stride, weight.data_ptr(), _lib.ptr(bias), q.data_ptr(), k.data_ptr(),
            v.data_ptr(), B, T, key_dim, value_dim, width, cu_ptr, n_seqs, _ACTIVATIONS[activation],
            _lib.stream_handle(input_qkv.device)))
    return q, k, v


def prep_qkv_gates(
    input_qkv: torch.Tensor,
    weight: torch.Tensor,
    hidden_states: torch.Tensor,
    gate_weight: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    *,
    key_dim: int | None = None,
    value_dim: int | None = None,
    head_k_dim: int = 128,
    head_v_dim: int = 128,
    cu_seqlens: torch.Tensor | None = None,
):
    """``prep_qkv(input_qkv, weight)`` (SiLU, no bias) and
    ``gate_projection(hidden_states, gate_weight, a_log, dt_bias)`` of one layer
    in one launch (``fd_packed_conv_gate_fwd``): returns ``(q, k, v, decay, beta)``,
    bit-identical to the two calls made one after the other.  Each part takes the
    arguments, and raises the errors, of its own function."""
    B, T, key_dim, value_dim, row_stride, width, cu_ptr, n_seqs = _check_conv(
        input_qkv, weight, None, key_dim, value_dim, head_k_dim, head_v_dim, "silu", cu_seqlens)
    from .unpack_gate_transform_kernel import _PARAM_DTYPES, _check_gate_projection
    gB, gT, hidden, H = _check_gate_projection(hidden_states, gate_weight, a_log, dt_bias)
    if (gB, gT) != (B, T) or hidden_states.device != input_qkv.device:
        raise ValueError("hidden_states must be [B, T, hidden] with input_qkv's B and T, on its device")
    with torch.cuda.device(input_qkv.device):
        q, k, v = _alloc_qkv(input_qkv, B, T, key_dim, value_dim, head_k_dim, head_v_dim)
        decay = torch.empty((B, T, H), device=input_qkv.device, dtype=torch.float32)
        beta = torch.empty((B, T, H), device=input_qkv.device, dtype=torch.bfloat16)
        _lib.check("fd_packed_conv_gate_fwd", _lib.lib().fd_packed_conv_gate_fwd(
            input_qkv.data_ptr(), row_stride, weight.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), B, T,
            key_dim, value_dim, width, cu_ptr, n_seqs, hidden_states.data_ptr(), hidden_states.stride(1),
            gate_weight.data_ptr(), hidden, a_log.data_ptr(), _PARAM_DTYPES[a_log.dtype], dt_bias.data_ptr(),
            _PARAM_DTYPES[dt_bias.dtype], decay.data_ptr(), beta.data_ptr(), H,
            _lib.stream_handle(input_qkv.device)))
    return q, k, v, decay, beta
