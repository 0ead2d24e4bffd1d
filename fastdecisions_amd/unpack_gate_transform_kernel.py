"""Gate transform of the Gated-DeltaNet layers on the gfx950 HIP kernel ``fd_gate_transform_fwd``.

Drop-in for the reference's ``unpack_gate(combined, a_log, dt_bias)``
(ref: src/decider/unpack_gate_transform_kernel.py:94-133): ``combined`` is the
``[B, T, 2H]`` bf16 output of the combined a/b projection (a in the first H
channels, b in the last H), ``a_log`` / ``dt_bias`` are ``[H]`` bf16 or fp32;
returns ``decay = -exp(a_log) * softplus(a + dt_bias)`` fp32 ``[B, T, H]`` and
``beta = sigmoid(b)`` bf16 ``[B, T, H]``, launched on the current stream.  The
reference fixes H = 16; any H works here.

``gate_transform(a, b, a_log, dt_bias)`` takes the two projections separately
(any row-contiguous ``[B, T, H]`` views, e.g. of one combined tensor).

``gate_projection(x, weight, a_log, dt_bias)`` also does the combined a|b
projection itself (``fd_gate_proj_fwd``): ``weight`` is
``cat(in_proj_a.weight, in_proj_b.weight)`` ``[2H, hidden]`` and ``x`` the
layer input ``[B, T, hidden]``, replacing the reference's separate GEMM and
transform (ref: src/decider/combined_gates.py:19-43).
"""
from __future__ import annotations

import torch

from . import _lib

_PARAM_DTYPES = {torch.bfloat16: _lib.FD_DTYPE_BF16, torch.float32: _lib.FD_DTYPE_F32}


def _check_params(a_log, dt_bias, heads, device):
    for name, parameter in (("a_log", a_log), ("dt_bias", dt_bias)):
        if parameter.shape != (heads,):
            raise ValueError(f"{name} must have shape [{heads}]")
        if parameter.device != device:
            raise ValueError(f"{name} must share combined's device")
        if parameter.dtype not in _PARAM_DTYPES:
            raise ValueError(f"{name} must be BF16 or FP32")
        if not parameter.is_contiguous():
            raise ValueError(f"{name} must be contiguous")


def gate_transform(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor):
    if not a.is_cuda or a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or b.device != a.device:
        raise ValueError("a and b must be CUDA BF16 on one device")
    if a.ndim != 3 or a.shape != b.shape:
        raise ValueError("a and b must have the same shape [B, T, H]")
    B, T, H = a.shape
    if B < 1 or T < 1:
        raise ValueError("B and T must be positive")
    for t in (a, b):
        if t.stride(2) != 1 or t.stride(0) != T * t.stride(1):
            raise ValueError("a and b must be row-contiguous views [B, T, H] (unit head stride, packed rows)")
    _check_params(a_log, dt_bias, H, a.device)
    with torch.cuda.device(a.device):
        decay = torch.empty((B, T, H), device=a.device, dtype=torch.float32)
        beta = torch.empty((B, T, H), device=a.device, dtype=torch.bfloat16)
        _lib.check("fd_gate_transform_fwd", _lib.lib().fd_gate_transform_fwd(
            a.data_ptr(), b.data_ptr(), a.stride(1), b.stride(1), a_log.data_ptr(), _PARAM_DTYPES[a_log.dtype],
            dt_bias.data_ptr(), _PARAM_DTYPES[dt_bias.dtype], decay.data_ptr(), beta.data_ptr(), B * T, H,
            _lib.stream_handle(a.device)))
    return decay, beta


def unpack_gate(combined: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor):
    # combined: contiguous BF16 [B, T, 2H]
    if combined.ndim != 3 or combined.shape[-1] % 2:
        raise ValueError("combined must have shape [B, T, 2H]")
    if not combined.is_cuda or combined.dtype != torch.bfloat16:
        raise ValueError("combined must be CUDA BF16")
    if not combined.is_contiguous():
        raise ValueError("combined must be contiguous")
    B, T, H2 = combined.shape
    if B < 1 or T < 1:
        raise ValueError("B and T must be positive")
    H = H2 // 2
    return gate_transform(combined[..., :H], combined[..., H:], a_log, dt_bias)


def _check_gate_projection(x, weight, a_log, dt_bias):
    """gate_projection's checks of x, weight and the parameters; returns (B, T, hidden, H)."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or weight.device != x.device:
        raise ValueError("x and weight must be CUDA BF16 on one device")
    if x.ndim != 3 or weight.ndim != 2 or weight.shape[1] != x.shape[2] or weight.shape[0] % 2:
        raise ValueError("x must be [B, T, hidden] and weight [2H, hidden]")
    B, T, hidden = x.shape
    H = weight.shape[0] // 2
    if B < 1 or T < 1:
        raise ValueError("B and T must be positive")
    if x.stride(2) != 1 or (B > 1 and x.stride(0) != T * x.stride(1)) or not weight.is_contiguous():
        raise ValueError("x must be row-contiguous [B, T, hidden] and weight contiguous")
    _check_params(a_log, dt_bias, H, x.device)
    return B, T, hidden, H


def gate_projection(x: torch.Tensor, weight: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor,
                    ab: torch.Tensor | None = None):
    B, T, hidden, H = _check_gate_projection(x, weight, a_log, dt_bias)
    if ab is not None and (ab.shape != (B, T, 2 * H) or ab.dtype != torch.bfloat16 or not ab.is_contiguous()
                           or ab.device != x.device):
        raise ValueError("ab must be a contiguous BF16 [B, T, 2H] tensor on x's device")
    with torch.cuda.device(x.device):
        decay = torch.empty((B, T, H), device=x.device, dtype=torch.float32)
        beta = torch.empty((B, T, H), device=x.device, dtype=torch.bfloat16)
        _lib.check("fd_gate_proj_fwd", _lib.lib().fd_gate_proj_fwd(
            x.data_ptr(), x.stride(1), weight.data_ptr(), hidden, a_log.data_ptr(), _PARAM_DTYPES[a_log.dtype],
            dt_bias.data_ptr(), _PARAM_DTYPES[dt_bias.dtype], decay.data_ptr(), beta.data_ptr(), _lib.ptr(ab),
            B * T, H, _lib.stream_handle(x.device)))
    return decay, beta
