"""Gated RMSNorm and the MLP's SiLU gate on the gfx950 HIP kernels
``fd_gated_rmsnorm_fwd`` / ``fd_silu_mul_fwd``.

* ``gated_rms_norm(x, gate, weight, eps)`` — transformers' ``Qwen3_5RMSNormGated``
  (the norm after the delta rule, ref: src/decider/packed_conv.py:60-61) with the
  eager rounding; x / gate ``[..., D]`` bf16, D in {64, 128, 256};
* ``silu_mul(gate_up)`` — ``silu(gate) * up`` of transformers' ``Qwen3_5MLP`` on one
  combined ``[..., 2I]`` gate|up projection output, returning ``[..., I]``.
"""
from __future__ import annotations

import torch

from . import _lib

_W_DTYPES = {torch.bfloat16: _lib.FD_DTYPE_BF16, torch.float32: _lib.FD_DTYPE_F32}


def gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x: contiguous [..., D]; gate: [..., heads, D] view with the same number of rows, a unit
    feature stride and uniformly strided tokens (e.g. part of a combined projection output)."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16 or gate.device != x.device:
        raise ValueError("x and gate must be CUDA BF16 on one device")
    D = x.shape[-1]
    if D not in (64, 128, 256) or gate.shape[-1] != D or gate.numel() != x.numel() or gate.ndim < 2:
        raise ValueError("x [..., D] and gate [..., heads, D] must hold the same rows, D in {64, 128, 256}")
    if not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError("x must be contiguous and 16-byte aligned")
    heads = gate.shape[-2]
    hs = gate.stride(-2)
    if gate.ndim == 2:
        ts = heads * hs
    else:
        ts = gate.stride(-3)
        dims, strides = gate.shape[:-3], gate.stride()[:-3]
        expect = ts * gate.shape[-3]
        for size, stride in zip(reversed(dims), reversed(strides)):
            if size != 1 and stride != expect:
                raise ValueError("gate tokens must be uniformly strided")
            expect *= size
    if gate.stride(-1) != 1 or gate.data_ptr() % 16 or hs % 8 or ts % 8:
        raise ValueError("gate rows must be contiguous and 16-byte aligned")
    if weight.shape != (D,) or weight.dtype not in _W_DTYPES or weight.device != x.device or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous BF16 or FP32 vector [{D}] on x's device")
    rows = x.numel() // D
    with torch.cuda.device(x.device):
        out = torch.empty_like(x)
        _lib.check("fd_gated_rmsnorm_fwd", _lib.lib().fd_gated_rmsnorm_fwd(
            x.data_ptr(), gate.data_ptr(), ts, hs, heads, weight.data_ptr(), _W_DTYPES[weight.dtype],
            out.data_ptr(), rows, D, float(eps), _lib.stream_handle(x.device)))
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    if not gate_up.is_cuda or gate_up.dtype != torch.bfloat16 or gate_up.shape[-1] % 16:
        raise ValueError("gate_up must be CUDA BF16 [..., 2I] with I a multiple of 8")
    if not gate_up.is_contiguous() or gate_up.data_ptr() % 16:
        raise ValueError("gate_up must be contiguous and 16-byte aligned")
    width = gate_up.shape[-1] // 2
    rows = gate_up.numel() // gate_up.shape[-1]
    with torch.cuda.device(gate_up.device):
        out = torch.empty((*gate_up.shape[:-1], width), device=gate_up.device, dtype=torch.bfloat16)
        _lib.check("fd_silu_mul_fwd", _lib.lib().fd_silu_mul_fwd(
            gate_up.data_ptr(), gate_up.shape[-1], out.data_ptr(), rows, width, _lib.stream_handle(gate_up.device)))
    return out


def silu_mul_split(gate_up1: torch.Tensor, gate_up2: torch.Tensor) -> torch.Tensor:
    """``silu_mul`` over two gate|up projections ``[..., 2*I1]`` and ``[..., 2*I2]``
    (``fd_silu_mul_split_fwd``): returns ``[..., I1 + I2]``, features ``[0, I1)``
    from the first, each computed exactly as ``silu_mul`` computes it."""
    for t in (gate_up1, gate_up2):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.shape[-1] % 16:
            raise ValueError("gate_up must be CUDA BF16 [..., 2I] with I a multiple of 8")
        if not t.is_contiguous() or t.data_ptr() % 16:
            raise ValueError("gate_up must be contiguous and 16-byte aligned")
    if gate_up1.shape[:-1] != gate_up2.shape[:-1] or gate_up1.device != gate_up2.device:
        raise ValueError("gate_up1 and gate_up2 must have the same leading shape and device")
    w1, w2 = gate_up1.shape[-1] // 2, gate_up2.shape[-1] // 2
    rows = gate_up1.numel() // gate_up1.shape[-1]
    with torch.cuda.device(gate_up1.device):
        out = torch.empty((*gate_up1.shape[:-1], w1 + w2), device=gate_up1.device, dtype=torch.bfloat16)
        _lib.check("fd_silu_mul_split_fwd", _lib.lib().fd_silu_mul_split_fwd(
            gate_up1.data_ptr(), gate_up1.shape[-1], w1, gate_up2.data_ptr(), gate_up2.shape[-1], w2, out.data_ptr(),
            rows, _lib.stream_handle(gate_up1.device)))
    return out
