"""Slot-only readout on the gfx950 HIP kernel ``fd_slot_readout_fwd``.

Mirrors the reference's opt-in ``SlotProjectionForward`` (ref:
src/decider/slot_projection.py:6-21): the letter projection runs only at the
requested ``(row, position)`` slots, from fixed-size device index buffers so the
forward can be replayed from a graph.  Here the model's final RMSNorm moves to
the slots as well (it is row-local), and the masked softmax of the readout
(ref: src/decider/engine.py:48-56) runs in the same kernel:

* ``slot_readout(hidden, norm_weight, letters, slot_rows, slot_positions, nopts,
  eps=..., temperature=1.0)`` -> ``(logits [N, K] fp32, probs [N, K] fp32)``;
  ``hidden`` is the residual stream *before* the final norm;
* ``SlotProjectionForward(model)`` — ``forward(input_ids, slot_rows,
  slot_positions)`` -> ``[N, K]`` fp32 letter logits, as the reference's module.
"""
from __future__ import annotations

import torch

from . import _lib

_W_DTYPES = {torch.bfloat16: _lib.FD_DTYPE_BF16, torch.float32: _lib.FD_DTYPE_F32}


def _index(t: torch.Tensor, n: int, device, name: str) -> torch.Tensor:
    if t.ndim != 1 or t.numel() != n or t.device != device:
        raise ValueError(f"{name} must be a vector [{n}] on hidden's device")
    return t.to(torch.int32).contiguous()


def slot_readout(hidden: torch.Tensor, norm_weight: torch.Tensor, letters: torch.Tensor, slot_rows: torch.Tensor,
                 slot_positions: torch.Tensor, nopts: torch.Tensor | None = None, *, eps: float = 1e-6,
                 gain_offset: bool = True, temperature: float = 1.0, with_probs: bool = True):
    if not hidden.is_cuda or hidden.dtype != torch.bfloat16 or hidden.ndim != 3 or not hidden.is_contiguous():
        raise ValueError("hidden must be a contiguous CUDA BF16 tensor [B, T, H]")
    B, T, H = hidden.shape
    if letters.ndim != 2 or letters.shape[1] != H or letters.dtype != torch.bfloat16 or not letters.is_contiguous():
        raise ValueError(f"letters must be a contiguous BF16 matrix [K, {H}]")
    if norm_weight.shape != (H,) or norm_weight.dtype not in _W_DTYPES or not norm_weight.is_contiguous():
        raise ValueError(f"norm_weight must be a contiguous BF16 or FP32 vector [{H}]")
    if letters.device != hidden.device or norm_weight.device != hidden.device:
        raise ValueError("weights must share hidden's device")
    N = slot_rows.numel()
    rows = _index(slot_rows, N, hidden.device, "slot_rows")
    pos = _index(slot_positions, N, hidden.device, "slot_positions")
    nop = None if nopts is None else _index(nopts, N, hidden.device, "nopts")
    K = letters.shape[0]
    with torch.cuda.device(hidden.device):
        logits = torch.empty((N, K), device=hidden.device, dtype=torch.float32)
        probs = torch.empty((N, K), device=hidden.device, dtype=torch.float32) if with_probs else None
        _lib.check("fd_slot_readout_fwd", _lib.lib().fd_slot_readout_fwd(
            hidden.data_ptr(), B, T, H, norm_weight.data_ptr(), _W_DTYPES[norm_weight.dtype], int(gain_offset),
            float(eps), letters.data_ptr(), K, rows.data_ptr(), pos.data_ptr(), _lib.ptr(nop), N,
            float(temperature), logits.data_ptr(), _lib.ptr(probs), _lib.stream_handle(hidden.device)))
    return logits, probs


class SlotProjectionForward(torch.nn.Module):
    """Return [slot_capacity, options] letter logits; the caller supplies valid flat
    row / position indices (fixed-size device buffers for graph replay; unused
    entries may point at row 0, position 0 and their outputs are discarded)."""

    def __init__(self, model):
        super().__init__()
        self.model = model

    def forward(self, input_ids, slot_rows, slot_positions, **kw):
        return self.model.slot_logits(input_ids, slot_rows, slot_positions, **kw)[0]
