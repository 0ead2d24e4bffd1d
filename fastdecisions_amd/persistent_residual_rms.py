"""Residual add + RMSNorm torch ops and the decoder-layer patch that uses them.

Mirrors ref: src/decider/persistent_residual_rms.py:

* ``residual_rms_op(a, b, weight)`` — the reference op ``fastdecisions::residual_rms``
  (ref: :7-14), normed output only;
* ``fused_add_rms_norm_op(x, residual, weight, eps) -> (normed, residual)`` and
  ``rms_norm_op(x, weight, eps)`` — the same kernel returning the updated
  residual too, and without a residual;
* ``_forward`` — replacement ``Qwen3_5DecoderLayer.forward`` (ref: :17-33):
  input RMSNorm on the kernel, the token mixer, then one fused kernel for
  ``residual + mixer`` and the post-attention RMSNorm, whose second output is
  the residual the MLP adds onto (the reference recomputes it in Python, :33);
* ``_chain_step`` — the same layer with the residual add of the previous
  layer's MLP still pending: that add goes into this layer's input RMSNorm
  kernel (``h = bf16(residual + mlp)``, then the norm of h), so a stack of
  patched layers runs no separate add kernel; the decider's layer loop uses
  it when every decoder layer is patched;
* ``install_persistent_residual_rms(core, all_layers=False)`` — patches the
  linear-attention layers as the reference does (ref: :36-49), or every
  decoder layer with ``all_layers=True`` (which also enables the chained
  residual); requires width <= 8192 and the layer's eps (the reference
  additionally fixes width 2048 and eps 1e-6).
"""
from __future__ import annotations

from types import MethodType

import torch

from .persistent_residual_rms_kernel import fused_add_rms_norm, residual_rms, rms_norm


@torch.library.custom_op("fastdecisions::residual_rms", mutates_args=(), device_types="cuda")
def residual_rms_op(a: torch.Tensor, b: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return residual_rms(a, b, weight)


@residual_rms_op.register_fake
def _residual_rms_fake(a, b, weight):
    return a.new_empty(a.shape)


@torch.library.custom_op("fastdecisions::fused_add_rms_norm", mutates_args=(), device_types="cuda")
def fused_add_rms_norm_op(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return fused_add_rms_norm(x, residual, weight, eps)


@fused_add_rms_norm_op.register_fake
def _fused_add_rms_norm_fake(x, residual, weight, eps):
    return x.new_empty(x.shape), x.new_empty(x.shape)


@torch.library.custom_op("fastdecisions::rms_norm", mutates_args=(), device_types="cuda")
def rms_norm_op(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return rms_norm(x, weight, eps)


@rms_norm_op.register_fake
def _rms_norm_fake(x, weight, eps):
    return x.new_empty(x.shape)


def _forward(self, hidden_states, position_embeddings, attention_mask=None, position_ids=None,
             past_key_values=None, **kwargs):
    if (past_key_values is not None or self.training or torch.is_grad_enabled()
            or not hidden_states.is_cuda or hidden_states.dtype != torch.bfloat16
            or not hidden_states.is_contiguous()):
        return self._persistent_original_forward(
            hidden_states, position_embeddings, attention_mask=attention_mask,
            position_ids=position_ids, past_key_values=past_key_values, **kwargs)
    residual = hidden_states
    normalized = rms_norm_op(hidden_states, self.input_layernorm.weight, self.input_layernorm.eps)
    if self.block_type == "linear_attention":
        mixed = self.linear_attn(hidden_states=normalized, cache_params=None, attention_mask=attention_mask,
                                 **kwargs)
    else:
        mixed, _ = self.self_attn(hidden_states=normalized, attention_mask=attention_mask,
                                  position_ids=position_ids, past_key_values=None,
                                  position_embeddings=position_embeddings, **kwargs)
    normalized, residual = fused_add_rms_norm_op(mixed.contiguous(), residual, self.post_attention_layernorm.weight,
                                                 self.post_attention_layernorm.eps)
    return residual + self.mlp(normalized)


def _chain_step(self, residual, delta, position_embeddings, attention_mask=None, position_ids=None, **kwargs):
    """Decoder layer on (residual, delta) with the previous layer's ``residual + delta``
    not yet formed (``delta`` is None for the first layer); returns this layer's
    (residual, mlp output).  Same arithmetic as the eager layer: the add is rounded
    to bf16 (it is the updated residual) before it is normalised."""
    if delta is None:
        normalized = rms_norm_op(residual, self.input_layernorm.weight, self.input_layernorm.eps)
    else:
        normalized, residual = fused_add_rms_norm_op(delta, residual, self.input_layernorm.weight,
                                                     self.input_layernorm.eps)
    if self.block_type == "linear_attention":
        mixed = self.linear_attn(hidden_states=normalized, cache_params=None, attention_mask=attention_mask,
                                 **kwargs)
    else:
        mixed, _ = self.self_attn(hidden_states=normalized, attention_mask=attention_mask,
                                  position_ids=position_ids, past_key_values=None,
                                  position_embeddings=position_embeddings, **kwargs)
    normalized, residual = fused_add_rms_norm_op(mixed.contiguous(), residual, self.post_attention_layernorm.weight,
                                                 self.post_attention_layernorm.eps)
    return residual, self.mlp(normalized)


def chain_ready(core, hidden_states) -> bool:
    """True when every decoder layer of ``core`` runs ``_chain_step`` and the inputs are
    ones the patched layers accept (inference, CUDA, bf16, contiguous)."""
    return (getattr(core, "_fd_residual_chain", False) and not torch.is_grad_enabled() and hidden_states.is_cuda
            and hidden_states.dtype == torch.bfloat16 and hidden_states.is_contiguous())


def install_persistent_residual_rms(core, all_layers: bool = False) -> int:
    """Patch linear-attention decoder layers (or all with ``all_layers``); return the count."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5DecoderLayer
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5DecoderLayer) and (all_layers or module.block_type == "linear_attention"):
            for norm in (module.input_layernorm, module.post_attention_layernorm):
                width = norm.weight.shape[0]
                if width % 8 or not 8 <= width <= 8192:
                    raise ValueError("Fused RMSNorm requires a width that is a multiple of 8 in [8, 8192]")
            if not hasattr(module, "_persistent_original_forward"):
                module._persistent_original_forward = module.forward
                module.forward = MethodType(_forward, module)
                module._fd_chain_step = MethodType(_chain_step, module)
            count += 1
    if all_layers and count:
        core._fd_residual_chain = True
    return count
