"""``fastdecisions::native_gqa`` torch op and the attention-layer patch that uses it.

The reference defines this op and its patched ``Qwen3_5Attention.forward``
inside its model benchmark (ref: experiments/native_gqa/bench_native_gqa_model.py:34-56);
here they are part of the package:

* ``native_gqa`` — functional op ``(q, k, v) -> out`` over the HIP kernel, with a
  fake implementation that states the permuted ``[B, T, H, D]`` output
  (ref: :38-41), so it is one node under ``torch.compile`` and capturable in a
  HIP graph;
* ``native_gqa_varlen`` — the same over packed requests (``cu_seqlens``);
* ``install_native_gqa(core)`` — binds ``candidate_forward`` on every
  ``Qwen3_5Attention`` of a model and returns the count.  Unsupported calls
  (KV cache, training, grad, non-CUDA, non-bf16, an ``attention_mask`` that is
  not plain causal) fall back to the original forward, as the other install
  patches of the reference do (ref: src/decider/packed_conv.py:27-38); the
  reference checks the masks once, in eager execution, before it swaps the
  kernel in (ref: experiments/native_gqa/bench_native_gqa_model.py:84-107);
* ``attn_prologue`` / ``native_gqa_gated`` — the attention layer's prologue
  (q/k RMSNorm + partial RoPE, one kernel) and the attention with its sigmoid
  output gate applied in the store; ``install_attention_fusions(core)``
  switches ``candidate_forward`` to them (q/k/v projections and o_proj stay
  library GEMMs).
"""
from __future__ import annotations

from types import MethodType

import torch
import torch.nn.functional as F

from typing import Optional

from .attention_prologue_kernel import attention_prologue
from .native_gqa_kernel import native_gqa_attention


@torch.library.custom_op("fastdecisions::native_gqa", mutates_args=(), device_types="cuda")
def native_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    return native_gqa_attention(q, k, v)


@native_gqa.register_fake
def _native_gqa_fake(q, k, v):
    b, h, t, d = q.shape
    return q.new_empty((b, t, h, d)).permute(0, 2, 1, 3)


@torch.library.custom_op("fastdecisions::native_gqa_varlen", mutates_args=(), device_types="cuda")
def native_gqa_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                      max_seqlen: int) -> torch.Tensor:
    return native_gqa_attention(q, k, v, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


@native_gqa_varlen.register_fake
def _native_gqa_varlen_fake(q, k, v, cu_seqlens, max_seqlen):
    b, h, t, d = q.shape
    return q.new_empty((b, t, h, d)).permute(0, 2, 1, 3)


@torch.library.custom_op("fastdecisions::attn_prologue", mutates_args=(), device_types="cuda")
def attn_prologue(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                  cos: torch.Tensor, sin: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return attention_prologue(q, k, q_weight, k_weight, cos, sin, eps)


@attn_prologue.register_fake
def _attn_prologue_fake(q, k, q_weight, k_weight, cos, sin, eps):
    return q.new_empty(q.shape), k.new_empty(k.shape)


@torch.library.custom_op("fastdecisions::native_gqa_gated", mutates_args=(), device_types="cuda")
def native_gqa_gated(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor,
                     cu_seqlens: Optional[torch.Tensor], max_seqlen: int) -> torch.Tensor:
    if cu_seqlens is None:
        return native_gqa_attention(q, k, v, gate=gate)
    return native_gqa_attention(q, k, v, gate=gate, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)


@native_gqa_gated.register_fake
def _native_gqa_gated_fake(q, k, v, gate, cu_seqlens, max_seqlen):
    b, h, t, d = q.shape
    return q.new_empty((b, t, h, d)).permute(0, 2, 1, 3)


def _fusable(self, position_embeddings) -> bool:
    cos, sin = position_embeddings
    return (self.head_dim == 128 and self.q_norm.eps == self.k_norm.eps
            and self.q_norm.weight.dtype == self.k_norm.weight.dtype
            and self.q_norm.weight.dtype in (torch.bfloat16, torch.float32)
            and cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16 and cos.ndim == 3
            and cos.shape[-1] in (16, 32, 64, 128))


def _fused_forward(self, hidden_states, position_embeddings, cu_seqlens, max_seqlen):
    """The attention layer with its prologue and output gate in HIP kernels."""
    shape = hidden_states.shape[:-1]
    d = self.head_dim
    if hasattr(self, "_fd_qkv_weight"):
        # q|gate, k, v from one GEMM, read as strided views
        proj = F.linear(hidden_states, self._fd_qkv_weight)
        nq = self.q_proj.weight.shape[0]
        nk = self.k_proj.weight.shape[0]
        qg = proj[..., :nq].view(*shape, -1, 2 * d)
        kp = proj[..., nq:nq + nk].view(*shape, -1, d)
        v = proj[..., nq + nk:].view(*shape, -1, d).transpose(1, 2)
    else:
        qg = self.q_proj(hidden_states).view(*shape, -1, 2 * d)   # per head: query | gate
        kp = self.k_proj(hidden_states).view(*shape, -1, d)
        v = self.v_proj(hidden_states).view(*shape, -1, d).transpose(1, 2)
    cos, sin = position_embeddings
    q, k = attn_prologue(qg[..., :d], kp, self.q_norm.weight, self.k_norm.weight, cos.contiguous(),
                         sin.contiguous(), float(self.q_norm.eps))
    out = native_gqa_gated(q.transpose(1, 2), k.transpose(1, 2), v, qg[..., d:].transpose(1, 2), cu_seqlens,
                           int(max_seqlen))
    return self.o_proj(out.transpose(1, 2).reshape(*shape, -1)), None


def plain_causal(mask, t: int) -> bool:
    """True when ``mask`` adds nothing to the in-kernel causal mask over ``t`` tokens: None, a boolean
    mask equal to the lower triangle, or an additive mask that is 0 on and below the diagonal and
    below -1e4 above it (the checks of ref: experiments/native_gqa/bench_native_gqa_model.py:84-99).
    A tensor mask is read back to the host, so during graph capture (where that is not allowed)
    it counts as not plain and the caller falls back to the original forward."""
    if mask is None:
        return True
    if not isinstance(mask, torch.Tensor) or mask.ndim < 2 or tuple(mask.shape[-2:]) != (t, t):
        return False
    if mask.is_cuda and torch.cuda.is_current_stream_capturing():
        return False
    allowed = torch.ones((t, t), device=mask.device, dtype=torch.bool).tril()
    if mask.dtype == torch.bool:
        return bool(torch.equal(mask, allowed.expand_as(mask)))
    if not mask.is_floating_point():
        return False
    return bool((mask[..., allowed] == 0).all().item()) and bool((mask[..., ~allowed] < -1e4).all().item())


def candidate_forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None,
                      **kwargs):
    """Qwen3_5Attention.forward with the attention itself on the HIP kernel
    (ref: experiments/native_gqa/bench_native_gqa_model.py:43-56).  The causal
    mask is applied in-kernel, so the kernel runs only when ``attention_mask`` adds
    nothing to it (``plain_causal``); any other mask (padding, segments, a bias)
    runs the original forward, which applies it."""
    if (past_key_values is not None or self.training or torch.is_grad_enabled()
            or not hidden_states.is_cuda or hidden_states.dtype != torch.bfloat16
            or self.head_dim not in (64, 128, 256)
            or not plain_causal(attention_mask, hidden_states.shape[1])):
        return self._native_gqa_original_forward(hidden_states, position_embeddings, attention_mask,
                                                 past_key_values=past_key_values, **kwargs)
    cu_seqlens = kwargs.get("cu_seq_lens_q")
    if getattr(self, "_fd_attn_fused", False) and _fusable(self, position_embeddings):
        max_len = kwargs["max_length_q"] if cu_seqlens is not None else hidden_states.shape[1]
        return _fused_forward(self, hidden_states, position_embeddings, cu_seqlens, max_len)
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb
    shape = hidden_states.shape[:-1]
    heads_shape = (*shape, -1, self.head_dim)
    q, gate = torch.chunk(self.q_proj(hidden_states).view(*shape, -1, self.head_dim * 2), 2, dim=-1)
    gate = gate.reshape(*shape, -1)
    q = self.q_norm(q.reshape(heads_shape)).transpose(1, 2)
    k = self.k_norm(self.k_proj(hidden_states).view(heads_shape)).transpose(1, 2)
    v = self.v_proj(hidden_states).view(heads_shape).transpose(1, 2)
    q, k = apply_rotary_pos_emb(q, k, *position_embeddings)
    if cu_seqlens is not None:
        out = native_gqa_varlen(q, k, v, cu_seqlens, int(kwargs["max_length_q"]))
    else:
        out = native_gqa(q, k, v)
    out = out.transpose(1, 2).reshape(*shape, -1)
    return self.o_proj(out * torch.sigmoid(gate)), None


def install_native_gqa(core) -> int:
    """Patch every Qwen3_5Attention of this model instance; return the number patched."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5Attention
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5Attention):
            if not hasattr(module, "_native_gqa_original_forward"):
                module._native_gqa_original_forward = module.forward
                module.forward = MethodType(candidate_forward, module)
            count += 1
    return count


def install_attention_fusions(core) -> int:
    """Run every attention layer's prologue and output gate in HIP kernels, with q|gate,
    k and v from one GEMM on the concatenated weight (a non-persistent buffer; reinvoke
    after changing weights); return the count.  Installs ``candidate_forward`` where it is
    not there yet."""
    install_native_gqa(core)
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5Attention
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5Attention):
            module._fd_attn_fused = True
            projs = (module.q_proj, module.k_proj, module.v_proj)
            if all(p.bias is None for p in projs):
                with torch.no_grad():
                    weight = torch.cat([p.weight for p in projs], dim=0).detach()
                if "_fd_qkv_weight" in module._buffers:
                    module._fd_qkv_weight = weight
                else:
                    module.register_buffer("_fd_qkv_weight", weight, persistent=False)
            count += 1
    return count
