"""``fastdecisions::packed_conv`` torch op and the Gated-DeltaNet patch that uses it.

Mirrors ref: src/decider/packed_conv.py:

* ``packed_conv(x, weight) -> (q, k, v)`` — functional op over ``prep_qkv`` with
  a fake that states the ``[B, T, 16, 128]`` outputs (ref: :12-21);
  ``packed_conv_varlen`` adds ``cu_seqlens`` for packed requests;
* ``_forward`` — replacement ``Qwen3_5GatedDeltaNet.forward`` (ref: :24-62):
  ``in_proj_qkv`` -> packed conv straight into head-split q/k/v -> gates ->
  gated delta rule -> gated RMSNorm -> ``out_proj``; falls back to the original
  method for caches, training, grad, non-CUDA/non-bf16 inputs and other
  geometries (ref: :27-38).  The reference also requires T == 2048; any T works here;
* ``packed_conv_gates(x, weight, hidden_states, gate_weight, a_log, dt_bias,
  cu_seqlens=None) -> (q, k, v, g, beta)`` — the conv and the combined a|b gate
  projection + gate transform in one launch (no counterpart in the reference;
  bit-identical to ``packed_conv`` followed by ``fastdecisions::gate_proj``);
  the patched forward uses it when the combined projections are installed;
* ``install_packed_conv(core)`` — binds it on every ``Qwen3_5GatedDeltaNet``
  and returns the count (ref: :65-75).

With packed requests (``cu_seq_lens_q`` in kwargs) the conv restarts its
window at every request start.  The gated delta rule runs on the HIP kernels
(``fastdecisions::gated_delta_rule``, per-request states from ``cu_seqlens``)
once ``install_gated_delta_rule`` has switched the layer; otherwise it runs
transformers' torch form, which ignores ``cu_seqlens``, once per request
(``fd_segments``, or the boundaries read back from ``cu_seq_lens_q`` when a
caller passes only that), so no state crosses a request boundary either way.
"""
from __future__ import annotations

from types import MethodType

import torch
import torch.nn.functional as F

from .packed_conv_kernel import prep_qkv, prep_qkv_gates


@torch.library.custom_op("fastdecisions::packed_conv", mutates_args=(), device_types="cuda")
def packed_conv(x: torch.Tensor, weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return prep_qkv(x, weight)


@packed_conv.register_fake
def _packed_conv_fake(x, weight):
    batch, seq, channels = x.shape
    shape = (batch, seq, channels // 3 // 128, 128)
    return tuple(x.new_empty(shape) for _ in range(3))


@torch.library.custom_op("fastdecisions::packed_conv_varlen", mutates_args=(), device_types="cuda")
def packed_conv_varlen(x: torch.Tensor, weight: torch.Tensor,
                       cu_seqlens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return prep_qkv(x, weight, cu_seqlens=cu_seqlens)


@packed_conv_varlen.register_fake
def _packed_conv_varlen_fake(x, weight, cu_seqlens):
    batch, seq, channels = x.shape
    shape = (batch, seq, channels // 3 // 128, 128)
    return tuple(x.new_empty(shape) for _ in range(3))


@torch.library.custom_op("fastdecisions::packed_conv_gates", mutates_args=(), device_types="cuda")
def packed_conv_gates(x: torch.Tensor, weight: torch.Tensor, hidden_states: torch.Tensor, gate_weight: torch.Tensor,
                      a_log: torch.Tensor, dt_bias: torch.Tensor,
                      cu_seqlens: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                      torch.Tensor, torch.Tensor]:
    """``packed_conv`` and ``fastdecisions::gate_proj`` of one layer in one launch."""
    return prep_qkv_gates(x, weight, hidden_states, gate_weight, a_log, dt_bias, cu_seqlens=cu_seqlens)


@packed_conv_gates.register_fake
def _packed_conv_gates_fake(x, weight, hidden_states, gate_weight, a_log, dt_bias, cu_seqlens=None):
    batch, seq, channels = x.shape
    shape = (batch, seq, channels // 3 // 128, 128)
    gates = (batch, seq, gate_weight.shape[0] // 2)
    return (*(x.new_empty(shape) for _ in range(3)), x.new_empty(gates, dtype=torch.float32),
            x.new_empty(gates, dtype=torch.bfloat16))


def _segments(kwargs):
    """Host-side request boundaries of a packed batch (a list of (start, end)), or None.

    They come from ``fd_segments`` when the caller passes them (the decider model
    does, so graph capture never synchronises); a caller that passes only
    ``cu_seq_lens_q`` gets them from one device-to-host copy of it, so the torch
    delta rule below still runs once per request."""
    bounds = kwargs.get("fd_segments")
    if bounds is not None:
        return list(bounds)
    cu = kwargs.get("cu_seq_lens_q")
    if cu is None:
        return None
    c = [int(v) for v in cu.tolist()]
    return list(zip(c[:-1], c[1:]))


def _gate_proj_fits(self, hidden_states) -> bool:
    """Sizes the fused a|b projection + gate transform kernel takes."""
    return (self.num_v_heads in (8, 16, 24, 32) and hidden_states.shape[-1] % 128 == 0
            and hidden_states.stride(-1) == 1 and hidden_states.is_contiguous())


def _eager_layout(query, key, value):
    """q, k, v [B, T, H, D] as the views the eager layer hands transformers' delta rule: slices of
    the [B, C, T] conv output transposed back.  The values are the same; the rule's l2norm of q and
    k reduces over D in an order PyTorch picks from the layout, and only in this layout is it eager's."""
    b, t = query.shape[:2]
    mixed = torch.cat([query.reshape(b, t, -1), key.reshape(b, t, -1), value.reshape(b, t, -1)], dim=-1)
    mixed = mixed.transpose(1, 2).contiguous().transpose(1, 2)
    dk, dv = key.shape[2] * key.shape[3], value.shape[2] * value.shape[3]
    q, k, v = torch.split(mixed, [dk, dk, dv], dim=-1)
    return (q.reshape(b, t, -1, query.shape[3]), k.reshape(b, t, -1, key.shape[3]),
            v.reshape(b, t, -1, value.shape[3]))


def _forward(self, hidden_states, cache_params=None, attention_mask=None, **kwargs):
    # The original method owns caches, training and other geometries (ref: src/decider/packed_conv.py:25-38).
    if (cache_params is not None or self.training or torch.is_grad_enabled()
            or not hidden_states.is_cuda or hidden_states.dtype != torch.bfloat16
            or self.key_dim != self.value_dim or self.num_k_heads != self.num_v_heads
            or self.head_k_dim != 128 or self.head_v_dim != 128
            or self.conv1d.weight.shape != (3 * self.key_dim, 1, self.conv_kernel_size)
            or not 1 <= self.conv_kernel_size <= 4
            or self.conv1d.bias is not None or self.activation != "silu"):
        return self._packed_original_forward(hidden_states, cache_params=cache_params,
                                             attention_mask=attention_mask, **kwargs)

    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    hidden_states = mq.apply_mask_to_padding_states(hidden_states, attention_mask)
    batch, seq, _ = hidden_states.shape
    combined = hasattr(self, "_fd_in_proj_weight")
    if combined:
        # q|k|v and z from one GEMM, read below as strided views; a|b from its own
        proj = F.linear(hidden_states, self._fd_in_proj_weight)
        c0 = 2 * self.key_dim + self.value_dim
        c1 = c0 + self.value_dim
        mixed = proj[..., :c0]
    else:
        mixed = self.in_proj_qkv(hidden_states)
    cu_seqlens = kwargs.get("cu_seq_lens_q")
    fused_gates = combined and _gate_proj_fits(self, hidden_states)
    if fused_gates:
        # the conv and the a|b projection + gate transform in one launch
        query, key, value, g, beta = packed_conv_gates(mixed, self.conv1d.weight, hidden_states,
                                                       self._combined_gate_weight, self.A_log, self.dt_bias,
                                                       cu_seqlens)
    elif cu_seqlens is not None:
        query, key, value = packed_conv_varlen(mixed, self.conv1d.weight, cu_seqlens)
    else:
        query, key, value = packed_conv(mixed, self.conv1d.weight)
    if combined:
        z = proj[..., c0:c1].view(batch, seq, -1, self.head_v_dim)
        if not fused_gates:
            from .combined_gates import unpack_gate_op
            ab = F.linear(hidden_states, self._combined_gate_weight)
            g, beta = unpack_gate_op(ab, self.A_log, self.dt_bias)
    elif hasattr(self, "_combined_gate_weight"):
        z = self.in_proj_z(hidden_states).reshape(batch, seq, -1, self.head_v_dim)
        if _gate_proj_fits(self, hidden_states):
            # both gate projections and both transforms in one kernel whose rows do not depend on
            # the token count (a library GEMM of this small N picks its reduction split by M)
            from .combined_gates import gate_proj_op
            g, beta = gate_proj_op(hidden_states, self._combined_gate_weight, self.A_log, self.dt_bias)
        else:
            # one GEMM for both gate projections, one kernel for both transforms (ref: :45-48)
            from .combined_gates import unpack_gate_op
            ab = F.linear(hidden_states, self._combined_gate_weight)
            g, beta = unpack_gate_op(ab, self.A_log, self.dt_bias)
    else:
        z = self.in_proj_z(hidden_states).reshape(batch, seq, -1, self.head_v_dim)
        b = self.in_proj_b(hidden_states)
        a = self.in_proj_a(hidden_states)
        beta = b.sigmoid()
        g = -self.A_log.float().exp() * F.softplus(a.float() + self.dt_bias)
    if getattr(self, "_fd_gated_delta", False) and getattr(self, "_fd_gated_norm", False):
        # the delta rule and the gated RMSNorm in one library call (one kernel sequence)
        from .gated_delta import gated_delta_rule_norm
        core_attn_out = gated_delta_rule_norm(query, key, value, g, beta, z, self.norm.weight,
                                              float(self.norm.variance_epsilon), cu_seqlens)
        return self.out_proj(core_attn_out.reshape(batch, seq, -1))
    segments = None if getattr(self, "_fd_gated_delta", False) else _segments(kwargs)
    if not getattr(self, "_fd_gated_delta", False):
        query, key, value = _eager_layout(query, key, value)
    if getattr(self, "_fd_gated_delta", False):
        from .gated_delta import gated_delta_rule
        core_attn_out = gated_delta_rule(query, key, value, g, beta, cu_seqlens)
    elif segments is None:
        core_attn_out, _ = mq.torch_chunk_gated_delta_rule(
            query, key, value, g=g, beta=beta, initial_state=None, output_final_state=False,
            use_qk_l2norm_in_kernel=True)
    else:
        parts = []
        for s, e in segments:
            if e > s:
                out, _ = mq.torch_chunk_gated_delta_rule(
                    query[:, s:e], key[:, s:e], value[:, s:e], g=g[:, s:e], beta=beta[:, s:e],
                    initial_state=None, output_final_state=False, use_qk_l2norm_in_kernel=True)
                parts.append(out)
        core_attn_out = torch.cat(parts, dim=1)
    if getattr(self, "_fd_gated_norm", False):
        from .layer_fusions import gated_rms_norm_op
        core_attn_out = gated_rms_norm_op(core_attn_out.reshape(-1, self.head_v_dim), z, self.norm.weight,
                                          float(self.norm.variance_epsilon))
    else:
        core_attn_out = self.norm(core_attn_out.reshape(-1, self.head_v_dim),
                                  z.reshape(-1, self.head_v_dim))
    return self.out_proj(core_attn_out.reshape(batch, seq, -1))


def install_packed_conv(core) -> int:
    """Patch this model's Gated-DeltaNet modules only; return the number installed (ref: :65-75)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5GatedDeltaNet):
            if not hasattr(module, "_packed_original_forward"):
                module._packed_original_forward = module.forward
                module.forward = MethodType(_forward, module)
            count += 1
    return count
