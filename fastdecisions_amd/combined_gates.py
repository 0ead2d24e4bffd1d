"""Combined a/b gate projection and the ``fastdecisions::unpack_gate`` op.

Mirrors ref: src/decider/combined_gates.py: ``unpack_gate_op(combined, a_log,
dt_bias) -> (decay, beta)`` over ``unpack_gate`` (ref: :6-16), and
``install_combined_gates(core)`` (ref: :19-43), which snapshots
``cat(in_proj_a.weight, in_proj_b.weight)`` into a non-persistent buffer so the
packed Gated-DeltaNet forward (``fastdecisions_amd.packed_conv._forward``)
computes both gate projections and both transforms in one kernel,
``fastdecisions::gate_proj`` (8, 16, 24 or 32 heads, hidden a multiple of
128), whose rows do not depend on the token count and, with 16 heads, equal
the eager in_proj_a / in_proj_b GEMMs' bit for bit (the kernel sums in the
order hipBLASLt uses for a 16-output projection); other head counts take
one GEMM and the ``unpack_gate`` kernel, as the reference does.  Reinvoke
after changing the projection weights.  Any head count works (the reference
requires two bias-free [16, 2048] projections).

``install_combined_projections(core)`` goes further: all four input
projections of a Gated-DeltaNet layer (q|k|v, z, a, b) become one GEMM whose
output the packed conv, the gated norm and the gate transform read as strided
views (``fastdecisions::gate_transform`` takes a and b as separate views).
"""
from __future__ import annotations

import torch

from .unpack_gate_transform_kernel import gate_projection, gate_transform, unpack_gate


@torch.library.custom_op("fastdecisions::gate_transform", mutates_args=(), device_types="cuda")
def gate_transform_op(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
                      dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return gate_transform(a, b, a_log, dt_bias)


@gate_transform_op.register_fake
def _gate_transform_fake(a, b, a_log, dt_bias):
    return (a.new_empty(a.shape, dtype=torch.float32), a.new_empty(a.shape, dtype=torch.bfloat16))


@torch.library.custom_op("fastdecisions::gate_proj", mutates_args=(), device_types="cuda")
def gate_proj_op(x: torch.Tensor, weight: torch.Tensor, a_log: torch.Tensor,
                 dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return gate_projection(x, weight, a_log, dt_bias)


@gate_proj_op.register_fake
def _gate_proj_fake(x, weight, a_log, dt_bias):
    shape = (*x.shape[:-1], weight.shape[0] // 2)
    return (x.new_empty(shape, dtype=torch.float32), x.new_empty(shape, dtype=torch.bfloat16))


@torch.library.custom_op("fastdecisions::unpack_gate", mutates_args=(), device_types="cuda")
def unpack_gate_op(combined: torch.Tensor, a_log: torch.Tensor,
                   dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return unpack_gate(combined, a_log, dt_bias)


@unpack_gate_op.register_fake
def _fake(combined, a_log, dt_bias):
    shape = (*combined.shape[:-1], combined.shape[-1] // 2)
    return (combined.new_empty(shape, dtype=torch.float32),
            combined.new_empty(shape, dtype=torch.bfloat16))


def install_combined_gates(core) -> int:
    """Snapshot the combined a/b weight of every Gated-DeltaNet layer; return the count."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    from .packed_conv import install_packed_conv
    install_packed_conv(core)
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5GatedDeltaNet):
            a, b = module.in_proj_a, module.in_proj_b
            if (a.weight.shape != b.weight.shape or a.weight.shape[0] != module.num_v_heads
                    or a.bias is not None or b.bias is not None):
                raise ValueError("Combined gates require two bias-free [num_v_heads, hidden] projections")
            with torch.no_grad():
                weight = torch.cat((a.weight, b.weight), dim=0).detach()
            if "_combined_gate_weight" in module._buffers:
                module._combined_gate_weight = weight
            else:
                module.register_buffer("_combined_gate_weight", weight, persistent=False)
            count += 1
    return count


def install_combined_projections(core) -> int:
    """One GEMM for in_proj_qkv | in_proj_z of every Gated-DeltaNet layer, and one
    narrow GEMM for in_proj_a | in_proj_b (non-persistent buffers; reinvoke after
    changing weights).

    The a|b rows stay out of the wide GEMM: at the decider's shapes the 32 extra
    output columns cost hipBLASLt a partial column of 256-wide tiles and a worse
    tiling (M=2048, K=2048 measured on MI355X: N=8224 79.6 us, N=8192 55.3 us, the
    separate N=32 GEMM 6.1 us)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    install_combined_gates(core)
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5GatedDeltaNet):
            projs = (module.in_proj_qkv, module.in_proj_z)
            if any(p.bias is not None for p in projs) or not hasattr(module, "_combined_gate_weight"):
                continue
            with torch.no_grad():
                weight = torch.cat([p.weight for p in projs], dim=0).detach()
                pad = -weight.shape[0] % 8  # zero rows keep the output's row stride a multiple of 8
                if pad:
                    weight = torch.cat([weight, weight.new_zeros((pad, weight.shape[1]))], dim=0)
            if "_fd_in_proj_weight" in module._buffers:
                module._fd_in_proj_weight = weight
            else:
                module.register_buffer("_fd_in_proj_weight", weight, persistent=False)
            count += 1
    return count
