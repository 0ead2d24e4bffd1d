"""Fusions on the decider forward around the hot-path kernels.

* ``fastdecisions::gated_rms_norm`` — the Gated-DeltaNet output norm
  (``Qwen3_5RMSNormGated``) in one kernel; ``install_gated_norm(core)`` makes the
  packed Gated-DeltaNet forward use it (``fastdecisions_amd.packed_conv._forward``);
* ``fastdecisions::silu_mul`` and ``install_mlp_fusion(core)`` — every
  ``Qwen3_5MLP`` computes gate and up with one GEMM on the concatenated weight
  (a non-persistent buffer, refreshed by reinstalling) and ``silu(gate) * up``
  in one kernel; unsupported calls (grad, training, non-CUDA, non-bf16) run
  the original forward.  With an intermediate size above 4096 the GEMM runs as
  two, on [gate[:4096]; up[:4096]] and [gate[4096:]; up[4096:]]
  (``fastdecisions::silu_mul_split`` joins them): at 2048 tokens hipBLASLt
  tiles an 8192-wide output better than a 12288-wide one.
"""
from __future__ import annotations

from types import MethodType

import torch
import torch.nn.functional as F

from .gated_norm_kernel import gated_rms_norm, silu_mul, silu_mul_split


@torch.library.custom_op("fastdecisions::gated_rms_norm", mutates_args=(), device_types="cuda")
def gated_rms_norm_op(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return gated_rms_norm(x, gate, weight, eps)


@gated_rms_norm_op.register_fake
def _gated_rms_norm_fake(x, gate, weight, eps):
    return x.new_empty(x.shape)


@torch.library.custom_op("fastdecisions::silu_mul", mutates_args=(), device_types="cuda")
def silu_mul_op(gate_up: torch.Tensor) -> torch.Tensor:
    return silu_mul(gate_up)


@silu_mul_op.register_fake
def _silu_mul_fake(gate_up):
    return gate_up.new_empty((*gate_up.shape[:-1], gate_up.shape[-1] // 2))


@torch.library.custom_op("fastdecisions::silu_mul_split", mutates_args=(), device_types="cuda")
def silu_mul_split_op(gate_up1: torch.Tensor, gate_up2: torch.Tensor) -> torch.Tensor:
    return silu_mul_split(gate_up1, gate_up2)


@silu_mul_split_op.register_fake
def _silu_mul_split_fake(gate_up1, gate_up2):
    return gate_up1.new_empty((*gate_up1.shape[:-1], (gate_up1.shape[-1] + gate_up2.shape[-1]) // 2))


# Gate|up split point: the first GEMM takes this many gate and up features (8192 outputs).
_MLP_SPLIT = 4096


def install_gated_norm(core) -> int:
    """Run every Gated-DeltaNet layer's output norm in one kernel; return the count."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    from .packed_conv import install_packed_conv
    install_packed_conv(core)
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5GatedDeltaNet) and module.head_v_dim in (64, 128, 256):
            module._fd_gated_norm = True
            count += 1
    return count


def _mlp_forward(self, x):
    if (self.training or torch.is_grad_enabled() or not x.is_cuda or x.dtype != torch.bfloat16
            or self._fd_gate_up_weight.dtype != torch.bfloat16):
        return self._fd_mlp_original_forward(x)
    if self._fd_gate_up_weight2 is not None:
        h = silu_mul_split_op(F.linear(x, self._fd_gate_up_weight), F.linear(x, self._fd_gate_up_weight2))
        return self.down_proj(h)
    return self.down_proj(silu_mul_op(F.linear(x, self._fd_gate_up_weight)))


def install_mlp_fusion(core) -> int:
    """Combined gate|up GEMM + fused SiLU gate for every Qwen3_5MLP; return the count."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5MLP
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5MLP):
            if (module.gate_proj.bias is not None or module.up_proj.bias is not None
                    or module.config.hidden_act not in ("silu", "swish") or module.intermediate_size % 8):
                continue
            gate, up = module.gate_proj.weight, module.up_proj.weight
            n = module.intermediate_size
            with torch.no_grad():
                if n > _MLP_SPLIT and (n - _MLP_SPLIT) % 8 == 0:
                    weight = torch.cat((gate[:_MLP_SPLIT], up[:_MLP_SPLIT]), dim=0).detach()
                    weight2 = torch.cat((gate[_MLP_SPLIT:], up[_MLP_SPLIT:]), dim=0).detach()
                else:
                    weight, weight2 = torch.cat((gate, up), dim=0).detach(), None
            for name, value in (("_fd_gate_up_weight", weight), ("_fd_gate_up_weight2", weight2)):
                if name in module._buffers:
                    setattr(module, name, value)
                else:
                    module.register_buffer(name, value, persistent=False)
            if not hasattr(module, "_fd_mlp_original_forward"):
                module._fd_mlp_original_forward = module.forward
                module.forward = MethodType(_mlp_forward, module)
            count += 1
    return count
