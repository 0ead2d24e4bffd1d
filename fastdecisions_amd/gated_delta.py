"""``fastdecisions::gated_delta_rule`` torch op and its installer.

The op wraps ``chunk_gated_delta_rule`` in the form the decider's Gated-DeltaNet
forward calls it (ref: src/decider/packed_conv.py:55-59: q/k l2-normalised in the
kernel, no initial state, no final state), plus ``cu_seqlens`` for packed
requests.  ``install_gated_delta_rule(core)`` makes the packed Gated-DeltaNet
forward (``fastdecisions_amd.packed_conv._forward``, installed here when it is
not there yet) run the delta rule on the HIP kernels instead of transformers'
torch loop; it returns the number of layers switched.
"""
from __future__ import annotations

from typing import Optional

import torch

from .gated_delta_kernel import chunk_gated_delta_rule


@torch.library.custom_op("fastdecisions::gated_delta_rule", mutates_args=(), device_types="cuda")
def gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                     cu_seqlens: Optional[torch.Tensor]) -> torch.Tensor:
    out, _ = chunk_gated_delta_rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_seqlens)
    return out


@gated_delta_rule.register_fake
def _gated_delta_rule_fake(q, k, v, g, beta, cu_seqlens):
    return v.new_empty(v.shape)


@torch.library.custom_op("fastdecisions::gated_delta_rule_norm", mutates_args=(), device_types="cuda")
def gated_delta_rule_norm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                          z: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                          cu_seqlens: Optional[torch.Tensor]) -> torch.Tensor:
    """The delta rule followed by the layer's gated RMSNorm in one call of the library
    (``self.norm(core_attn_out, z)``, ref: src/decider/packed_conv.py:60-61)."""
    out, _ = chunk_gated_delta_rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_seqlens,
                                    norm=(z, norm_weight, eps))
    return out


@gated_delta_rule_norm.register_fake
def _gated_delta_rule_norm_fake(q, k, v, g, beta, z, norm_weight, eps, cu_seqlens):
    return v.new_empty(v.shape)


def install_gated_delta_rule(core) -> int:
    """Run every Gated-DeltaNet layer's delta rule on the HIP kernels; return the count."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet
    from .packed_conv import install_packed_conv
    install_packed_conv(core)
    count = 0
    for module in core.modules():
        if isinstance(module, Qwen3_5GatedDeltaNet):
            module._fd_gated_delta = True
            count += 1
    return count
