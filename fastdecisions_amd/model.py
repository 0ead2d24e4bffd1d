"""Synthetic decider-2b-shaped hybrid model and its forward.

The real decider-2b checkpoint is fetched from the Hub by the reference
(ref: src/decider/model.py:12-13) and is not available offline, so the model
is built from transformers' Qwen3.5 text modules — the modules the reference
patches — with seeded random weights:

* hidden 2048, 28 layers; ``layer_types`` every 4th layer full attention
  (layers 3, 7, ..., 27: 7 GQA + 21 Gated-DeltaNet, the 3:1 interleave);
* GQA layers 16 query / 4 KV heads x 128 (q_proj emits q || gate), q/k RMSNorm,
  partial RoPE 0.25; Gated-DeltaNet layers 16 key / 16 value heads x 128, conv 4;
* MLP intermediate 6144 (not fixed by the reference config; stated here),
  vocabulary 65536, rope_theta 1e7, RMSNorm eps 1e-6;
* weights: every linear / embedding / conv weight ~ N(0, 0.02); offset-form
  RMSNorm weights (gain 1 + w) ~ N(0, 0.02); gated-norm weights 1 + 0.02 N(0, 1);
  A_log = log U(1, 16); dt_bias = 1; 10 letter rows ~ N(0, 0.02) stand for the
  option-letter rows of the LM head (ref: src/decider/model.py:14-16, A..J as
  ref: src/decider/prompt.py:10-12).

``DeciderModel.forward(ids)`` returns letter logits ``[B, T, K]`` in fp32, as the
reference engine's ``_fwd_eager`` (ref: src/decider/engine.py:115-117).  With
``cu_seqlens`` the rows of one ``[1, T]`` batch are packed requests: positions
restart per request and the patched layers keep requests apart.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch
import torch.nn.functional as F
from torch import nn


@dataclass(frozen=True)
class DeciderShape:
    vocab_size: int = 65536
    hidden_size: int = 2048
    intermediate_size: int = 6144
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 128
    linear_num_heads: int = 16
    linear_head_dim: int = 128
    conv_kernel: int = 4
    full_attention_interval: int = 4
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10_000_000.0
    partial_rotary_factor: float = 0.25
    n_letters: int = 10


DECIDER_2B_SHAPED = DeciderShape()
# A few-layer shape that keeps every decider geometry the kernels care about
# (head dims 128, 16 linear heads, 16/4 GQA heads) for fast GPU tests.
DECIDER_4_LAYERS = replace(DECIDER_2B_SHAPED, num_hidden_layers=4, vocab_size=4096)
# A small CPU-friendly shape for host-side tests.
TINY = DeciderShape(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                    num_attention_heads=4, num_key_value_heads=1, head_dim=64, linear_num_heads=2,
                    linear_head_dim=128)


def make_config(shape: DeciderShape = DECIDER_2B_SHAPED, attn_implementation: str = "sdpa"):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(
        vocab_size=shape.vocab_size, hidden_size=shape.hidden_size, intermediate_size=shape.intermediate_size,
        num_hidden_layers=shape.num_hidden_layers, num_attention_heads=shape.num_attention_heads,
        num_key_value_heads=shape.num_key_value_heads, head_dim=shape.head_dim,
        linear_num_key_heads=shape.linear_num_heads, linear_num_value_heads=shape.linear_num_heads,
        linear_key_head_dim=shape.linear_head_dim, linear_value_head_dim=shape.linear_head_dim,
        linear_conv_kernel_dim=shape.conv_kernel, rms_norm_eps=shape.rms_norm_eps,
        full_attention_interval=shape.full_attention_interval, max_position_embeddings=32768,
        rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta,
                         "partial_rotary_factor": shape.partial_rotary_factor, "mrope_section": [11, 11, 10]},
        use_cache=False,
    )
    cfg._attn_implementation = attn_implementation
    return cfg


class DeciderModel(nn.Module):
    """Qwen3.5 text stack + option-letter rows; ``forward`` -> letter logits [B, T, K] (fp32)."""

    def __init__(self, shape: DeciderShape = DECIDER_2B_SHAPED, attn_implementation: str = "sdpa"):
        super().__init__()
        from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel
        self.shape = shape
        self.config = make_config(shape, attn_implementation)
        self.core = Qwen3_5TextModel(self.config)
        self.letters = nn.Parameter(torch.empty(shape.n_letters, shape.hidden_size))

    def hidden(self, ids: torch.Tensor, *, cu_seqlens: torch.Tensor | None = None,
               segments: list[tuple[int, int]] | None = None, max_seqlen: int | None = None,
               final_norm: bool = True) -> torch.Tensor:
        """Final normed hidden states [B, T, H] (the residual stream before the final
        norm with ``final_norm=False``).  For packed requests pass ``cu_seqlens``
        (device int32), ``segments`` (host (start, end) pairs) and ``max_seqlen``."""
        core = self.core
        h = core.embed_tokens(ids)
        B, T = ids.shape
        kwargs = {}
        if cu_seqlens is None:
            pos = torch.arange(T, device=ids.device)[None].expand(B, T)
        else:
            if B != 1 or segments is None or max_seqlen is None:
                raise ValueError("packed requests need B == 1, cu_seqlens, segments and max_seqlen")
            pos = torch.cat([torch.arange(e - s, device=ids.device) for s, e in segments])[None]
            kwargs = dict(cu_seq_lens_q=cu_seqlens, cu_seq_lens_k=cu_seqlens, max_length_q=int(max_seqlen),
                          max_length_k=int(max_seqlen), fd_segments=tuple(segments))
        pe = core.rotary_emb(h, pos)
        layers = core.layers[: self.config.num_hidden_layers]
        from .persistent_residual_rms import chain_ready, fused_add_rms_norm_op
        if len(layers) and chain_ready(core, h):
            # every layer patched: each MLP residual add runs inside the next RMSNorm kernel
            residual, delta = h, None
            for layer in layers:
                residual, delta = layer._fd_chain_step(residual, delta, position_embeddings=pe, attention_mask=None,
                                                       position_ids=pos, **kwargs)
            if final_norm:
                return fused_add_rms_norm_op(delta, residual, core.norm.weight, core.norm.eps)[0]
            return residual + delta
        for layer in layers:
            h = layer(h, position_embeddings=pe, attention_mask=None, position_ids=pos, past_key_values=None,
                      **kwargs)
        return core.norm(h) if final_norm else h

    def forward(self, ids: torch.Tensor, **kw) -> torch.Tensor:
        return F.linear(self.hidden(ids, **kw), self.letters).float()

    def slot_logits(self, ids: torch.Tensor, slot_rows: torch.Tensor, slot_positions: torch.Tensor,
                    nopts: torch.Tensor | None = None, temperature: float = 1.0, **kw):
        """Letter logits [N, K] (fp32) and masked probabilities at the slots only: the
        layers run on every token, the final norm and the projection only at the
        slots (fd_slot_readout_fwd; ref: src/decider/slot_projection.py:6-21)."""
        from .slot_projection import slot_readout
        h = self.hidden(ids, final_norm=False, **kw)
        return slot_readout(h.contiguous(), self.core.norm.weight, self.letters, slot_rows, slot_positions, nopts,
                            eps=self.core.norm.eps, temperature=temperature)


def _init_value(name: str, shape, gen: torch.Generator, device) -> torch.Tensor:
    def normal(std):
        return torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std
    if name.endswith("A_log"):
        return torch.empty(shape, device=device, dtype=torch.float32).uniform_(1.0, 16.0, generator=gen).log_()
    if name.endswith("dt_bias"):
        return torch.ones(shape, device=device, dtype=torch.float32)
    if name.endswith("linear_attn.norm.weight"):  # Qwen3_5RMSNormGated: plain gain
        return 1.0 + normal(0.02)
    return normal(0.02)  # linear / embedding / conv weights and offset-form RMSNorm weights


@torch.no_grad()
def build_decider(shape: DeciderShape = DECIDER_2B_SHAPED, seed: int = 0, device="cuda",
                  dtype=torch.bfloat16, attn_implementation: str = "sdpa") -> DeciderModel:
    """Seeded random-init decider on ``device``.  Parameters are drawn in
    ``named_parameters`` order from one generator on ``device``.  The model's
    reference PyTorch path computes the causal conv as BASELINE config 2 defines
    it (``engine.patch_conv``, which this calls, as the reference's engine does
    before it builds its model, ref: src/decider/engine.py:86-90)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding
    from .engine import patch_conv
    patch_conv()
    device = torch.device(device)
    with torch.device("meta"):
        model = DeciderModel(shape, attn_implementation)
    model = model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    for name, p in model.named_parameters():
        p.copy_(_init_value(name, p.shape, gen, device).to(p.dtype))
    model = model.to(dtype)
    # RoPE frequencies stay fp32 (a fresh module, built after the dtype cast)
    model.core.rotary_emb = Qwen3_5TextRotaryEmbedding(model.config).to(device)
    return model.eval()


# Install levels, each adding to the one before:
#   north_star           the reference's three patches: packed conv (Gated-DeltaNet layers, delta rule
#                        still transformers' torch form), native GQA (attention layers), residual add +
#                        RMSNorm (linear-attention decoder layers)
#   residual_chain       add+RMSNorm in every decoder layer, each MLP residual add inside the next norm
#   gated_delta          the chunked gated-delta rule on the HIP kernels
#   combined_gates       both gate projections and the gate transform in one kernel (fd_gate_proj_fwd;
#                        one GEMM + the transform kernel for head counts it does not take)
#   gated_norm           the delta rule's gated RMSNorm in the delta-rule launch sequence
#   attention_fusions    q/k RMSNorm + RoPE prologue, gated GQA store, q|gate|k|v as one GEMM
#   combined_projections q|k|v|z as one GEMM, conv + a|b projection + gate transform in one launch
#   mlp_fusion           gate|up as two GEMMs + one SiLU*mul kernel
INSTALL_LEVELS = ("north_star", "residual_chain", "gated_delta", "combined_gates", "gated_norm",
                  "attention_fusions", "combined_projections", "mlp_fusion")


def install_hip_kernels(model: DeciderModel, level: str = INSTALL_LEVELS[-1]) -> dict:
    """Route the hot ops of every layer to the HIP kernels, up to and including ``level``
    (one of ``INSTALL_LEVELS``; the default installs everything); returns per-step patch counts.
    Installing a later level onto a model installed at an earlier one adds the missing steps."""
    from .combined_gates import install_combined_gates, install_combined_projections
    from .gated_delta import install_gated_delta_rule
    from .layer_fusions import install_gated_norm, install_mlp_fusion
    from .native_gqa import install_attention_fusions, install_native_gqa
    from .packed_conv import install_packed_conv
    from .persistent_residual_rms import install_persistent_residual_rms
    if level not in INSTALL_LEVELS:
        raise ValueError(f"level must be one of {INSTALL_LEVELS} (got {level!r})")
    core = model.core
    steps = dict(
        north_star=lambda: dict(packed_conv=install_packed_conv(core), native_gqa=install_native_gqa(core),
                                residual_rms=install_persistent_residual_rms(core)),
        residual_chain=lambda: dict(residual_rms_all_layers=install_persistent_residual_rms(core, all_layers=True)),
        gated_delta=lambda: dict(gated_delta=install_gated_delta_rule(core)),
        combined_gates=lambda: dict(combined_gates=install_combined_gates(core)),
        gated_norm=lambda: dict(gated_norm=install_gated_norm(core)),
        attention_fusions=lambda: dict(attention_fusions=install_attention_fusions(core)),
        combined_projections=lambda: dict(combined_projections=install_combined_projections(core)),
        mlp_fusion=lambda: dict(mlp_fusion=install_mlp_fusion(core)))
    counts = {}
    for name in INSTALL_LEVELS[:INSTALL_LEVELS.index(level) + 1]:
        counts.update(steps[name]())
    return counts


def synthetic_ids(batch: int, seq_len: int, vocab: int, seed: int, device="cuda") -> torch.Tensor:
    """Token ids uniform over the vocabulary, drawn on the CPU for portability."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (batch, seq_len), generator=g).to(device)
