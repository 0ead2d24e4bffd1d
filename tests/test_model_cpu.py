"""CPU tests of the host side: the synthetic decider, the install patches' fallbacks,
the workloads and the slot readout."""
from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def tiny():
    from fastdecisions_amd.model import TINY, build_decider
    return build_decider(TINY, seed=0, device="cpu", dtype=torch.float32)


def test_forward_matches_transformers_own_forward(tiny):
    from fastdecisions_amd.model import synthetic_ids
    ids = synthetic_ids(2, 50, tiny.shape.vocab_size, seed=3, device="cpu")
    with torch.no_grad():
        ours = tiny.hidden(ids)
        theirs = tiny.core(input_ids=ids, use_cache=False).last_hidden_state
    assert torch.equal(ours, theirs)


def test_layer_interleave_and_parameter_init(tiny):
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, make_config
    cfg = make_config(DECIDER_2B_SHAPED)
    assert cfg.layer_types.count("full_attention") == 7 and cfg.layer_types.count("linear_attention") == 21
    assert [i for i, t in enumerate(cfg.layer_types) if t == "full_attention"] == list(range(3, 28, 4))
    for name, p in tiny.named_parameters():
        if name.endswith("dt_bias"):
            assert torch.all(p == 1)
        elif name.endswith("A_log"):
            assert torch.all((p >= 0) & (p <= np.log(16) + 1e-6))
        elif name.endswith("linear_attn.norm.weight"):
            assert abs(p.mean().item() - 1) < 0.01
        else:
            assert abs(p.std().item() - 0.02) < 0.01, name
    again = __import__("fastdecisions_amd.model", fromlist=["build_decider"]).build_decider(
        tiny.shape, seed=0, device="cpu", dtype=torch.float32)
    assert all(torch.equal(a, b) for a, b in zip(tiny.parameters(), again.parameters()))


def test_install_patches_fall_back_on_cpu(tiny):
    """Every patched forward must defer to the original method for non-CUDA inputs
    (ref: src/decider/packed_conv.py:27-38)."""
    from fastdecisions_amd.model import install_hip_kernels, synthetic_ids
    ids = synthetic_ids(1, 40, tiny.shape.vocab_size, seed=4, device="cpu")
    with torch.no_grad():
        before = tiny(ids)
    counts = install_hip_kernels(tiny)
    assert counts == dict(packed_conv=3, native_gqa=1, residual_rms=3, residual_rms_all_layers=4, gated_delta=3,
                          combined_gates=3, gated_norm=3, attention_fusions=1, combined_projections=3, mlp_fusion=4)
    assert install_hip_kernels(tiny) == counts  # idempotent
    with torch.no_grad():
        after = tiny(ids)
    assert torch.equal(before, after)


def test_install_levels_are_nested():
    """Each level installs what the one before did and its own step; the reference's three patches
    alone come first."""
    from fastdecisions_amd.model import INSTALL_LEVELS, TINY, build_decider, install_hip_kernels
    assert INSTALL_LEVELS[0] == "north_star"
    seen = set()
    for level in INSTALL_LEVELS:
        model = build_decider(TINY, seed=0, device="cpu", dtype=torch.float32)
        keys = set(install_hip_kernels(model, level))
        assert seen < keys
        seen = keys
    model = build_decider(TINY, seed=0, device="cpu", dtype=torch.float32)
    assert install_hip_kernels(model, "north_star") == dict(packed_conv=3, native_gqa=1, residual_rms=3)
    assert not getattr(model.core, "_fd_residual_chain", False)
    assert not any(getattr(m, "_fd_gated_delta", False) for m in model.core.modules())
    with pytest.raises(ValueError, match="level must be one of"):
        install_hip_kernels(model, "everything")


def test_plain_causal_mask_guard():
    """The native GQA patch runs the kernel only for masks that add nothing to its in-kernel causal mask
    (the reference's checks, ref: experiments/native_gqa/bench_native_gqa_model.py:84-99)."""
    from fastdecisions_amd.native_gqa import plain_causal
    t = 6
    tril = torch.ones((t, t), dtype=torch.bool).tril()
    additive = torch.zeros((1, 1, t, t)).masked_fill(~tril, torch.finfo(torch.float32).min)
    assert plain_causal(None, t)
    assert plain_causal(tril[None, None].expand(2, 1, t, t), t)
    assert plain_causal(additive, t)
    assert plain_causal(additive.to(torch.bfloat16), t)
    padded = tril.clone()
    padded[:, 0] = False  # a left-padded first token
    assert not plain_causal(padded[None, None], t)
    segments = tril.clone()
    segments[3:, :3] = False  # two packed requests
    assert not plain_causal(segments[None, None], t)
    biased = additive.clone()
    biased[..., 2, 1] = 0.5  # an attention bias
    assert not plain_causal(biased, t)
    leaky = additive.clone()
    leaky[..., 0, 1] = -10.0  # a future position not fully masked
    assert not plain_causal(leaky, t)
    assert not plain_causal(tril[None, None], t + 1)  # another length
    assert not plain_causal(torch.zeros((1, 1, t, t), dtype=torch.int32), t)


def test_non_causal_mask_runs_the_original_attention(tiny, monkeypatch):
    """candidate_forward hands a padding mask to the original forward even where it would otherwise run
    the kernel (inputs made to look like CUDA bf16 inference)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5Attention
    from fastdecisions_amd import native_gqa
    attn = next(m for m in tiny.core.modules() if isinstance(m, Qwen3_5Attention))
    native_gqa.install_native_gqa(tiny.core)
    calls = []
    monkeypatch.setattr(attn, "_native_gqa_original_forward", lambda *a, **k: calls.append(k) or ("orig", None))

    class Hidden:  # stands in for a CUDA bf16 [1, 4, hidden] tensor: only the attributes the guard reads
        is_cuda = True
        dtype = torch.bfloat16
        shape = (1, 4, tiny.shape.hidden_size)
    mask = torch.ones((4, 4), dtype=torch.bool).tril()
    mask[:, 0] = False
    with torch.no_grad():
        assert attn.forward(Hidden(), (None, None), mask[None, None]) == ("orig", None)
    assert len(calls) == 1


def test_workloads_are_seeded_and_pack_consistently():
    from fastdecisions_amd.workloads import config4_request, config5_requests, pack
    a, b = config4_request(65536), config4_request(65536)
    assert torch.equal(a.ids, b.ids) and a.slots == [2044, 2045, 2046, 2047] and a.nopts == [4] * 4
    reqs = config5_requests(65536)
    lengths = [int(r.ids.numel()) for r in reqs]
    assert len(reqs) == 4 and all(256 <= n <= 8192 for n in lengths)
    assert all(2 <= r.nopts[0] <= 10 for r in reqs)
    ids, cu, segments, max_len, slots = pack(reqs, device="cpu")
    assert cu.tolist() == [0] + list(np.cumsum(lengths))
    assert max_len == max(lengths) and ids.shape == (1, sum(lengths))
    assert slots == [e - 1 for _, e in segments]
    for r, (s, e) in zip(reqs, segments):
        assert torch.equal(ids[0, s:e], r.ids)


def test_read_slots_matches_oracle_readout(golden):
    from oracle import cpu as oracle
    from fastdecisions_amd.engine import decisions, read_slots
    d = golden("readout")
    n = d["logits"].shape[0]
    out = torch.from_numpy(d["logits"]).float()[None]  # one row, N slot positions
    probs = read_slots(out, [0] * n, list(range(n)), d["nopts"].tolist())
    assert decisions(probs) == d["choice"].tolist()
    _, p = oracle.decide(d["logits"].astype(np.float32), d["nopts"])
    assert np.allclose(probs.numpy(), p, atol=1e-6)


def test_request_segments_come_from_cu_seqlens_when_not_given():
    """The torch delta-rule fallback of the patched Gated-DeltaNet runs once per request: with only
    cu_seq_lens_q passed, the boundaries are read back from it; fd_segments wins when both are given."""
    from fastdecisions_amd.packed_conv import _segments
    cu = torch.tensor([0, 3, 3, 10], dtype=torch.int32)
    assert _segments({"cu_seq_lens_q": cu}) == [(0, 3), (3, 3), (3, 10)]
    assert _segments({"cu_seq_lens_q": cu, "fd_segments": ((0, 10),)}) == [(0, 10)]
    assert _segments({}) is None
