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
    assert counts == dict(packed_conv=3, native_gqa=1, residual_rms=4, gated_delta=3, combined_gates=3, combined_projections=3, attention_fusions=1, gated_norm=3,
                      mlp_fusion=4)
    assert install_hip_kernels(tiny) == counts  # idempotent
    with torch.no_grad():
        after = tiny(ids)
    assert torch.equal(before, after)


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
