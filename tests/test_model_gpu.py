"""GPU parity of the whole decider forward with the HIP kernels installed.

Bar (north_star): identical argmax decisions on every synthetic request, HIP
path (the four kernels) vs the reference PyTorch path (SDPA / F.conv1d / eager
RMSNorm / transformers' torch gated delta rule) on the
same seeded model and inputs — BASELINE config 4 (B=1, T=2048, 4 tail slots)
and config 5 (4 packed requests, per-request causal masking, each compared
with the request run alone through the eager model).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_model():
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, build_decider
    announce("build decider-2b-shaped model (seed 0)")
    return build_decider(DECIDER_2B_SHAPED, seed=0, device="cuda")


def _uninstall(model):
    for m in model.modules():
        for attr in ("_packed_original_forward", "_native_gqa_original_forward", "_persistent_original_forward"):
            if hasattr(m, attr):
                m.forward = getattr(m, attr)
                delattr(m, attr)
        if hasattr(m, "_fd_gated_delta"):
            delattr(m, "_fd_gated_delta")
        for flag in ("_fd_chain_step", "_fd_residual_chain"):
            if hasattr(m, flag):
                delattr(m, flag)
        for buf in ("_combined_gate_weight", "_fd_in_proj_weight", "_fd_qkv_weight"):
            if buf in m._buffers:
                del m._buffers[buf]
        if hasattr(m, "_fd_attn_fused"):
            delattr(m, "_fd_attn_fused")
        if hasattr(m, "_fd_gated_norm"):
            delattr(m, "_fd_gated_norm")
        if hasattr(m, "_fd_mlp_original_forward"):
            m.forward = m._fd_mlp_original_forward
            delattr(m, "_fd_mlp_original_forward")
            del m._buffers["_fd_gate_up_weight"]
            m._buffers.pop("_fd_gate_up_weight2", None)


def test_install_counts_and_fallback(full_model):
    from fastdecisions_amd.model import install_hip_kernels
    counts = install_hip_kernels(full_model)
    try:
        assert counts == dict(packed_conv=21, native_gqa=7, residual_rms=21, residual_rms_all_layers=28, gated_delta=21,
                              combined_gates=21, gated_norm=21, attention_fusions=7, combined_projections=21,
                              mlp_fusion=28)
        # guarded fallbacks: grad mode goes to the original eager methods
        ids = torch.randint(0, 100, (1, 64), device="cuda")
        with torch.enable_grad():
            a = full_model(ids)
        with torch.no_grad():
            b = full_model(ids)
        assert a.shape == b.shape
    finally:
        _uninstall(full_model)


def test_config4_decisions_identical(full_model):
    from oracle import cpu as oracle
    from fastdecisions_amd.engine import Engine, margins, read_slots
    from fastdecisions_amd.model import install_hip_kernels
    from fastdecisions_amd.workloads import config4_request
    req = config4_request(full_model.shape.vocab_size)
    ids = req.ids[None].cuda()
    announce("config4 eager forward")
    with torch.no_grad():
        ref = full_model(ids)
    install_hip_kernels(full_model)
    try:
        announce("config4 HIP forward (eager launch + graph)")
        with torch.no_grad():
            got = full_model(ids)
        eng = Engine(full_model)
        graphed = eng.logits_all(ids).clone()
        torch.cuda.synchronize()
        assert torch.equal(graphed, got)  # graph replay == eager launch of the same kernels
        rows = [0] * len(req.slots)
        p_ref = read_slots(ref, rows, req.slots, req.nopts)
        p_got = read_slots(got, rows, req.slots, req.nopts)
        d_ref, _ = oracle.decide(ref[0, req.slots].cpu().numpy(), req.nopts)
        d_got, _ = oracle.decide(got[0, req.slots].cpu().numpy(), req.nopts)
        m = margins(ref, rows, req.slots, req.nopts)
        diff = (got - ref).abs()
        print(f"config4: decisions eager={d_ref.tolist()} hip={d_got.tolist()} margins={np.round(m, 4).tolist()} "
              f"max|dlogit|={diff.max().item():.4f} max|dp|={(p_got - p_ref).abs().max().item():.4f}")
        assert np.array_equal(d_ref, d_got)
        assert np.array_equal(p_ref.argmax(-1).numpy(), d_ref)
    finally:
        _uninstall(full_model)


def test_everything_but_attention_and_delta_rule_reproduces_eager(full_model):
    """Every HIP kernel installed except the GQA attention (with its prologue and gated store) and
    the chunked delta rule: the forward's logits equal the eager reference path's bit for bit on
    config-4 requests.  The conv (torch's fp32 GPU conv + SiLU), every RMSNorm (PyTorch's row-mean
    order), the a|b gate projection (hipBLASLt's order for the 16-output projections) and its
    transform, the gated norm, SiLU*mul and the combined projections (whose concatenated GEMMs give
    each part the separate GEMM's bits at these shapes) reproduce the eager ops exactly; only the
    attention and the delta rule compute in another order."""
    from fastdecisions_amd.combined_gates import install_combined_gates, install_combined_projections
    from fastdecisions_amd.layer_fusions import install_gated_norm, install_mlp_fusion
    from fastdecisions_amd.packed_conv import install_packed_conv
    from fastdecisions_amd.persistent_residual_rms import install_persistent_residual_rms
    from fastdecisions_amd.workloads import config4_request
    reqs = [config4_request(full_model.shape.vocab_size, seed=s) for s in (1, 2, 3)]
    announce("eager forward of 3 config-4 requests")
    with torch.no_grad():
        ref = [full_model(r.ids[None].cuda()) for r in reqs]
    core = full_model.core
    install_packed_conv(core)
    install_persistent_residual_rms(core, all_layers=True)
    install_combined_gates(core)
    install_gated_norm(core)
    install_combined_projections(core)
    install_mlp_fusion(core)
    try:
        announce("HIP forward without the attention and delta-rule kernels")
        with torch.no_grad():
            got = [full_model(r.ids[None].cuda()) for r in reqs]
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, ref)):
            print(f"request {i}: largest logit difference {(a.float() - b.float()).abs().max().item():.3g}")
            assert torch.equal(a, b), i
    finally:
        _uninstall(full_model)


def test_config5_packed_varlen_decisions_identical(full_model):
    from oracle import cpu as oracle
    from fastdecisions_amd.model import install_hip_kernels
    from fastdecisions_amd.workloads import config5_requests, pack
    reqs = config5_requests(full_model.shape.vocab_size)
    announce(f"config5 lengths={[int(r.ids.numel()) for r in reqs]} nopts={[r.nopts for r in reqs]}")
    ref = []
    with torch.no_grad():
        for r in reqs:  # oracle: each request alone through the eager model
            lg = full_model(r.ids[None].cuda())
            ref.append(lg[0, r.slots].cpu().numpy())
    install_hip_kernels(full_model)
    try:
        ids, cu, segments, max_len, slots = pack(reqs)
        announce("config5 packed HIP forward")
        with torch.no_grad():
            got = full_model(ids, cu_seqlens=cu, segments=segments, max_seqlen=max_len)
            alone_hip = [full_model(r.ids[None].cuda())[0, r.slots].cpu().numpy() for r in reqs]
        torch.cuda.synchronize()
        got_slots = got[0, slots].cpu().numpy()
        for i, r in enumerate(reqs):
            want, _ = oracle.decide(ref[i], r.nopts)
            have, _ = oracle.decide(got_slots[i:i + 1], r.nopts)
            alone, _ = oracle.decide(alone_hip[i], r.nopts)
            top = np.sort(ref[i][0, :r.nopts[0]])[::-1]
            print(f"config5 request {i}: len={r.ids.numel()} n={r.nopts[0]} eager={want.tolist()} "
                  f"packed-hip={have.tolist()} alone-hip={alone.tolist()} margin={top[0] - top[1]:.4f} "
                  f"max|dlogit|={np.abs(got_slots[i] - ref[i][0]).max():.4f}")
            assert np.array_equal(want, have)
            assert np.array_equal(want, alone)
            # packing must not change a request's logits: measured identical; bound at the
            # reference's logit atol
            assert np.abs(got_slots[i] - alone_hip[i][0]).max() <= 0.05
    finally:
        _uninstall(full_model)
