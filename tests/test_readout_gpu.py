"""GPU parity of the slot-only readout (fd_slot_readout_fwd) and of the slot-only
forward of the whole model.

Bars: logits within one bf16 ulp of the logit's magnitude against the eager
golden and the float64 oracle, probabilities within 1e-2 absolute (1e-3 once
the logits agree), identical argmax; at model level the slot-only forward
makes the same decisions as the full [B, T, K] forward on config 4 and on
every request of config 5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import announce, from_bits

pytestmark = pytest.mark.gpu


def test_golden_fixture(oracle, golden):
    from fastdecisions_amd.slot_projection import slot_readout
    d = golden("readout_slots")
    announce("slot readout golden")
    hidden, letters = from_bits(d["hidden"]), from_bits(d["letters"])
    w = torch.from_numpy(d["norm_w"]).to(torch.bfloat16).cuda()
    rows, pos, nopts = (torch.from_numpy(d[k]).cuda() for k in ("rows", "pos", "nopts"))
    for temp, key in ((1.0, "probs"), (2.0, "probs_t2")):
        lg, p = slot_readout(hidden, w, letters, rows, pos, nopts, eps=1e-6, temperature=temp)
        torch.cuda.synchronize()
        lg, p = lg.cpu().numpy(), p.cpu().numpy()
        assert np.abs(lg - d["logits"]).max() <= 2.0 ** -8 * np.abs(d["logits"]).max()
        assert np.abs(p - d[key]).max() < 1e-2
        assert np.array_equal(p.argmax(1), d[key].argmax(1))
        olg, op = oracle.slot_readout(d["hidden"], d["norm_w"], d["letters"], d["rows"], d["pos"], d["nopts"],
                                      temperature=temp)
        assert np.abs(lg - olg).max() <= 2.0 ** -8 * np.abs(olg).max()
        assert all((p[i, n:] == 0).all() for i, n in enumerate(d["nopts"]))


def test_many_slots_and_letters(oracle):
    from fastdecisions_amd.slot_projection import slot_readout
    gen = torch.Generator().manual_seed(8)
    B, T, H, K, N = 3, 300, 2048, 255, 64
    hidden = torch.randn((B, T, H), generator=gen).to(torch.bfloat16)
    w = (torch.randn(H, generator=gen) * 0.02).to(torch.bfloat16)
    letters = (torch.randn((K, H), generator=gen) * 0.02).to(torch.bfloat16)
    rows = torch.randint(0, B, (N,), generator=gen, dtype=torch.int32)
    pos = torch.randint(0, T, (N,), generator=gen, dtype=torch.int32)
    nopts = torch.randint(1, K + 1, (N,), generator=gen, dtype=torch.int32)
    announce("slot readout N=64 K=255")
    lg, p = slot_readout(hidden.cuda(), w.cuda(), letters.cuda(), rows.cuda(), pos.cuda(), nopts.cuda())
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    olg, op = oracle.slot_readout(bits(hidden), w.float().numpy(), bits(letters), rows.numpy(), pos.numpy(),
                                  nopts.numpy())
    lg, p = lg.cpu().numpy(), p.cpu().numpy()
    assert np.abs(lg - olg).max() <= 2.0 ** -8 * np.abs(olg).max()
    assert np.abs(p - op).max() < 1e-3 + 2.0 ** -7 * op.max()


def test_model_slot_forward_decisions(request):
    from fastdecisions_amd.engine import Engine, read_slots
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, build_decider, install_hip_kernels
    from fastdecisions_amd.workloads import config4_request, config5_requests, pack
    announce("slot-only model forward (config 4 and config 5)")
    model = build_decider(DECIDER_2B_SHAPED, seed=0, device="cuda")
    install_hip_kernels(model)
    eng = Engine(model)
    req = config4_request(model.shape.vocab_size)
    ids = req.ids[None].cuda()
    rows = [0] * len(req.slots)
    full = read_slots(eng.logits_all(ids), rows, req.slots, req.nopts)
    lg, p = eng.slot_probs(ids, rows, req.slots, req.nopts)
    lg2, p2 = eng.slot_probs(ids, rows, req.slots, req.nopts)   # graph replay
    torch.cuda.synchronize()
    assert torch.equal(lg, lg2)
    assert full.argmax(-1).tolist() == p.cpu().argmax(-1).tolist()
    assert (full - p.cpu()).abs().max() < 0.05
    reqs = config5_requests(model.shape.vocab_size)
    pids, cu, segments, max_len, slots = pack(reqs)
    with torch.no_grad():
        out = model(pids, cu_seqlens=cu, segments=segments, max_seqlen=max_len)
        lgv, pv = model.slot_logits(pids, torch.zeros(len(slots), dtype=torch.int32, device="cuda"),
                                    torch.tensor(slots, dtype=torch.int32, device="cuda"),
                                    torch.tensor([r.nopts[0] for r in reqs], dtype=torch.int32, device="cuda"),
                                    cu_seqlens=cu, segments=segments, max_seqlen=max_len)
    full_v = read_slots(out, [0] * len(slots), slots, [r.nopts[0] for r in reqs])
    torch.cuda.synchronize()
    print(f"slot forward: config4 {p.cpu().argmax(-1).tolist()} config5 {pv.cpu().argmax(-1).tolist()}")
    assert full_v.argmax(-1).tolist() == pv.cpu().argmax(-1).tolist()
