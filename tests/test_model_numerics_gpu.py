"""Model-level numerics of the HIP forward against the reference path and an fp32 ground truth (BASELINE configs 4 and 5).

The reference judges a kernel swap by the model's letter logits and slot
probabilities: ``logits_outside_tolerance`` (|new - old| > 0.05 + 0.02 |old|),
the largest logit and probability differences and the changed decisions
(ref: experiments/native_gqa/bench_native_gqa_model.py:125-140;
ref: experiments/residual_rms/bench_persistent_residual_rms_model.py:91-102).
On 32 seeded config-4 requests (B=1, T=2048, 4 tail slots of 4 letters each)
and the config-5 packed batch, these forwards of the same bf16 weights run:

* the reference PyTorch path (eager: SDPA, fp32 ``conv1d`` + SiLU then one
  cast as BASELINE config 2 defines the conv, eager RMSNorm, transformers'
  torch gated-delta rule), and two variants of it that are equally the
  reference path: SDPA on its math backend instead of flash, and the GEMMs on
  rocBLAS instead of hipBLASLt.  Where their decisions differ from each other,
  a slot is a tie at bf16 precision;
* the fp32 forward (ground truth);
* the HIP path at every install level of ``INSTALL_LEVELS`` in turn (each adds
  to the one before: first the reference's three patches alone, then the delta
  rule, the gate kernels and the fusions), so that every slot whose decision
  changes is attributed to the level that changed it.

Bars:

* decisions, per slot and level: where HIP and the reference path choose
  different letters, HIP's letter must be fp32's, or one that a reference
  variant also chooses there, or fp32's margin between its two best letters
  must be below twice the largest margin error (against fp32) that the
  reference path and its variants show at that slot.  Two paths that each
  err by up to that much can disagree at such a margin, so the slot is a tie
  at bf16 precision that the reference path itself does not resolve; the
  test prints how many slots that criterion covers;
* HIP's decisions differ from fp32's on no more slots than the worst
  reference variant's, plus one;
* the full HIP path's error against fp32 is no worse than 1.5x the largest of
  the reference paths' (largest logit and probability error, logits outside
  the reference tolerance);
* packed requests give the same logits as the same requests run alone, bit
  for bit, at every level.
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce

# eager, fp32 and 8 HIP install levels over 36 requests: about a minute of GPU work in the fixture
pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

N_REQUESTS = 32


@pytest.fixture(scope="module")
def runs():
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, INSTALL_LEVELS, build_decider, install_hip_kernels
    from fastdecisions_amd.numerics import fp32_copy
    from fastdecisions_amd.workloads import config4_request, config5_requests, pack
    announce(f"numerics: {N_REQUESTS} config-4 requests + config 5; eager bf16, fp32, HIP at {len(INSTALL_LEVELS)} levels")
    model = build_decider(DECIDER_2B_SHAPED, seed=0, device="cuda")
    vocab = DECIDER_2B_SHAPED.vocab_size
    reqs = [config4_request(vocab, seed=s) for s in range(1, N_REQUESTS + 1)] + config5_requests(vocab)
    out = dict(reqs=reqs, n4=N_REQUESTS, levels=INSTALL_LEVELS)
    ids5, cu5, segments5, max_len5, _ = pack(reqs[N_REQUESTS:])
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with torch.no_grad():
        out["eager"] = [model(r.ids[None].cuda()).cpu() for r in reqs]
        with sdpa_kernel(SDPBackend.MATH):
            out["eager_sdpa_math"] = [model(r.ids[None].cuda()).cpu() for r in reqs]
        blas = torch.backends.cuda.preferred_blas_library()
        torch.backends.cuda.preferred_blas_library("cublas")  # rocBLAS on ROCm
        try:
            out["eager_rocblas"] = [model(r.ids[None].cuda()).cpu() for r in reqs]
        finally:
            torch.backends.cuda.preferred_blas_library(blas)
        m32 = fp32_copy(model)
        out["fp32"] = [m32(r.ids[None].cuda()).cpu() for r in reqs]
        del m32
        torch.cuda.empty_cache()
        for level in INSTALL_LEVELS:
            announce(f"numerics: HIP path up to {level}")
            install_hip_kernels(model, level)
            alone = [model(r.ids[None].cuda()).cpu() for r in reqs]
            packed = model(ids5, cu_seqlens=cu5, segments=segments5, max_seqlen=max_len5).cpu()
            out[level] = alone[:N_REQUESTS] + [packed[:, s:e] for s, e in segments5]
            out[level + "/alone5"] = alone[N_REQUESTS:]
        # the full install through the engine's captured graph (the benchmark's path)
        from fastdecisions_amd.engine import Engine
        eng = Engine(model)
        out["graph"] = [eng.logits_all(r.ids[None].cuda()).clone().cpu() for r in reqs[:N_REQUESTS]]
    torch.cuda.synchronize()
    del model
    torch.cuda.empty_cache()
    return out


def _slots(runs):
    """(request index, slot position, allowed letters) of every slot."""
    return [(i, s, n) for i, r in enumerate(runs["reqs"]) for s, n in zip(r.slots, r.nopts)]


REFERENCE_PATHS = ("eager", "eager_sdpa_math", "eager_rocblas")
TIE_SLACK = 2.0  # two paths' margin errors of up to ref_err each can differ by twice that


def _decision_table(runs, name):
    """Per slot: the letters of the reference paths, fp32 and ``name``; fp32's top-two margin and each
    reference path's margin error (its difference of those two letters' logits minus fp32's)."""
    rows = []
    for i, s, n in _slots(runs):
        lf = runs["fp32"][i][0, s, :n].float()
        order = torch.argsort(lf, descending=True)
        a, b = int(order[0]), int(order[1])
        margin = float(lf[a] - lf[b])
        ref = {k: runs[k][i][0, s, :n].float() for k in REFERENCE_PATHS}
        rows.append(dict(req=i, slot=s, fp32=a, hip=int(runs[name][i][0, s, :n].float().argmax()),
                         ref={k: int(v.argmax()) for k, v in ref.items()}, margin=margin,
                         ref_err=max(abs(float(v[a] - v[b]) - margin) for v in ref.values())))
    return rows


def _flips(rows):
    return [r for r in rows if r["hip"] != r["ref"]["eager"]]


def _unexplained(rows):
    """Flips against the reference path that are neither fp32's letter, nor a reference variant's choice,
    nor at a slot whose fp32 margin is within the reference paths' own margin error (times the slack)."""
    return [r for r in _flips(rows) if r["hip"] != r["fp32"] and r["hip"] not in r["ref"].values()
            and r["margin"] >= TIE_SLACK * r["ref_err"]]


def test_decision_flips_attributed_per_install_level(runs):
    """Every slot's decision at every install level; each flip against the reference path is attributed
    to the first level at which it appears, and must be a tie the reference path does not resolve."""
    total = len(_slots(runs))
    rows0 = _decision_table(runs, "fp32")
    for k in REFERENCE_PATHS:
        print(f"{k:>20}: identical to the reference path on "
              f"{sum(r['ref'][k] == r['ref']['eager'] for r in rows0)}/{total}, to fp32 on "
              f"{sum(r['ref'][k] == r['fp32'] for r in rows0)}/{total}")
    worst_ref = max(sum(r["ref"][k] != r["fp32"] for r in rows0) for k in REFERENCE_PATHS)
    ties = sum(r["margin"] < TIE_SLACK * r["ref_err"] for r in rows0)
    print(f"{ties}/{total} slots have an fp32 margin below {TIE_SLACK}x the reference paths' margin error there")
    prev = set()
    bad = []
    for level in runs["levels"]:
        rows = _decision_table(runs, level)
        flips = _flips(rows)
        keys = {(r["req"], r["slot"]) for r in flips}
        new = [r for r in flips if (r["req"], r["slot"]) not in prev]
        gone = prev - keys
        wrong = sum(r["hip"] != r["fp32"] for r in rows)
        print(f"{level:>20}: identical to the reference path on {total - len(flips)}/{total}, to fp32 on "
              f"{total - wrong}/{total}; new flips "
              + ", ".join(f"req{r['req']}@{r['slot']} (fp32 margin {r['margin']:.4f}, reference margin error "
                          f"{r['ref_err']:.4f}, hip {'=' if r['hip'] == r['fp32'] else '!='} fp32, "
                          f"{'a reference variant agrees' if r['hip'] in r['ref'].values() else 'no variant agrees'})"
                          for r in new)
              + (f"; flips gone {sorted(gone)}" if gone else ""))
        prev = keys
        bad += [(level, r) for r in _unexplained(rows)]
        assert wrong <= worst_ref + 1, (level, wrong, worst_ref)
    assert not bad, bad


def test_graph_replay_decides_like_the_eager_mode_calls(runs):
    last = runs["levels"][-1]
    for a, b in zip(runs["graph"], runs[last][:runs["n4"]]):
        assert torch.equal(a, b)


def test_hip_error_against_fp32_is_no_worse_than_eager(runs):
    from fastdecisions_amd.numerics import compare, merge
    last = runs["levels"][-1]
    n4 = runs["n4"]

    def merged(name, part):
        reqs = runs["reqs"][part]
        return merge([compare(n, o, [0] * len(r.slots), r.slots, r.nopts)
                      for n, o, r in zip(runs[name][part], runs["fp32"][part], reqs)])
    keys = ("max_abs_logit_diff", "max_abs_prob_diff", "logits_outside_tolerance")
    for label, part in (("config4", slice(0, n4)), ("config5", slice(n4, None))):
        refs = {k: merged(k, part) for k in REFERENCE_PATHS}
        hip = merged(last, part)
        for k, v in refs.items():
            print(f"{label} vs fp32: {k:>15} " + ", ".join(f"{q} {v[q]:.4g}" for q in keys))
        print(f"{label} vs fp32: {'hip':>15} " + ", ".join(f"{q} {hip[q]:.4g}" for q in keys))
        # each error at most 1.5x the largest of the reference paths' (config 5's largest
        # probability error is a maximum over 4 slots, as noisy as one path's draw)
        for q in keys:
            assert hip[q] <= 1.5 * max(v[q] for v in refs.values()), (label, q)
        # decisions against fp32 are bounded per level against every reference variant
        # (test_decision_flips_attributed_per_install_level): a count over 4-6 near-ties is too
        # noisy a statistic to hold to 1.5x one path's


def test_packed_requests_equal_requests_alone(runs):
    """Packed requests give the same logits as the same requests run alone, bit for bit, at every
    install level (the reference holds them to its tolerances, ref:
    experiments/residual_rms/bench_persistent_residual_rms_model.py:91-102).  This build's kernels
    give packed and lone requests identical rows (their own tests), and so does the a|b gate
    projection, which runs in this build's kernel rather than a library GEMM: a GEMM with
    N = 2 x heads picks its reduction split by the token count, and gave packed logits 0.09 away from
    the lone ones.  The other library GEMMs of the forward give identical rows at both token counts."""
    n4 = runs["n4"]
    for level in runs["levels"]:
        worst = 0.0
        for packed, alone in zip(runs[level][n4:], runs[level + "/alone5"]):
            worst = max(worst, float((packed.float() - alone.float()).abs().max()))
        print(f"config5 at {level}: packed vs alone, largest logit difference over all positions {worst:.4g}")
        assert worst == 0.0, (level, worst)
