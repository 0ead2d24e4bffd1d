"""Model-level numerics of the HIP forward against eager and an fp32 ground truth (BASELINE configs 4 and 5).

The reference judges a kernel swap by the model's letter logits and slot
probabilities: ``logits_outside_tolerance`` (|new - old| > 0.05 + 0.02 |old|),
the largest logit and probability differences and the changed decisions
(ref: experiments/native_gqa/bench_native_gqa_model.py:125-140;
ref: experiments/residual_rms/bench_persistent_residual_rms_model.py:91-102).
Three forwards of the same bf16 weights run on 32 seeded config-4 requests
(B=1, T=2048, 4 tail slots of 4 letters each) and the config-5 packed batch:
the reference PyTorch path (eager), the fp32 forward (ground truth) and the
HIP path, the last at every install level of ``INSTALL_LEVELS`` in turn
(each adds to the one before: first the reference's three patches alone, then
the delta rule, the gate kernels and the fusions), so that every slot whose
decision changes can be attributed to the level that changed it.

Bars:

* decisions: at every level, a slot where HIP and eager choose different
  letters must be one where HIP's letter is fp32's, or where fp32's margin
  between its two best letters is below that slot's own bf16 error of the
  reference path (the largest |eager - fp32| over its letters), i.e. a tie
  the reference path itself cannot resolve;
* the full HIP path's error against fp32 is no worse than 1.5x eager's
  (largest logit and probability error, logits outside the reference
  tolerance, decisions that differ from fp32's);
* packed requests equal the same requests run alone.
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
    with torch.no_grad():
        out["eager"] = [model(r.ids[None].cuda()).cpu() for r in reqs]
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


def _decision_table(runs, name):
    """Per slot: eager, fp32 and HIP letters, fp32's top-two margin and eager's bf16 error at the slot."""
    rows = []
    for i, s, n in _slots(runs):
        le, lf, lh = (runs[k][i][0, s, :n].float() for k in ("eager", "fp32", name))
        top = torch.topk(lf, 2).values
        rows.append(dict(req=i, slot=s, eager=int(le.argmax()), fp32=int(lf.argmax()), hip=int(lh.argmax()),
                         margin=float(top[0] - top[1]), eager_err=float((le - lf).abs().max())))
    return rows


def _flips(rows):
    return [r for r in rows if r["hip"] != r["eager"]]


def _unexplained(rows):
    """HIP-vs-eager flips where HIP's letter is not fp32's and fp32's margin exceeds eager's own error."""
    return [r for r in _flips(rows) if r["hip"] != r["fp32"] and r["margin"] >= r["eager_err"]]


def test_decision_flips_attributed_per_install_level(runs):
    """Every slot's decision at every install level; each flip against eager is attributed to the first
    level at which it appears, and must be one the reference path itself cannot resolve."""
    total = len(_slots(runs))
    prev = set()
    bad = []
    eager_vs_fp32 = sum(r["eager"] != r["fp32"] for r in _decision_table(runs, "fp32"))
    print(f"{total} slots; eager bf16 differs from fp32 on {eager_vs_fp32}")
    for level in runs["levels"]:
        rows = _decision_table(runs, level)
        flips = _flips(rows)
        keys = {(r["req"], r["slot"]) for r in flips}
        new = [r for r in flips if (r["req"], r["slot"]) not in prev]
        gone = prev - keys
        print(f"{level:>20}: identical to eager on {total - len(flips)}/{total}; differs from fp32 on "
              f"{sum(r['hip'] != r['fp32'] for r in rows)}; new flips "
              + ", ".join(f"req{r['req']}@{r['slot']} (margin {r['margin']:.4f}, eager err {r['eager_err']:.4f}, "
                          f"hip {'=' if r['hip'] == r['fp32'] else '!='} fp32)" for r in new)
              + (f"; flips gone {sorted(gone)}" if gone else ""))
        prev = keys
        bad += [(level, r) for r in _unexplained(rows)]
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
    for label, part in (("config4", slice(0, n4)), ("config5", slice(n4, None))):
        eager, hip = merged("eager", part), merged(last, part)
        print(f"{label} vs fp32: eager {eager}\n{label} vs fp32: hip   {hip}")
        assert hip["max_abs_logit_diff"] <= 1.5 * eager["max_abs_logit_diff"]
        assert hip["max_abs_prob_diff"] <= 1.5 * eager["max_abs_prob_diff"]
        assert hip["logits_outside_tolerance"] <= 1.5 * eager["logits_outside_tolerance"]
        assert hip["decisions_changed"] <= max(2, int(1.5 * eager["decisions_changed"]))


def test_packed_requests_equal_requests_alone(runs):
    from fastdecisions_amd.numerics import compare
    n4 = runs["n4"]
    for level in runs["levels"]:
        worst = 0.0
        for r, packed, alone in zip(runs["reqs"][n4:], runs[level][n4:], runs[level + "/alone5"]):
            rep = compare(packed, alone, [0] * len(r.slots), r.slots, r.nopts)
            worst = max(worst, rep["max_abs_logit_diff"])
            assert rep["decisions_changed"] == 0, (level, rep)
        print(f"config5 at {level}: packed vs alone, largest logit difference over all positions {worst:.4g}")
        assert worst <= 0.05
