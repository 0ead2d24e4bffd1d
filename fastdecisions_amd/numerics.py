"""Model-level numerics of one forward against another, as the reference's benchmarks measure them.

* ``logits_outside_tolerance`` — letter logits with ``|new - old| > 0.05 + 0.02 |old|``
  over every position of the ``[B, T, K]`` output, the largest ``|new - old|``, the
  largest probability difference of the masked softmax at each slot, and the
  decisions (argmax at a slot) that changed
  (ref: experiments/native_gqa/bench_native_gqa_model.py:125-140);
* the same rule is ``torch.testing.assert_close(new, old, rtol=.02, atol=.05)`` on
  the logits and ``rtol=.02, atol=.005`` on the slot probabilities
  (ref: experiments/residual_rms/bench_persistent_residual_rms_model.py:91-102);
  ``logits_close`` / ``probs_close`` say whether a forward passes them;
* beyond the reference: ``rankings_changed`` compares the full order of the
  allowed letters at each slot, not just the top one, and ``min_margin`` is the
  smallest logit gap between neighbours in the reference order at a slot whose
  ranking changed (how close to a tie the flip was).

``old`` is the reference forward (for ground truth: the fp32 forward of the same
bf16 weights), ``new`` the forward under test.
"""
from __future__ import annotations

import torch

LOGIT_ATOL, LOGIT_RTOL = 0.05, 0.02
PROB_ATOL, PROB_RTOL = 0.005, 0.02


def compare(new: torch.Tensor, old: torch.Tensor, rows, slots, nopts, temperature: float = 1.0) -> dict:
    """new/old: letter logits [B, T, K]; slots given as parallel lists (row, position, allowed letters)."""
    new = new.float()
    old = old.float()
    diff = (new - old).abs()
    bound = LOGIT_ATOL + LOGIT_RTOL * old.abs()
    outside = int((diff > bound).sum().item())
    max_p = 0.0
    probs_close = True
    changed = ranked = 0
    flip_margins = []
    for r, s, n in zip(rows, slots, nopts):
        a_lg = old[r, s, :n]
        b_lg = new[r, s, :n]
        a = (a_lg / temperature).softmax(-1)
        b = (b_lg / temperature).softmax(-1)
        max_p = max(max_p, (a - b).abs().max().item())
        probs_close &= bool(((a - b).abs() <= PROB_ATOL + PROB_RTOL * a.abs()).all().item())
        changed += int(a.argmax().item() != b.argmax().item())
        order_a = torch.argsort(a_lg, descending=True, stable=True)
        order_b = torch.argsort(b_lg, descending=True, stable=True)
        if not torch.equal(order_a, order_b):
            ranked += 1
            gaps = a_lg[order_a][:-1] - a_lg[order_a][1:]
            flip_margins.append(float(gaps.min().item()))
    return dict(max_abs_logit_diff=float(diff.max().item()), logits_outside_tolerance=outside,
                n_logits=int(diff.numel()), logits_close=outside == 0, max_abs_prob_diff=max_p,
                probs_close=probs_close, slots=len(list(slots)), decisions_changed=changed,
                rankings_changed=ranked, min_margin_of_changed_rankings=min(flip_margins) if flip_margins else None)


def merge(reports: list[dict]) -> dict:
    """Totals / worst cases over several compare() reports (one per request)."""
    if not reports:
        return {}
    margins = [r["min_margin_of_changed_rankings"] for r in reports if r["min_margin_of_changed_rankings"] is not None]
    return dict(requests=len(reports),
                max_abs_logit_diff=max(r["max_abs_logit_diff"] for r in reports),
                logits_outside_tolerance=sum(r["logits_outside_tolerance"] for r in reports),
                n_logits=sum(r["n_logits"] for r in reports),
                logits_close=all(r["logits_close"] for r in reports),
                max_abs_prob_diff=max(r["max_abs_prob_diff"] for r in reports),
                probs_close=all(r["probs_close"] for r in reports),
                slots=sum(r["slots"] for r in reports),
                decisions_changed=sum(r["decisions_changed"] for r in reports),
                rankings_changed=sum(r["rankings_changed"] for r in reports),
                min_margin_of_changed_rankings=min(margins) if margins else None)


def fp32_copy(model):
    """The same model with every parameter and buffer upcast to fp32: the ground truth runs
    the bf16 weights exactly, so its difference from a bf16 forward is arithmetic error only."""
    import copy
    return copy.deepcopy(model).float()
