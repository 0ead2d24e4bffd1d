"""The bench line's host logic, on the CPU: the one-GPU contract and the decision report."""
from __future__ import annotations

import subprocess
import sys
from types import SimpleNamespace

import torch

from conftest import ROOT


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""


def _logits(rows):
    """[1, T=4, K=3] letter logits with the given rows at slots 0..len-1."""
    t = torch.zeros((1, 4, 3))
    for s, r in enumerate(rows):
        t[0, s] = torch.tensor(r)
    return t


def test_decision_report_counts_and_explains_flips():
    import bench
    # one request, three slots of 3 letters
    req = SimpleNamespace(slots=[0, 1, 2], nopts=[3, 3, 3])
    fp32 = [_logits([[1.0, 0.0, 0.0], [0.0, 1.0, 0.9], [0.0, 0.0, 1.0]])]
    eager = [_logits([[1.0, 0.0, 0.0], [0.0, 1.0, 0.95], [0.0, 0.0, 1.0]])]
    # a reference variant flips slot 1 (a tie at bf16: fp32's margin 0.1)
    rocblas = [_logits([[1.0, 0.0, 0.0], [0.0, 0.9, 1.0], [0.0, 0.0, 1.0]])]
    refs = {"eager": eager, "eager_rocblas": rocblas}
    # path A flips slot 1 as the variant does; path B flips slot 2 where fp32's margin is 1.0
    path_a = [_logits([[1.0, 0.0, 0.0], [0.0, 0.9, 1.0], [0.0, 0.0, 1.0]])]
    path_b = [_logits([[1.0, 0.0, 0.0], [0.0, 1.0, 0.9], [0.0, 2.0, 1.0]])]
    out = bench.decision_report([req], refs, fp32, {"a": path_a, "b": path_b})
    assert out["eager"] == {"identical_to_reference": "3/3", "identical_to_fp32": "3/3"}
    assert out["eager_rocblas"] == {"identical_to_reference": "2/3", "identical_to_fp32": "2/3"}
    a, b = out["a"], out["b"]
    assert a["identical_to_reference"] == "2/3" and a["explained"]
    assert a["flips"][0]["slot"] == 1 and a["flips"][0]["a_reference_variant_chose_it"]
    assert not a["flips"][0]["chose_fp32_letter"]
    # slot 2: no variant chose letter 1, fp32's margin (1.0) is far above the reference error there
    assert b["identical_to_reference"] == "2/3" and not b["explained"]
    assert b["flips"][0] == dict(request=0, slot=2, fp32_margin=1.0, reference_margin_error=0.0,
                                 chose_fp32_letter=False, a_reference_variant_chose_it=False)
