"""TEST INFRASTRUCTURE — the reference PyTorch path timed on host CPU cores.

Used only by bench.py's cpu_baseline leg.  Every function runs the eager
PyTorch recipe that the GPU kernels replace, on the CPU, and returns the
median wall time of repeated runs after warm-up:

* ``gqa_config1`` — BASELINE config 1 exactly: B=1, T=1024, 16 q / 4 kv heads,
  D=128, fp32, q/k/v ~ N(0,1)/sqrt(128) drawn in that order from seed 0;
  ``F.scaled_dot_product_attention(q, repeat_kv(k,4), repeat_kv(v,4), is_causal=True)``;
* ``conv_config2`` — fp32 depthwise ``F.conv1d`` + SiLU on [1, 2048, 6144];
* ``rmsnorm_config3`` — eager ``residual + x`` and Qwen3.5 RMSNorm on [4, 2048, 2048];
* ``decider_forward`` — the whole eager decider forward (transformers' Qwen3.5
  layers: SDPA, F.conv1d, eager RMSNorm, torch gated-delta rule) at B=1,
  T=2048 in fp32, all 28 layers.
"""
from __future__ import annotations

import os
import platform
import statistics
import time

import torch
import torch.nn.functional as F


def cpu_info() -> dict:
    """The host CPU as /proc/cpuinfo names it (the first processor's ``model name``, family,
    model and stepping), with the cores this process may run on and torch's thread count."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if fields:
                    break  # end of the first processor's block
                continue
            key, val = (p.strip() for p in line.split(":", 1))
            if key in ("model name", "cpu family", "model", "stepping", "vendor_id"):
                fields.setdefault(key, val)
    except OSError:
        pass
    return dict(cores_visible=len(os.sched_getaffinity(0)), torch_threads=torch.get_num_threads(),
                cpu_model=fields.get("model name", platform.processor() or "unknown"),
                cpu_id=" ".join(f"{k}={fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping")
                                if k in fields))


def _median_ms(fn, warmup: int, runs: int) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


@torch.no_grad()
def gqa_config1(warmup: int = 3, runs: int = 10) -> float:
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 16, 1024, 128), generator=g) / 128 ** 0.5
    k = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5
    v = torch.randn((1, 4, 1024, 128), generator=g) / 128 ** 0.5

    def run():
        kr = k[:, :, None].expand(1, 4, 4, 1024, 128).reshape(1, 16, 1024, 128)
        vr = v[:, :, None].expand(1, 4, 4, 1024, 128).reshape(1, 16, 1024, 128)
        return F.scaled_dot_product_attention(q, kr, vr, is_causal=True)
    return _median_ms(run, warmup, runs)


@torch.no_grad()
def conv_config2(warmup: int = 3, runs: int = 10) -> float:
    g = torch.Generator().manual_seed(0)
    x = torch.randn((1, 2048, 6144), generator=g).to(torch.bfloat16)
    w = (torch.randn((6144, 4), generator=g) * 0.25).to(torch.bfloat16)

    def run():
        y = F.conv1d(x.float().transpose(1, 2), w.float()[:, None], padding=3, groups=6144)[..., :2048]
        y = F.silu(y).transpose(1, 2).to(torch.bfloat16)
        return [t.contiguous().view(1, 2048, 16, 128) for t in y.split(2048, dim=-1)]
    return _median_ms(run, warmup, runs)


@torch.no_grad()
def rmsnorm_config3(warmup: int = 3, runs: int = 10) -> float:
    g = torch.Generator().manual_seed(0)
    x = torch.randn((4, 2048, 2048), generator=g).to(torch.bfloat16)
    r = torch.randn((4, 2048, 2048), generator=g).to(torch.bfloat16)
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm
    norm = Qwen3_5RMSNorm(2048, eps=1e-6)
    norm.weight.data = (torch.randn((2048,), generator=g) * 0.02).to(torch.bfloat16)

    def run():
        h = r + x
        return norm(h), h
    return _median_ms(run, warmup, runs)


@torch.no_grad()
def decider_forward(seq_len: int = 2048, warmup: int = 1, runs: int = 4) -> dict:
    """Eager fp32 forward of the whole decider-2b-shaped model (28 layers: 21 Gated-DeltaNet +
    7 GQA, embedding, final norm and letter readout) at B=1, T=``seq_len``; the median of ``runs``
    after ``warmup`` (the bench keeps the sample to about half a minute of CPU work: one forward
    takes several seconds)."""
    from fastdecisions_amd.model import DECIDER_2B_SHAPED, build_decider, synthetic_ids
    t0 = time.perf_counter()
    model = build_decider(DECIDER_2B_SHAPED, seed=0, device="cpu", dtype=torch.float32)
    build_s = time.perf_counter() - t0
    ids = synthetic_ids(1, seq_len, DECIDER_2B_SHAPED.vocab_size, seed=1, device="cpu")
    for _ in range(warmup):
        model(ids)
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        model(ids)
        times.append((time.perf_counter() - t) * 1e3)
    return dict(median_ms=statistics.median(times), runs_ms=times, layers=DECIDER_2B_SHAPED.num_hidden_layers,
                warmup=warmup, runs=runs, build_s=build_s)
