"""Seeded synthetic requests of the benchmark configurations (BASELINE configs 4 and 5).

The reference scores real DecisionBench rows fetched from the Hub
(ref: experiments/native_gqa/bench_native_gqa_model.py:66-78); offline, the
requests are synthetic token ids with answer slots at the sequence tail:

* config 4 — one request, B = 1, T = 2048, ids uniform over the vocabulary;
  4 candidate-answer slots at the tail (positions T-4 .. T-1), each choosing
  among 4 letters;
* config 5 — 4 requests packed into one row, lengths round(exp(U(ln 256, ln 8192))),
  ids uniform; each request's answer slot is its last token, with 2..10 letters
  (uniform), as ``prompt.py`` allows 2..10 lettered options
  (ref: src/decider/prompt.py:10-12).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Request:
    ids: torch.Tensor        # [T] long (host)
    slots: list[int]         # answer-slot positions within the request
    nopts: list[int]         # allowed letters per slot


def config4_request(vocab: int, seq_len: int = 2048, seed: int = 1) -> Request:
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (seq_len,), generator=g)
    return Request(ids=ids, slots=[seq_len - 4 + i for i in range(4)], nopts=[4, 4, 4, 4])


def config5_requests(vocab: int, n: int = 4, lo: int = 256, hi: int = 8192, seed: int = 5) -> list[Request]:
    rng = np.random.default_rng(seed)
    lengths = [int(round(np.exp(rng.uniform(np.log(lo), np.log(hi))))) for _ in range(n)]
    nopts = [int(rng.integers(2, 11)) for _ in range(n)]
    g = torch.Generator().manual_seed(seed)
    return [Request(ids=torch.randint(0, vocab, (L,), generator=g), slots=[L - 1], nopts=[k])
            for L, k in zip(lengths, nopts)]


def pack(requests: list[Request], device="cuda"):
    """Concatenate requests into one [1, sum T] row; returns ids, cu_seqlens (device int32),
    host segments, max_seqlen and the packed slot positions."""
    lengths = [int(r.ids.numel()) for r in requests]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    ids = torch.cat([r.ids for r in requests])[None].to(device)
    cu = torch.tensor(offsets, dtype=torch.int32, device=device)
    segments = [(int(a), int(b)) for a, b in zip(offsets[:-1], offsets[1:])]
    slots = [int(offsets[i]) + s for i, r in enumerate(requests) for s in r.slots]
    return ids, cu, segments, max(lengths), slots
