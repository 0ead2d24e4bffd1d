"""HIP-graph engine for the decider forward and the slot readout.

Mirrors the parts of the reference ``Engine`` on the hot path
(ref: src/decider/engine.py): ``_fwd_eager`` (letter logits ``[B, T, K]`` in fp32,
:115-117), ``logits_all`` with one captured graph per ``(B, T)`` shape
(:123-149) — a HIP graph captured through ``torch.cuda.CUDAGraph`` after warm-up
on a side stream, instead of ``torch.compile`` + CUDA graphs — and
``read_slots`` (:48-56): one gather, mask letters ``>= nopts`` to -inf,
softmax at temperature 1, copy to host.  Decisions are the argmax
(ref: src/decider/infer.py:148-151).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def reference_conv1d_fn(hidden_states, weight, bias=None, activation=None, **kwargs):
    """transformers' ``causal_conv1d_fn`` ([B, C, T] -> [B, C, T]) as BASELINE config 2 defines the
    conv of the reference PyTorch path: fp32 ``F.conv1d`` (bias included), SiLU in fp32, one cast
    to the input dtype.  transformers' own fallback runs the conv in bf16 and rounds its output
    before the SiLU rounds again.  The reference's engine rebinds the same hook to a fused form
    (ref: src/decider/engine.py:25-45) that it runs under ``torch.compile``, where it too is
    computed in fp32 and rounded once."""
    T = hidden_states.shape[-1]
    y = F.conv1d(hidden_states.float(), weight.float().unsqueeze(1), None if bias is None else bias.float(),
                 padding=weight.shape[-1] - 1, groups=hidden_states.shape[1])[..., :T]
    if activation is not None:
        from transformers.activations import ACT2FN
        y = ACT2FN[activation](y)
    return y.to(hidden_states.dtype)


def patch_conv() -> None:
    """Route transformers' Qwen3.5 causal conv hook to ``reference_conv1d_fn`` (process-wide, as
    ref: src/decider/engine.py:43-45 does from its Engine constructor, :86-90).  The HIP path's
    patched Gated-DeltaNet forward does not call the hook; its fallback to the original forward does."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as mq
    mq.causal_conv1d_fn = reference_conv1d_fn


class Engine:
    def __init__(self, model, use_graphs: bool = True):
        self.model = model
        self.use_graphs = use_graphs
        self.graphs: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor, torch.cuda.CUDAGraph]] = {}
        self.pool = torch.cuda.graph_pool_handle() if use_graphs else None
        self.stats = dict(graph_captures=0, forwards=0)

    @torch.no_grad()
    def _fwd_eager(self, ids: torch.Tensor, **kw) -> torch.Tensor:
        return self.model(ids, **kw)

    @torch.no_grad()
    def _capture(self, B: int, T: int):
        dev = next(self.model.parameters()).device
        s_ids = torch.zeros((B, T), dtype=torch.long, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(3):
                self._fwd_eager(s_ids)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool):
            s_out = self._fwd_eager(s_ids)
        self.stats["graph_captures"] += 1
        return s_ids, s_out, graph

    @torch.no_grad()
    def logits_all(self, ids: torch.Tensor) -> torch.Tensor:
        """ids [B, T] long on the device -> letter logits [B, T, K] (fp32).  With graphs the
        returned tensor is the graph's static output, overwritten by the next call of that shape."""
        self.stats["forwards"] += 1
        if not self.use_graphs:
            return self._fwd_eager(ids)
        key = tuple(ids.shape)
        if key not in self.graphs:
            self.graphs[key] = self._capture(*key)
        s_ids, s_out, graph = self.graphs[key]
        s_ids.copy_(ids)
        graph.replay()
        return s_out

    @torch.no_grad()
    def slot_probs(self, ids: torch.Tensor, rows, slots, nopts):
        """Slot-only forward (the final norm, the letter projection and the masked
        softmax at the slots, ref: src/decider/slot_projection.py:6-21), replayed from
        a graph per (B, T, N) with the slot indices in fixed device buffers.
        Returns (logits [N, K], probabilities [N, K]) on the device (graph outputs)."""
        dev = ids.device
        idx = torch.tensor([list(rows), list(slots), list(nopts)], dtype=torch.int32).to(dev)
        if not self.use_graphs:
            return self.model.slot_logits(ids, idx[0], idx[1], idx[2])
        key = ("slots", *ids.shape, idx.shape[1])
        if key not in self.graphs:
            s_ids = torch.zeros_like(ids)
            s_idx = torch.zeros_like(idx)
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                for _ in range(3):
                    self.model.slot_logits(s_ids, s_idx[0], s_idx[1], s_idx[2])
            torch.cuda.current_stream(dev).wait_stream(side)
            torch.cuda.synchronize(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.pool):
                s_out = self.model.slot_logits(s_ids, s_idx[0], s_idx[1], s_idx[2])
            self.stats["graph_captures"] += 1
            self.graphs[key] = ((s_ids, s_idx), s_out, graph)
        (s_ids, s_idx), s_out, graph = self.graphs[key]
        s_ids.copy_(ids)
        s_idx.copy_(idx)
        graph.replay()
        return s_out

    def replay(self, key: tuple) -> torch.Tensor:
        """Replay the captured graph of ``key`` (a ``(B, T)`` shape, or the slot-only
        forward's ``("slots", B, T, N)``) on its current static input."""
        s_ids, s_out, graph = self.graphs[key]
        graph.replay()
        return s_out


def read_slots(out: torch.Tensor, rows, slots, nopts) -> torch.Tensor:
    """Gather slot logits, mask letters >= nopts, softmax; returns probabilities [N, K] on the host."""
    dev = out.device
    idx = torch.tensor([list(rows), list(slots), list(nopts)], dtype=torch.long).to(dev, non_blocking=True)
    lg = out[idx[0], idx[1]]
    lg = lg.masked_fill(torch.arange(lg.shape[1], device=dev)[None, :] >= idx[2][:, None], float("-inf"))
    return torch.softmax(lg.float(), dim=-1).cpu()


def decisions(probs: torch.Tensor) -> list[int]:
    return [int(i) for i in probs.argmax(dim=-1)]


def margins(out: torch.Tensor, rows, slots, nopts) -> list[float]:
    """Logit gap between the best and second-best allowed letter of each slot (decision stability)."""
    res = []
    for r, s, n in zip(rows, slots, nopts):
        top = torch.topk(out[r, s, :n].float(), 2).values
        res.append(float(top[0] - top[1]))
    return res
