"""Native GQA causal attention on the gfx950 HIP kernel ``fd_gqa_fwd``.

Drop-in for the reference launcher ``native_gqa_attention(q, k, v)``
(ref: src/decider/native_gqa_kernel.py:116-173): same logical shapes
(Q ``[B, Hq, T, D]``, K/V ``[B, Hkv, T, D]``, any strides with a contiguous
feature dimension), same validation messages, same output allocation (physical
``[B, T, Hq, D]`` returned as the ``[B, Hq, T, D]`` view), launched on the
current stream without synchronisation.

Differences, all widenings: head_dim 64/128/256 (the reference accepts only
256, ref: :132-133), an optional ``scale`` (default ``D**-0.5`` as ref: :168),
packed variable-length batches through ``cu_seqlens``/``max_seqlen``
(B == 1, T = total tokens; ``max_seqlen`` must be at least the longest
request, whose rows past it would otherwise stay unwritten), with causal
masking inside each request, and an
optional output ``gate`` (logical ``[B, Hq, T, D]`` like the output): the
attention layer's ``output * sigmoid(gate)`` applied in the kernel's store
(``fd_gqa_gated_fwd``; ref: experiments/native_gqa/bench_native_gqa_model.py:54-55).

``key_split`` (default on) lets a head_dim-256 call with fewer work items than
the GPU has CUs (e.g. B=1, T=2048, 8/2 heads) run its longest query tiles as two
halves of their key range, merged by a second launch.  Off, every tile runs
whole; a request's rows are then bit-identical alone, packed or in a padded
batch, which head_dim 64 and 128 always are (they never split).
"""
from __future__ import annotations

import torch

from . import _lib

SUPPORTED_HEAD_DIMS = (64, 128, 256)


def native_gqa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    gate: torch.Tensor | None = None,
    key_split: bool = True,
) -> torch.Tensor:
    # Logical shapes: Q [B, Hq, T, D], K/V [B, Hkv, T, D] (ref: :120).
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("Q, K and V must be four-dimensional")

    batch, q_heads, seq_len, head_dim = q.shape
    kv_heads = k.shape[1]

    if min(batch, q_heads, kv_heads, seq_len) < 1:
        raise ValueError("Batch, head counts and sequence length must be positive")
    if q_heads % kv_heads:
        raise ValueError("Query heads must be divisible by KV heads")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError("This launcher supports head dimension 64, 128 or 256")
    if k.shape != (batch, kv_heads, seq_len, head_dim) or v.shape != k.shape:
        raise ValueError("Incompatible Q/K/V shapes")

    for tensor in (q, k, v):
        if not tensor.is_cuda or tensor.device != q.device:
            raise ValueError("Q, K and V must share a CUDA device")
        if tensor.dtype != torch.bfloat16:
            raise ValueError("Q, K and V must be BF16")
        if tensor.stride(-1) != 1:
            raise ValueError("The feature dimension must be contiguous")
        if tensor.data_ptr() % 16 or any(s % 8 for s in tensor.stride()[:3]):
            raise ValueError("Q, K and V rows must be 16-byte aligned")

    if gate is not None:
        if gate.shape != q.shape or gate.dtype != torch.bfloat16 or gate.device != q.device:
            raise ValueError("gate must be a BF16 tensor shaped like Q on Q's device")
        if gate.stride(-1) != 1 or gate.data_ptr() % 16 or any(s % 8 for s in gate.stride()[:3]):
            raise ValueError("gate rows must be contiguous and 16-byte aligned")

    n_seqs = 0
    cu_ptr = None
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError("cu_seqlens requires batch size 1 (packed requests)")
        if (cu_seqlens.ndim != 1 or cu_seqlens.dtype != torch.int32 or cu_seqlens.device != q.device
                or cu_seqlens.numel() < 2 or not cu_seqlens.is_contiguous()):
            raise ValueError("cu_seqlens must be a contiguous int32 vector [n_seqs + 1] on Q's device")
        if max_seqlen is None:
            raise ValueError("max_seqlen is required with cu_seqlens")
        if not 0 <= int(max_seqlen) <= seq_len:
            raise ValueError("max_seqlen must lie in [0, T]")
        n_seqs = cu_seqlens.numel() - 1
        cu_ptr = cu_seqlens.data_ptr()
    else:
        max_seqlen = seq_len

    if scale is None:
        scale = head_dim ** -0.5

    with torch.cuda.device(q.device):
        # Physical layout [B, T, Hq, D], logical layout [B, Hq, T, D] (ref: :145-151).
        output = torch.empty(
            (batch, seq_len, q_heads, head_dim), device=q.device, dtype=q.dtype
        ).permute(0, 2, 1, 3)
        lib = _lib.lib()
        # workspace of the key split of long query tiles (head_dim 256 with few work items;
        # 0 bytes: the kernel runs unsplit)
        nbytes = 0
        if key_split:
            nbytes = lib.fd_gqa_workspace_bytes(batch, q_heads, kv_heads, seq_len, head_dim, n_seqs,
                                                int(max_seqlen))
            if nbytes < 0:
                _lib.check("fd_gqa_workspace_bytes", nbytes)
        work = torch.empty(nbytes, device=q.device, dtype=torch.uint8) if nbytes > 0 else None
        ws = (None if work is None else work.data_ptr(), nbytes)
        if gate is None:
            _lib.check("fd_gqa_fwd", lib.fd_gqa_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(),
                _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(output),
                batch, q_heads, kv_heads, seq_len, head_dim, float(scale),
                cu_ptr, n_seqs, int(max_seqlen), *ws, _lib.stream_handle(q.device)))
        else:
            _lib.check("fd_gqa_gated_fwd", lib.fd_gqa_gated_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), gate.data_ptr(), output.data_ptr(),
                _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(gate), _lib.strides4(output),
                batch, q_heads, kv_heads, seq_len, head_dim, float(scale),
                cu_ptr, n_seqs, int(max_seqlen), *ws, _lib.stream_handle(q.device)))
    return output
