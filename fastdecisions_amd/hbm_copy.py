"""``hbm_copy(src, dst)`` over the library's ``fd_hbm_copy``: a plain streaming device copy.

No counterpart in the reference.  ``bench.py`` times it at the byte count of each
bandwidth-bound kernel, on the same box and in the same run, as the measured HBM
ceiling those kernels are set against beside the 8 TB/s published peak.
"""
from __future__ import annotations

import torch

from . import _lib


SHAPES = ((1, 256), (2, 256), (4, 256), (1, 512), (2, 512), (4, 512))  # (chunks per thread, block)


def hbm_copy(src: torch.Tensor, dst: torch.Tensor, chunks_per_thread: int = 1, block: int = 256) -> torch.Tensor:
    """Copy ``src`` into ``dst`` (contiguous CUDA tensors of equal byte size, a multiple of 16,
    16-byte aligned, not overlapping) in one of the ``SHAPES``; returns ``dst``."""
    if not (src.is_cuda and dst.is_cuda and src.device == dst.device):
        raise ValueError("src and dst must be CUDA tensors on one device")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("src and dst must be contiguous")
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("src and dst must hold the same number of bytes")
    with torch.cuda.device(src.device):
        _lib.check("fd_hbm_copy", _lib.lib().fd_hbm_copy(src.data_ptr(), dst.data_ptr(), nbytes, chunks_per_thread,
                                                         block, _lib.stream_handle(src.device)))
    return dst
