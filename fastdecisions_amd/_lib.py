"""ctypes binding of ``libfd_kernels.so`` (the C ABI in ``include/fd_kernels.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded: streams and
device pointers handed over by torch are then valid inside the library.

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises ``RuntimeError`` naming the problem.

``FD_KERNELS_LIB`` names another build of the library to load instead of
the in-tree ``libfd_kernels.so`` (for comparing builds side by side); it must
export every symbol listed in ``SIGNATURES``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_PATH = Path(os.environ.get("FD_KERNELS_LIB", Path(__file__).resolve().parent / "libfd_kernels.so"))

FD_OK = 0
FD_ERR_INVALID_ARGUMENT = -1
FD_ERR_UNSUPPORTED = -2
FD_ERR_ALIGNMENT = -3
FD_ERR_LAUNCH = -4

FD_DTYPE_BF16 = 0
FD_DTYPE_F32 = 1
FD_ACT_NONE = 0
FD_ACT_SILU = 1

# Every symbol the header declares, with its ctypes signature.
_c_void_p = ctypes.c_void_p
_i64_4 = ctypes.POINTER(ctypes.c_int64)
SIGNATURES = {
    "fd_abi_version": (ctypes.c_int, []),
    "fd_last_error": (ctypes.c_char_p, []),
    "fd_gqa_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64_4, _i64_4, _i64_4, _i64_4,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
         _c_void_p, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int64, _c_void_p],
    ),
    "fd_gqa_gated_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64_4, _i64_4, _i64_4, _i64_4, _i64_4,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
         _c_void_p, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int64, _c_void_p],
    ),
    "fd_gqa_workspace_bytes": (ctypes.c_int64, [ctypes.c_int] * 7),
    "fd_attn_prologue_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, ctypes.c_int64, _c_void_p, ctypes.c_int64, ctypes.c_int64,
         _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _c_void_p, _c_void_p, ctypes.c_int,
         _c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p],
    ),
    "fd_packed_conv_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         _c_void_p, ctypes.c_int, ctypes.c_int, _c_void_p],
    ),
    "fd_add_rmsnorm_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int,
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_void_p],
    ),
    "fd_gated_delta_workspace_bytes": (
        ctypes.c_int64,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int],
    ),
    "fd_slot_readout_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
         _c_void_p, ctypes.c_int, _c_void_p, _c_void_p, _c_void_p, ctypes.c_int, ctypes.c_float, _c_void_p,
         _c_void_p, _c_void_p],
    ),
    "fd_gated_rmsnorm_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p,
         ctypes.c_int64, ctypes.c_int, ctypes.c_float, _c_void_p],
    ),
    "fd_packed_conv_strided_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         _c_void_p, ctypes.c_int, ctypes.c_int, _c_void_p],
    ),
    "fd_silu_mul_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, _c_void_p, ctypes.c_int64, ctypes.c_int, _c_void_p],
    ),
    "fd_silu_mul_split_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, ctypes.c_int, _c_void_p, ctypes.c_int64, ctypes.c_int, _c_void_p,
         ctypes.c_int64, _c_void_p],
    ),
    "fd_gate_proj_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, _c_void_p, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p, ctypes.c_int,
         _c_void_p, _c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int, _c_void_p],
    ),
    "fd_packed_conv_gate_fwd": (
        ctypes.c_int,
        [_c_void_p, ctypes.c_int64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int,
         _c_void_p, ctypes.c_int64, _c_void_p, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p, ctypes.c_int,
         _c_void_p, _c_void_p, ctypes.c_int, _c_void_p],
    ),
    "fd_silu_check": (
        ctypes.c_int,
        [ctypes.c_uint32, ctypes.c_uint32, _c_void_p, _c_void_p],
    ),
    "fd_gated_silu_check": (
        ctypes.c_int,
        [ctypes.c_uint32, ctypes.c_uint32, _c_void_p, _c_void_p],
    ),
    "fd_hbm_copy": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _c_void_p],
    ),
    "fd_gate_transform_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int64, _c_void_p, ctypes.c_int, _c_void_p, ctypes.c_int,
         _c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int, _c_void_p],
    ),
    "fd_gated_delta_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, ctypes.c_int64,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p],
    ),
    "fd_gated_delta_fwd_noalloc": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p],
    ),
    "fd_gated_delta_norm_fwd": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, ctypes.c_int64, ctypes.c_int64,
         _c_void_p, ctypes.c_int, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, ctypes.c_int64,
         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_void_p, ctypes.c_int, _c_void_p],
    ),
}

_LIB = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned an error code."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed with code {code}: {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load (once) and return the kernel library; raise if it is unavailable."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP kernel library not found at {LIB_PATH}; build it first "
                "(python -c 'import __graft_entry__ as g; g.build()' or python -m fastdecisions_amd._build)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(name: str, code: int) -> None:
    if code != FD_OK:
        raise KernelError(name, code, lib().fd_last_error().decode(errors="replace"))


def strides4(t) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*t.stride())


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
