"""CPU tests of the C-ABI boundary: the library loads, exports exactly what
include/fd_kernels.h declares, and rejects bad arguments before touching a GPU."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest
import torch

from conftest import ROOT

HEADER = ROOT / "include" / "fd_kernels.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"FD_API\s+[\w\s\*]+?\b(fd_\w+)\s*\(", text))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == {"fd_abi_version", "fd_last_error", "fd_gqa_fwd", "fd_packed_conv_fwd",
                                    "fd_add_rmsnorm_fwd", "fd_gated_delta_workspace_bytes", "fd_gated_delta_fwd",
                                    "fd_gate_transform_fwd", "fd_gqa_gated_fwd", "fd_attn_prologue_fwd",
                                    "fd_slot_readout_fwd", "fd_gated_rmsnorm_fwd", "fd_silu_mul_fwd",
                                    "fd_packed_conv_strided_fwd", "fd_gated_delta_norm_fwd",
                                    "fd_gate_proj_fwd", "fd_packed_conv_gate_fwd",
                                    "fd_silu_mul_split_fwd", "fd_gated_delta_fwd_noalloc",
                                    "fd_gqa_workspace_bytes", "fd_silu_check", "fd_gated_silu_check",
                                    "fd_hbm_copy"}


def test_library_exports_every_declared_symbol_and_nothing_else():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == declared_functions()
    assert set(_lib.SIGNATURES) == declared_functions()


def test_abi_version_matches_header():
    from fastdecisions_amd import _lib
    version = int(re.search(r"#define FD_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert _lib.lib().fd_abi_version() == version


def test_the_library_uses_torch_s_hip_runtime():
    from fastdecisions_amd import _lib
    _lib.lib()
    maps = [line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line]
    assert maps and all("torch" in path for path in maps), set(maps)


def _err(lib):
    return lib.fd_last_error().decode()


def test_rmsnorm_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    fake = 1 << 20  # 16-byte aligned, never dereferenced: validation fails first
    assert lib.fd_add_rmsnorm_fwd(fake, fake, fake, fake, None, 4, 7, 1e-6, 0, 1, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "width" in _err(lib)
    assert lib.fd_add_rmsnorm_fwd(fake, fake, fake, fake, None, 4, 2048, 1e-6, 5, 1, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_add_rmsnorm_fwd(fake + 2, fake, fake, fake, None, 4, 2048, 1e-6, 0, 1, None) == _lib.FD_ERR_ALIGNMENT
    assert lib.fd_add_rmsnorm_fwd(None, fake, fake, fake, None, 4, 2048, 1e-6, 0, 1, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_add_rmsnorm_fwd(fake, fake, fake, fake, fake, 4, 2048, -1.0, 0, 1, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_add_rmsnorm_fwd(fake, fake, fake, fake, fake, 4, 2048, 1e-6, 0, 1, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "distinct" in _err(lib)
    # zero rows is a valid no-op that never launches
    assert lib.fd_add_rmsnorm_fwd(fake, fake, fake, fake, None, 0, 2048, 1e-6, 0, 1, None) == _lib.FD_OK


def test_conv_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    call = lambda **kw: lib.fd_packed_conv_fwd(
        kw.get("x", f), f, None, f, f, f, kw.get("B", 1), kw.get("T", 16), kw.get("kd", 2048), kw.get("vd", 2048),
        kw.get("W", 4), kw.get("cu"), kw.get("n", 0), kw.get("act", 1), None)
    assert call(W=5) == _lib.FD_ERR_UNSUPPORTED
    assert call(kd=12) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(act=7) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(x=f + 8) == _lib.FD_ERR_ALIGNMENT
    assert call(B=2, cu=f, n=1) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "batch == 1" in _err(lib)
    assert call(B=0) == _lib.FD_OK  # empty batch: nothing to launch


def test_silu_check_argument_errors():
    import ctypes
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    assert lib.fd_silu_check(ctypes.c_uint32(0), ctypes.c_uint32(16), None, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_silu_check(ctypes.c_uint32(0xFFFFFFF0), ctypes.c_uint32(0x20), f, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "2^32" in _err(lib)
    assert lib.fd_silu_check(ctypes.c_uint32(5), ctypes.c_uint32(0), f, None) == _lib.FD_OK  # empty range
    assert lib.fd_gated_silu_check(ctypes.c_uint32(0), ctypes.c_uint32(16), None, None) == \
        _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_gated_silu_check(ctypes.c_uint32(0xFFFFFFF0), ctypes.c_uint32(0x20), f, None) == \
        _lib.FD_ERR_INVALID_ARGUMENT
    assert "2^32" in _err(lib)
    assert lib.fd_gated_silu_check(ctypes.c_uint32(5), ctypes.c_uint32(0), f, None) == _lib.FD_OK


def test_hbm_copy_argument_errors():
    import ctypes
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    assert lib.fd_hbm_copy(None, f, 16, 1, 256, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_hbm_copy(f, f + 4096, 24, 1, 256, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "multiple of 16" in _err(lib)
    assert lib.fd_hbm_copy(f, f + 4096, -16, 1, 256, None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert lib.fd_hbm_copy(f + 8, f + 4096, 16, 1, 256, None) == _lib.FD_ERR_ALIGNMENT
    assert lib.fd_hbm_copy(f, f + 4096, 16, 3, 256, None) == _lib.FD_ERR_UNSUPPORTED
    assert lib.fd_hbm_copy(f, f + 4096, 16, 1, 128, None) == _lib.FD_ERR_UNSUPPORTED
    assert lib.fd_hbm_copy(f, f + 4096, 0, 4, 512, None) == _lib.FD_OK  # nothing to copy, nothing launched


def test_gqa_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    good = (ctypes.c_int64 * 4)(16 * 2048 * 128, 2048 * 128, 128, 1)
    bad_inner = (ctypes.c_int64 * 4)(16 * 2048 * 128, 2048 * 128, 128, 2)
    bad_row = (ctypes.c_int64 * 4)(16 * 2048 * 128, 2048 * 128, 100, 1)

    def call(qs=good, Hq=16, Hkv=4, D=128, q=f, cu=None, n=0, mx=0, B=1, T=2048):
        return lib.fd_gqa_fwd(q, f, f, f, qs, good, good, good, B, Hq, Hkv, T, D, 0.088, cu, n, mx, None, 0, None)

    assert call(D=96) == _lib.FD_ERR_UNSUPPORTED
    assert call(Hq=15) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(qs=bad_inner) == _lib.FD_ERR_ALIGNMENT
    assert call(qs=bad_row) == _lib.FD_ERR_ALIGNMENT
    assert call(q=f + 4) == _lib.FD_ERR_ALIGNMENT
    assert call(cu=f, n=2, mx=4096, T=2048) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(B=2, cu=f, n=2, mx=10) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(T=0) == _lib.FD_OK


def test_gated_delta_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    need = lib.fd_gated_delta_workspace_bytes(1, 2048, 16, 128, 128, 0)
    # 32 chunks x 16 heads of per-chunk intermediates, plus the chunk table: exponentials,
    # q and k in bf16, w in three bf16 planes, u in fp32, A in fp32, and the bf16 output rows
    # the gated norm reads (64 tokens x 128 per chunk and head)
    per_chunk = (3 * 64 * 4 + 2 * 64 * 128 * 2 + 3 * 64 * 128 * 2 + 64 * 128 * 4 + 64 * 64 * 4
                 + 64 * 128 * 2)
    assert need >= 32 * 16 * per_chunk and need < 32 * 16 * per_chunk + 4096
    assert lib.fd_gated_delta_workspace_bytes(1, 2048, 16, 64, 128, 0) == _lib.FD_ERR_UNSUPPORTED
    assert lib.fd_gated_delta_workspace_bytes(2, 100, 4, 128, 128, 3) == _lib.FD_ERR_INVALID_ARGUMENT
    # varlen: one extra (partial) chunk per request at most
    assert lib.fd_gated_delta_workspace_bytes(1, 2048, 16, 128, 128, 4) > need

    def call(q=f, B=1, T=2048, hk=16, hv=16, dk=128, bdt=0, ws=need, cu=None, n=0, scale=0.088, work=f):
        return lib.fd_gated_delta_fwd(q, f, f, f, f, f, None, None, work, ws, B, T, hk, hv, dk, 128, scale, bdt, 1,
                                      cu, n, None)

    assert call(dk=64) == _lib.FD_ERR_UNSUPPORTED
    assert call(hk=3) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "multiple of k_heads" in _err(lib)
    assert call(bdt=7) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(q=f + 8) == _lib.FD_ERR_ALIGNMENT
    assert call(ws=need - 1) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "workspace too small" in _err(lib)
    assert call(B=2, cu=f, n=1) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "batch == 1" in _err(lib)
    assert call(scale=0.0) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(work=None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(B=0, ws=0) == _lib.FD_OK  # empty batch: nothing to launch


def test_gated_delta_norm_argument_errors():
    """fd_gated_delta_norm_fwd checks the norm's arguments, and the row count of the norm that
    follows the delta rule, before anything is launched (no HIP call: the pointers are never read)."""
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    need = lib.fd_gated_delta_workspace_bytes(1, 2048, 16, 128, 128, 0)

    def call(z=f, zts=16 * 128 * 2, zhs=128, w=f, wdt=0, eps=1e-6, T=2048, ws=need):
        return lib.fd_gated_delta_norm_fwd(f, f, f, f, f, z, zts, zhs, w, wdt, eps, f, None, None, f, ws,
                                           1, T, 16, 16, 128, 128, 0.088, 0, 1, None, 0, None)

    assert call(z=None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(w=None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(wdt=7) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(eps=-1.0) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(zhs=100) == _lib.FD_ERR_ALIGNMENT
    assert call(zts=128) == _lib.FD_ERR_ALIGNMENT  # the token stride must cover the 16 heads
    assert call(z=f + 8) == _lib.FD_ERR_ALIGNMENT
    # 2^27 tokens x 16 value heads = 2^31 norm rows: refused before the delta rule is launched
    assert call(T=1 << 27, ws=1 << 62) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "problem too large" in _err(lib)


def test_noalloc_delta_rule_rejects_sizes_beyond_its_static_scratch():
    """fd_gated_delta_fwd_noalloc checks its sizes against the static scratch before any HIP call."""
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = ctypes.c_void_p(256)  # never dereferenced: the size checks come first
    scale = ctypes.c_float(128 ** -0.5)
    assert lib.fd_gated_delta_workspace_bytes(1, 2048, 16, 128, 128, 0) <= 134217728  # the decider call fits
    rc = lib.fd_gated_delta_fwd_noalloc(f, f, f, f, f, f, None, None, 1, 4096, 16, 16, 128, 128, scale,
                                        _lib.FD_DTYPE_BF16, 1, None, 0, None)
    assert rc == _lib.FD_ERR_UNSUPPORTED and b"static scratch" in lib.fd_last_error()
    rc = lib.fd_gated_delta_fwd_noalloc(f, f, f, f, f, f, None, None, 1, 64, 16, 16, 64, 128, scale,
                                        _lib.FD_DTYPE_BF16, 1, None, 0, None)
    assert rc == _lib.FD_ERR_UNSUPPORTED


def test_gate_transform_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20

    def call(a=f, sa=32, sb=32, ld=0, bd=1, rows=2048, heads=16):
        return lib.fd_gate_transform_fwd(a, f + 32, sa, sb, f, ld, f, bd, f, f, rows, heads, None)

    assert call(a=None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(heads=0) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(sa=8) == _lib.FD_ERR_INVALID_ARGUMENT
    assert call(ld=3) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "dtypes" in _err(lib)
    assert call(rows=0) == _lib.FD_OK


def test_joined_launch_argument_errors():
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    f = 1 << 20
    conv_gate = lambda **kw: lib.fd_packed_conv_gate_fwd(
        f, 6144, f, f, f, f, kw.get("B", 1), 16, 2048, 2048, kw.get("W", 4), None, 0,
        kw.get("hs", f), 2048, f, kw.get("hidden", 2048), f, 1, f, 1, f, f, kw.get("heads", 16), None)
    assert conv_gate(heads=12) == _lib.FD_ERR_UNSUPPORTED
    assert "heads must be" in _err(lib) and "fd_packed_conv_gate_fwd" in _err(lib)
    assert conv_gate(hidden=1000) == _lib.FD_ERR_UNSUPPORTED
    assert conv_gate(W=5) == _lib.FD_ERR_UNSUPPORTED
    assert conv_gate(hs=f + 8) == _lib.FD_ERR_ALIGNMENT
    assert conv_gate(B=0) == _lib.FD_OK  # no tokens: nothing to launch
    split = lambda **kw: lib.fd_silu_mul_split_fwd(
        f, kw.get("s1", 8192), kw.get("w1", 4096), kw.get("g2", f), kw.get("s2", 4096), kw.get("w2", 2048),
        kw.get("out", f), kw.get("rows", 2048), None)
    assert split(w1=12) == _lib.FD_ERR_INVALID_ARGUMENT
    assert "fd_silu_mul_split_fwd" in _err(lib)
    assert split(g2=None) == _lib.FD_ERR_INVALID_ARGUMENT
    assert split(s2=4000) == _lib.FD_ERR_INVALID_ARGUMENT
    assert split(out=f + 4) == _lib.FD_ERR_ALIGNMENT
    assert split(rows=0) == _lib.FD_OK


def test_python_wrappers_keep_the_reference_errors_on_cpu_tensors():
    from fastdecisions_amd.native_gqa_kernel import native_gqa_attention
    from fastdecisions_amd.packed_conv_kernel import prep_qkv
    from fastdecisions_amd.persistent_residual_rms_kernel import residual_rms
    with pytest.raises(ValueError, match="input_qkv must be on CUDA"):
        prep_qkv(torch.zeros((1, 2048, 6144), dtype=torch.bfloat16), torch.zeros((6144, 4), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="Q, K and V must share a CUDA device"):
        native_gqa_attention(*(torch.zeros((1, 4, 8, 128), dtype=torch.bfloat16),) * 3)
    with pytest.raises(ValueError, match="All tensors must share a CUDA device"):
        residual_rms(*(torch.zeros((2, 2048), dtype=torch.bfloat16),) * 2, torch.zeros(2048))
    with pytest.raises(ValueError, match="Incompatible Q/K/V shapes"):
        native_gqa_attention(torch.zeros((1, 4, 8, 128)), torch.zeros((1, 2, 9, 128)), torch.zeros((1, 2, 9, 128)))


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from fastdecisions_amd import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="HIP kernel library not found"):
        _lib.lib()


def test_noalloc_rejects_sizes_beyond_the_scratch():
    """fd_gated_delta_fwd_noalloc checks the workspace its sizes need against the static scratch before
    any device call; a B=1 T=4096 call with 16 value heads needs more.  The tensor pointers are real
    (host buffers here, never read: the check returns first)."""
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    T, H = 4096, 16
    need = lib.fd_gated_delta_workspace_bytes(1, T, H, 128, 128, 0)
    header = (ROOT / "include" / "fd_kernels.h").read_text()
    scratch = int(re.search(r"#define FD_GD_SCRATCH_BYTES (\d+)LL", header).group(1))
    assert need > scratch
    bufs = [ctypes.create_string_buffer(16 * 1024) for _ in range(6)]
    ptr = [ctypes.cast(b, ctypes.c_void_p) for b in bufs]
    rc = lib.fd_gated_delta_fwd_noalloc(ptr[0], ptr[1], ptr[2], ptr[3], ptr[4], ptr[5], None, None, 1, T, H, H,
                                        128, 128, ctypes.c_float(0.088), _lib.FD_DTYPE_BF16, 1, None, 0, None)
    assert rc == _lib.FD_ERR_UNSUPPORTED
    assert b"static scratch" in lib.fd_last_error()



def test_gqa_key_split_only_at_head_dim_256():
    """fd_gqa_workspace_bytes (host arithmetic only): head_dim 64 and 128 never ask for a key-split
    workspace, whatever the batch; head_dim 256 does with fewer work items than CUs, including groups
    below 4 query heads per KV head, and never for packed requests."""
    from fastdecisions_amd import _lib
    lib = _lib.lib()
    for D in (64, 128):
        for B, Hq, Hkv, T in ((1, 16, 4, 2048), (1, 16, 4, 300), (1, 4, 4, 1024), (2, 6, 3, 600)):
            assert lib.fd_gqa_workspace_bytes(B, Hq, Hkv, T, D, 0, 0) == 0, (B, Hq, Hkv, T, D)
    for B, Hq, Hkv, T in ((1, 8, 2, 2048), (1, 4, 4, 1024), (1, 6, 3, 600)):
        nbytes = lib.fd_gqa_workspace_bytes(B, Hq, Hkv, T, 256, 0, 0)
        assert nbytes > 0 and nbytes % 16 == 0, (B, Hq, Hkv, T)
    assert lib.fd_gqa_workspace_bytes(1, 8, 2, 2048, 256, 4, 700) == 0  # packed requests
    assert lib.fd_gqa_workspace_bytes(4, 8, 2, 2048, 256, 0, 0) == 0  # enough work items
