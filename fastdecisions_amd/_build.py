"""Build the gfx950 kernel library ``libfd_kernels.so`` in-tree with hipcc.

Each source is compiled to an object of its own (hipcc, ``--offload-arch=gfx950``,
``-ffp-contract=off`` so every fp32 operation rounds where the source says it
does, packed-fp32 instructions disabled), then linked into one shared library
whose exported symbols are exactly the C ABI of ``include/fd_kernels.h``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libfd_kernels.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = "gfx950"

SOURCES = ["fd_abi.cpp", "add_rmsnorm.hip", "packed_conv.hip", "gqa_fwd.hip", "gated_delta.hip", "gate_transform.hip", "attn_prologue.hip", "slot_readout.hip", "gated_norm.hip", "hbm_copy.hip"]

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
]
DEVICE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def rocm_path() -> str:
    return os.environ.get("ROCM_PATH", "/opt/rocm")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the kernel library cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source and link ``libfd_kernels.so``; returns its path."""
    cc = hipcc()
    objdir = PKG_DIR / "_build"
    objdir.mkdir(exist_ok=True)
    cmds = []
    objs = []
    for src in SOURCES:
        path = CSRC / src
        obj = objdir / (src.rsplit(".", 1)[0] + ".o")
        objs.append(obj)
        cmd = [cc, *COMMON_FLAGS]
        if src.endswith(".hip"):
            cmd += ["-x", "hip", *DEVICE_FLAGS]
        else:
            cmd += ["-x", "c++", "-D__HIP_PLATFORM_AMD__", f"-I{rocm_path()}/include"]
        cmd += ["-c", str(path), "-o", str(obj)]
        cmds.append(cmd)
    def compile_one(cmd):
        if verbose:
            print(" ".join(cmd), flush=True)
        return cmd, subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        results = list(pool.map(compile_one, cmds))
    failed = [(cmd, p.stdout) for cmd, p in results if p.returncode != 0]
    if failed:
        for cmd, out in failed:
            sys.stderr.write(" ".join(cmd) + "\n" + out + "\n")
        raise RuntimeError(f"{len(failed)} kernel source(s) failed to compile")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
            "-Wl,--no-undefined", "-Wl,-soname," + LIB_NAME]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
