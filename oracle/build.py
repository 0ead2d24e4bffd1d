"""TEST INFRASTRUCTURE — build recipe of the CPU oracle library (gcc)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "fd_oracle.c"
LIB = ORACLE_DIR / "liboracle_fd.so"

# -ffp-contract=off: every fp32 operation rounds where the C source says so.
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall"]


def build() -> Path:
    cc = os.environ.get("CC", "gcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError("oracle build failed: " + " ".join(cmd))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
