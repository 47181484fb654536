"""Build libuttt_amd.so (gfx950) in-tree with hipcc.

``python -m utttcompanion_amd.build`` compiles every ``csrc/*.hip`` into one shared
library next to this file.  The flags disable packed-fp32 code generation (the
packed fp32 forms are avoided on this hardware pool) and target gfx950 only.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libuttt_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "uttt_amd.h")
ARCH = os.environ.get("UTTT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the uTTT HIP library cannot be built")


def sources() -> list:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose: bool = False) -> str:
    """Compile all kernels into LIB_PATH (atomically replaced).  Returns the path."""
    fd, tmp = tempfile.mkstemp(prefix=LIB_NAME + ".", suffix=".tmp", dir=HERE)
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.dirname(HEADER_PATH), *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
