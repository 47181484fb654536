"""Every HIP kernel compiles for gfx950 without vector-register spills or scratch (private memory).

Scratch shows up when a per-thread array is indexed with a runtime value; it turns register
traffic into memory traffic and made one kernel 5x slower before this check existed.  The
check compiles each source with hipcc's resource-usage remarks (no GPU needed).  Scalar-register
spills are allowed while the kernel has no scratch: they then go to lanes of a vector register
(v_writelane / v_readlane), not to memory.
"""
import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "utttcompanion_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("source", sorted(os.path.basename(p) for p in glob.glob(os.path.join(CSRC, "*.hip"))))
def test_kernels_use_no_scratch_and_do_not_spill(source, tmp_path):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-c", os.path.join(CSRC, source), "-o", str(tmp_path / "k.o"),
           "-Rpass-analysis=kernel-resource-usage"]
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, check=True).stdout
    current, bad = None, []
    for line in out.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            current = m.group(1)
        m = re.search(r"(ScratchSize \[bytes/lane\]|VGPRs Spill): (\d+)", line)
        if m and int(m.group(2)) != 0:
            bad.append(f"{current}: {m.group(1)} = {m.group(2)}")
    assert not bad, "\n".join(bad)
