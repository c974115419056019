"""Every HIP kernel compiles for gfx950 without spilling a vector register
and without scratch memory: a spill in a GEMM epilogue costs a scratch
round trip per element and inflates the HBM write counters. The sources are
compiled the way brosoundml_amd/build.py compiles them, with the compiler's
resource report (-Rpass-analysis=kernel-resource-usage) read back."""
import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "brosoundml_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC) and not shutil.which("hipcc"), reason="no hipcc")


def resources(src, tmp_path):
    cmd = [HIPCC, "-c", src, "-o", str(tmp_path / "k.o"), "-O3", "-fPIC", "-std=c++17",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(CSRC, 'include')}", f"-I{CSRC}", "-x", "hip",
           "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Rpass-analysis=kernel-resource-usage"]
    out = subprocess.run(cmd, capture_output=True, text=True, check=True).stderr
    kernels, cur = {}, None
    for line in out.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            kernels[cur] = {}
            continue
        m = re.search(r"(VGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
        if m and cur:
            kernels[cur][m.group(1)] = int(m.group(2))
    return kernels


@pytest.mark.parametrize("src", sorted(glob.glob(os.path.join(CSRC, "*.hip"))), ids=os.path.basename)
def test_no_vector_spills_or_scratch(src, tmp_path):
    ks = resources(src, tmp_path)  # empty for a file of host code only
    bad = {k: v for k, v in ks.items() if v.get("VGPRs Spill", 0) or v.get("ScratchSize [bytes/lane]", 0)}
    assert not bad, bad
