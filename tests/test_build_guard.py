"""The build's check on kernel scratch memory (CPU only): a kernel whose
private memory exceeds what its spilled registers explain holds an array in
scratch memory, which the build refuses."""
import os
import re
import subprocess

import pytest

from mvlm_amd import build

REMARKS_OK = """Function Name: _ZN4mvlm1aEv
    VGPRs: 128
    AGPRs: 0
    ScratchSize [bytes/lane]: 88
    VGPRs Spill: 30
    SGPRs Spill: 0
Function Name: _ZN4mvlm1bEv
    VGPRs: 64
    ScratchSize [bytes/lane]: 0
    VGPRs Spill: 0
    SGPRs Spill: 0
"""

REMARKS_STACK = REMARKS_OK + """Function Name: _ZN4mvlm1cEv
    VGPRs: 96
    ScratchSize [bytes/lane]: 1040
    VGPRs Spill: 0
    SGPRs Spill: 0
"""


def test_spills_explain_scratch():
    assert build._stack_kernels(REMARKS_OK) == []


def test_scratch_beyond_spills_is_reported():
    bad = build._stack_kernels(REMARKS_STACK)
    assert len(bad) == 1 and bad[0].startswith("_ZN4mvlm1cEv: 1040 bytes")


def test_compiler_remarks_have_the_parsed_fields(tmp_path):
    """a dynamically indexed local array, compiled as the build compiles HIP
    sources: the remark text carries the fields the check reads, and the check
    flags the kernel (hipcc cross-compiles; no GPU involved)"""
    if not os.path.exists(build.HIPCC):
        pytest.skip("hipcc not available")
    src = tmp_path / "stack.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k(const int* i, float* o) {\n"
        "    float t[256];\n"
        "    for (int j = 0; j < 256; ++j) t[j] = o[j * 7 % 256];\n"
        "    o[threadIdx.x] = t[i[threadIdx.x] & 255];\n"
        "}\n")
    cmd = [build.HIPCC, f"--offload-arch={build.ARCH}", "-O3", "-x", "hip", "--offload-device-only", "-c",
           str(src), "-o", str(tmp_path / "stack.o"), "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    remarks = "\n".join(l.split("remark: ", 1)[1] for l in r.stderr.splitlines() if "remark: " in l)
    assert re.search(r"ScratchSize \[bytes/lane\]: \d+", remarks)
    bad = build._stack_kernels(remarks)
    assert len(bad) == 1 and "_Z1kPKiPf" in bad[0]
