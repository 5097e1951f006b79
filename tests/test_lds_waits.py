"""The pipelined prefill GEMM reads DMA-filled LDS with asm loads whose
completion the compiler does not track; this compiles the kernel for gfx950
and checks that no instruction touches a load's registers before the wait
that retires it (a copy made earlier copies a value not yet loaded)."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "channel_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_gemm_lds_waits(tmp_path):
    out = tmp_path / "gemm_q4.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-fno-gpu-rdc", "--cuda-device-only", "-S",
           os.path.join(CSRC, "gemm_q4.hip"), "-o", str(out)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    sys.path.insert(0, CSRC)
    try:
        import lds_wait_check
    finally:
        sys.path.remove(CSRC)
    res = lds_wait_check.check_file(str(out), "k_q4gemm_p")
    assert res, "no pipelined GEMM kernel found in the assembly"
    bad = {f: h for f, h in res.items() if h}
    assert not bad, bad
