"""The pipelined prefill GEMMs and the prefill attention read DMA-filled LDS
with asm loads whose completion the compiler does not track; this compiles
the kernels for gfx950 and checks that no instruction touches a load's
registers before the wait that retires it (a copy made earlier copies a
value not yet loaded)."""
import os
import subprocess

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
    import lds_wait_check
    res = lds_wait_check.check_file(str(out), "k_q4gemm_p")
    assert res, "no pipelined GEMM kernel found in the assembly"
    res2 = lds_wait_check.check_file(str(out), "k_q4gemm2d")
    assert len(res2) == 2, "expected both layouts of the DMA-fed gate/up"
    res.update(res2)
    res3 = lds_wait_check.check_file(str(out), "k_q4gemm2s")
    assert len(res3) == 2, "expected both layouts of the 256-token single-matrix contraction"
    res.update(res3)
    bad = {f: h for f, h in res.items() if h}
    assert not bad, bad


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_prefill_attn_lds_waits(tmp_path):
    import lds_wait_check
    out = tmp_path / "attention.s"
    _compile("attention.hip", out)
    res = lds_wait_check.check_file(str(out), "k_prefill_attn_mf")
    assert len(res) == 4, "expected the four GQA forms of the prefill attention"
    bad = {f: h for f, h in res.items() if h}
    assert not bad, bad


def _compile(src, out):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-fno-gpu-rdc", "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(out)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    return out.read_text()


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_swap_sums_read_both_halves(tmp_path):
    """The matvec reductions add the two results of each lane swap
    (v_permlane16/32_swap leaves one value in each operand register).  This
    compiler has folded such a sum into twice the first result; check that
    the first float add after every swap reads both swapped registers."""
    import re
    asm = _compile("matvec_q4r.hip", tmp_path / "matvec_q4r.s").splitlines()
    swaps = 0
    for i, line in enumerate(asm):
        m = re.match(r"\s*v_permlane(16|32)_swap_b32_e32\s+(v\d+),\s*(v\d+)", line)
        if not m:
            continue
        a, b = m.group(2), m.group(3)
        # the first float add that reads either swapped register
        add = None
        for l in asm[i + 1:i + 16]:
            if "v_add_f32" in l:
                regs = re.findall(r"\bv\d+\b", l.split(None, 1)[1])[1:]
                if a in regs or b in regs:
                    add = (l, regs)
                    break
        if add is None:
            continue          # a swap used for a lane exchange, not a pair sum
        assert sorted(add[1]) == sorted([a, b]), (line.strip(), add[0].strip())
        swaps += 1
    assert swaps > 0, "no swap sums found in the matvec assembly"
