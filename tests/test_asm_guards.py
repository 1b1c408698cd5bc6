"""Guards on the compiled gfx950 code that the C++ source cannot express. The GEMM in mnb.hip issues its LDS DMA
(global_load_lds_dwordx4) from inline assembly that sets m0, the DMA's LDS base, right before the instruction.
m0 is a register the compiler reserves and does not preserve across an asm statement, so this is sound only while
no compiler-generated code in those kernels keeps a value in m0: every m0 reference in the assembly must be the
asm's own set, immediately followed by its DMA."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is missing")


def test_m0_is_written_only_by_the_dma_asm(tmp_path):
    out = tmp_path / "mnb.s"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                        "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"),
                        "-I" + os.path.join(ROOT, "strands-decider-web_amd", "csrc"), "-x", "hip", "-S",
                        "--cuda-device-only", os.path.join(ROOT, "strands-decider-web_amd", "csrc", "mnb.hip"),
                        "-o", str(out)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr
    lines = [l.strip() for l in out.read_text().splitlines()]
    code = [l for l in lines if l and not l.startswith((";", "."))]
    refs = [i for i, l in enumerate(code) if re.search(r"\bm0\b", l)]
    assert refs, "the GEMM no longer sets m0; update this guard"
    for i in refs:
        assert code[i].startswith("s_mov_b32 m0,"), code[i]
        assert code[i + 1].startswith("global_load_lds_dwordx4"), (code[i], code[i + 1])
