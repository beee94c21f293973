"""The exact fast forms used by the attention and RMSNorm kernels (`iexp_fast`, `div_rcp`,
`norm_fd` in superslm_amd/csrc/int_math.h) against the forms they replace (`iexp_element`,
restating src/intmath.cpp:580-668, and `div_floor_pos`): the header is compiled for the host and both forms
run on the same random and edge-case inputs (q_ln2 up to kI64Max / 30, i-exp values up to the
2^47 ceiling, divisors up to 2^60)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="needs hipcc to compile the host check")
def test_fast_forms_match(tmp_path):
    exe = tmp_path / "check"
    subprocess.run(["hipcc", "-O2", "-x", "hip", "--offload-arch=gfx950", "-I", os.path.join(ROOT, "superslm_amd", "csrc"),
                    os.path.join(ROOT, "tests", "int_math_fast_check.cpp"), "-o", str(exe)], check=True,
                   capture_output=True)
    out = subprocess.run([str(exe), "400000"], check=True, capture_output=True, text=True).stdout
    print(out)
    assert "iexp: " in out and ", 0 mismatches" in out.splitlines()[0]
    assert "div: 0 mismatches" in out
    assert "div_q15_small: 0 mismatches" in out
    norm = [l for l in out.splitlines() if l.startswith("norm_fd:")][0]
    assert norm.endswith(", 0 mismatches") and int(norm.split()[1]) > 16_000_000
    small = [l for l in out.splitlines() if l.startswith("iexp_small:")][0]
    assert small.endswith(", 0 mismatches") and int(small.split("(")[1].split(" accepted")[0]) > 10000
    accepted = int(out.split("(")[1].split(" accepted")[0])
    assert accepted > 10000  # the accepted (non-refused) path is exercised, not only refusals
