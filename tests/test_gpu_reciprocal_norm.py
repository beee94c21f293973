"""The GPU reciprocal of the funnel plans (`reciprocal_norm`, superslm_amd/csrc/int_math.h:
double reciprocal, one Newton step, one u32 conversion, the reference's two correction steps)
equals `reciprocal_div` -- round_half_up(2^62 / dn), src/intmath.cpp:303-333, pinned against the
oracle by the host tests -- for every normalized divisor dn in [2^30, 2^31).  The check program
is built by __graft_entry__.build() (tests/reciprocal_norm_check.hip)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "reciprocal_norm_check")

pytestmark = pytest.mark.gpu


def test_reciprocal_norm_exhaustive():
    if not os.path.exists(EXE):
        pytest.fail("tests/reciprocal_norm_check is not built: run __graft_entry__.build()")
    out = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(out.stdout, out.stderr)
    assert out.returncode == 0 and ": 0 mismatches" in out.stdout
