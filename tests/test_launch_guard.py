"""The launch wrappers refuse a malformed launch with an exception the C ABI turns into a status,
instead of aborting the host process (tests/launch_guard_check.cpp; host only, launches nothing)."""
import os
import shutil
import subprocess

import pytest

from conftest import HIP_SO, ROOT


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_launch_wrappers_refuse_instead_of_aborting(tmp_path):
    if not os.path.exists(HIP_SO):
        raise RuntimeError("libsslm_hip.so is not built: run __graft_entry__.build()")
    exe = str(tmp_path / "launch_guard_check")
    obj = str(tmp_path / "launch_guard_check.o")
    subprocess.run(["hipcc", "-O1", "-std=c++17", "-w", "--offload-arch=gfx950", "-c",
                    os.path.join(ROOT, "tests", "launch_guard_check.cpp"), "-o", obj], check=True)
    libdir = os.path.dirname(HIP_SO)
    subprocess.run(["hipcc", obj, "-L" + libdir, "-lsslm_hip", "-Wl,-rpath," + libdir, "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stdout, r.stderr[-2000:])
