"""The device integer primitives (int_math.h), compiled for the host, against the C oracle.

The GPU kernels use faster formulations than the reference (double-precision estimates with
exact integer correction, 64-bit halves instead of 128-bit products); this runs them on the
CPU over random and boundary inputs of every domain the kernels feed them and requires
bit-identical results (tests/device_math_host_check.cpp)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_device_math_matches_oracle(tmp_path):
    exe = str(tmp_path / "device_math_host_check")
    obj = str(tmp_path / "sslm_oracle.o")
    subprocess.run(["gcc", "-std=c11", "-O2", "-c", os.path.join(ROOT, "oracle", "sslm_oracle.c"), "-o", obj],
                   check=True)
    main = str(tmp_path / "check.o")
    subprocess.run(["hipcc", "-O2", "-std=c++17", "-w", "--offload-arch=gfx950", "-c",
                    os.path.join(ROOT, "tests", "device_math_host_check.cpp"), "-o", main], check=True)
    subprocess.run(["hipcc", main, obj, "-o", exe], check=True)
    r = subprocess.run([exe, "100000"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-3000:]
