"""sslm_hip_gemm_requant_noalloc (the entry point that allocates nothing, its scratch in one
file-scope device array) against sslm_hip_gemm_requant, the allocating entry point it mirrors:
codes, per-row scales and statuses equal bit for bit, on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), and sizes beyond the documented
maximum refused without a launch."""
import ctypes

import numpy as np
import pytest

from superslm_amd.device import Device
from test_gpu_gemm import IN_SCALE, SITE, config0_inputs

pytestmark = pytest.mark.gpu


def _bind(hip_lib):
    L = hip_lib.lib
    common = [ctypes.c_void_p] * 3 + [ctypes.c_int32] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 3
    L.sslm_hip_gemm_requant.restype = ctypes.c_int
    L.sslm_hip_gemm_requant.argtypes = common
    L.sslm_hip_gemm_requant_noalloc.restype = ctypes.c_int
    L.sslm_hip_gemm_requant_noalloc.argtypes = common + [ctypes.c_void_p]
    L.sslm_hip_noalloc_scratch_bytes.restype = ctypes.c_size_t
    return L


def _call(L, dev, fn, a, w, fold, noalloc, site=SITE):
    m, k = a.shape
    n = w.shape[0]
    da, dw, df = (dev.upload(x) for x in (a, w, fold))
    codes = dev.upload(np.full((m, n), 99, np.int8))
    me = dev.upload(np.full((m, 2), 7, np.int64))
    st = dev.upload(np.full((m,), 5, np.int32))
    args = (da.ptr, dw.ptr, df.ptr, m, n, k, *IN_SCALE, *site, codes.ptr, me.ptr, st.ptr)
    rc = fn(*args, None) if noalloc else fn(*args)
    assert L.sslm_hip_synchronize() == 0
    return rc, codes.numpy(), me.numpy(), st.numpy()


@pytest.mark.parametrize("shapes", [((32, 896, 4864), (8, 896, 1024)), ((128, 256, 8192), (65, 128, 4096)),
                                    ((64, 1536, 2048), (1, 1536, 2048))])
def test_noalloc_matches_allocating_entry(shapes, hip_lib):
    L = _bind(hip_lib)
    dev = Device(hip_lib)
    assert 0 < L.sslm_hip_noalloc_scratch_bytes() <= 32 << 20
    for i, (m, k, n) in enumerate(shapes):
        print(f"case noalloc call {i} m={m} k={k} n={n}", flush=True)
        a, w, fold = config0_inputs(seed=100 + i, m=m, k=k, n=n)
        want = _call(L, dev, L.sslm_hip_gemm_requant, a, w, fold, False)
        got = _call(L, dev, L.sslm_hip_gemm_requant_noalloc, a, w, fold, True)
        assert want[0] == got[0] == 0
        assert np.array_equal(got[3], want[3]), "statuses differ"
        assert np.array_equal(got[1], want[1]), "codes differ"
        assert np.array_equal(got[2], want[2]), "scales differ"


def test_noalloc_refusal_status_matches(hip_lib):
    """A site constant outside the mantissa domain: every row refused, as by the allocating entry."""
    L = _bind(hip_lib)
    dev = Device(hip_lib)
    a, w, fold = config0_inputs(seed=7, m=16, k=256, n=512)
    bad_site = (1 << 33, -45)
    want = _call(L, dev, L.sslm_hip_gemm_requant, a, w, fold, False, site=bad_site)
    got = _call(L, dev, L.sslm_hip_gemm_requant_noalloc, a, w, fold, True, site=bad_site)
    assert np.array_equal(got[3], want[3]) and (got[3] != 0).all()


def test_noalloc_rejects_sizes_beyond_maximum(hip_lib):
    L = _bind(hip_lib)
    dev = Device(hip_lib)
    for m, k, n in ((129, 128, 256), (4, 128, 8208), (4, 120, 256), (4, 128, 8)):
        a, w, fold = config0_inputs(seed=1, m=m, k=k, n=n)
        rc, codes, _, st = _call(L, dev, L.sslm_hip_gemm_requant_noalloc, a, w, fold, True)
        assert rc == 1  # SSLM_INVALID_ARGUMENT
        assert (codes == 99).all() and (st == 5).all()  # nothing launched


def test_noalloc_on_stream_and_in_graph_replays(tmp_path):
    """The callers the entry point is for: a created stream, and HIP graph capture.  One captured
    call replayed three times with new inputs in the same buffers and eager work between replays;
    each replay equals the allocating entry point (tests/noalloc_graph_check.cpp, built here)."""
    import os
    import shutil
    import subprocess
    from conftest import HIP_SO, ROOT
    if shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    obj, exe = str(tmp_path / "check.o"), str(tmp_path / "noalloc_graph_check")
    subprocess.run(["hipcc", "-O1", "-std=c++17", "-w", "--offload-arch=gfx950", "-c",
                    os.path.join(ROOT, "tests", "noalloc_graph_check.cpp"), "-o", obj], check=True)
    libdir = os.path.dirname(HIP_SO)
    subprocess.run(["hipcc", obj, "-L" + libdir, "-lsslm_hip", "-Wl,-rpath," + libdir, "-o", exe], check=True)
    print("case noalloc graph capture", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().startswith("ok"), (r.returncode, r.stdout, r.stderr[-2000:])
