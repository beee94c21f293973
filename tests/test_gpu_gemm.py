"""The MFMA GEMM paths (decode GEMV and tiled prefill GEMM) against exact integer products, and
BASELINE configuration 0 (GEMM + WSC1 fold + requant funnel) against the oracle."""
import ctypes

import numpy as np
import pytest

from superslm_amd.device import Device

pytestmark = pytest.mark.gpu


def _lib(hip_lib):
    L = hip_lib.lib
    L.sslm_hip_gemm_i32.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int32] * 3 + [ctypes.c_void_p]
    L.sslm_hip_gemm_requant.argtypes = ([ctypes.c_void_p] * 3 + [ctypes.c_int32] * 3 + [ctypes.c_int64] * 4
                                        + [ctypes.c_void_p] * 3)
    return L


@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (3, 320, 1536), (16, 512, 896), (37, 4864, 896),
                                   (64, 1536, 8960), (1, 1536, 8960), (16, 2048, 1536), (16, 1536, 65536),
                                   (48, 96, 4096), (65, 384, 256), (200, 640, 1536), (512, 256, 128),
                                   # ragged row and column tiles at several K steps
                                   (300, 16512, 256), (257, 4224, 384),
                                   # wave-per-tile GEMV (N >= 16384 at M <= 16), ragged N and batches
                                   (16, 17920, 1536), (1, 151936, 1536), (13, 16400, 640), (7, 16448, 1280),
                                   # the gate|up shape of a 512-token chunk, 128-row tiles over 296
                                   # column tiles, ragged rows at two K steps
                                   (512, 17920, 1536), (100, 37888, 512), (448, 33024, 256)])
def test_gemm_i32_exact(m, n, k, hip_lib):
    L = _lib(hip_lib)
    dev = Device(hip_lib)
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    # |sums| < 2^53: float64 products are exact and take the BLAS path
    exp = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)
    da, dw = dev.upload(a), dev.upload(w)
    out = dev.zeros((m, n), np.int32)
    print(f"case gemm m={m} n={n} k={k}", flush=True)
    # twice: split-K decode shapes must leave their arrival counters ready for the next launch
    for _ in range(2):
        assert L.sslm_hip_gemm_i32(da.ptr, dw.ptr, m, n, k, out.ptr) == 0
        got = out.numpy().astype(np.int64)
        assert np.array_equal(got, exp)


def config0_inputs(seed=20260101, m=32, k=896, n=4864):
    """A [32, 896], W [4864, 896] uniform in [-127, 127]; per-output-row
    fold with multiplier uniform in [2^30, 2^31) and right shift uniform in [8, 20]."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    fold = np.zeros((n, 3), dtype=np.int32)
    fold[:, 1] = rng.integers(1 << 30, 1 << 31, size=n, dtype=np.int64).astype(np.int32)
    fold[:, 2] = rng.integers(8, 21, size=n, dtype=np.int32)
    return a, w, fold


IN_SCALE = (1 << 30, -37)
SITE = (1518500250, -45)


@pytest.mark.parametrize("m", [32, 1, 5, 16, 20, 128, 300])
def test_config0_requant_matches_oracle(m, hip_lib, oracle_lib):
    from oracle_bind import project_rows
    L = _lib(hip_lib)
    a, w, fold = config0_inputs(m=m)
    codes_o, scales_o, st_o = project_rows(oracle_lib, a, w, fold, IN_SCALE, SITE)
    n = w.shape[0]
    dev = Device(hip_lib)
    da, dw, df = (dev.upload(x) for x in (a, w, fold))
    codes = dev.zeros((m, n), np.int8)
    me = dev.zeros((m, 2), np.int64)
    st = dev.zeros((m,), np.int32)
    print(f"case config0 m={m}", flush=True)
    assert L.sslm_hip_gemm_requant(da.ptr, dw.ptr, df.ptr, m, n, a.shape[1], *IN_SCALE, *SITE,
                                   codes.ptr, me.ptr, st.ptr) == 0
    assert st.numpy().tolist() == st_o
    assert np.array_equal(codes.numpy(), codes_o)
    assert [tuple(r) for r in me.numpy().tolist()] == scales_o
