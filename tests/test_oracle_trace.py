"""The oracle's per-site trace hook (test infrastructure for bisecting parity failures): every
layer of a budget-1 decode call reports its sites in the layer loop's order, the last record is
the committed hidden row and scale, and the first is the RMSNorm of the row the layer started
from (or_rmsnorm_site recomputed here)."""
import ctypes

import numpy as np

from conftest import synthetic
from oracle_bind import OracleModel, Scale, load_oracle

TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.POINTER(ctypes.c_int8),
                            ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64)
ORDER = [0, 6, 1, 7, 2, 3, 8, 9, 4, 10, 5]  # attn norm, q, ctx, o, attn res, mlp norm, gate, up, act, down, mlp res


def test_trace_records_each_site_in_order():
    sm, _ = synthetic("small")
    lib = load_oracle()
    lib.or_set_trace.argtypes = [TRACE_FN, ctypes.c_void_p]
    lib.or_rmsnorm_site.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, Scale, ctypes.c_void_p,
                                    ctypes.POINTER(Scale)]
    om = OracleModel(lib, sm)
    seq = om.new_seq()
    assert seq.prefill([3, 1, 4, 1, 5]) == (0, 5)
    assert seq.decode_step(1)[0] == 0
    recs = []
    cb = TRACE_FN(lambda u, l, site, codes, n, m, e: recs.append(
        (l, site, np.ctypeslib.as_array(codes, shape=(n,)).copy(), (m, e))))
    lib.or_set_trace(cb, None)
    try:
        for layer in range(sm.config.layers):
            start = seq.hidden.copy()
            recs.clear()
            assert seq.decode_step(1)[0] == 0
            assert [r[1] for r in recs] == ORDER and all(r[0] == layer for r in recs)
            assert np.array_equal(recs[-1][2], seq.hidden) and recs[-1][3] == (seq.state.scale.m, seq.state.scale.e)
            if layer == 0:  # the embedded current token's row
                continue
            out = np.zeros(sm.config.hidden, dtype=np.int8)
            sc = Scale()
            gain = sm.weights[f"layer{layer}.attn_norm.gain"].astype(np.int32)
            assert lib.or_rmsnorm_site(start.ctypes.data, gain.ctypes.data, sm.config.hidden,
                                       Scale(*sm.consts[f"layer{layer}.attn_norm"]), out.ctypes.data,
                                       ctypes.byref(sc)) == 0
            assert np.array_equal(recs[0][2], out) and recs[0][3] == (sc.m, sc.e)
    finally:
        lib.or_set_trace(ctypes.cast(None, TRACE_FN), None)
