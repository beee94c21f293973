"""The oracle's per-site trace hook (test infrastructure for bisecting parity failures): every
layer of a budget-1 decode call reports its sites in the layer loop's order, the last record is
the committed hidden row and scale, and the first is the RMSNorm of the row the layer started
from (or_rmsnorm_site recomputed here).  The chunked prefill reports every site of every layer
once per token, and those records do not depend on how the prompt was cut into chunks: the last
token's records when it runs alone equal its records inside the whole prompt's chunk."""
import ctypes

import numpy as np

from conftest import synthetic
from oracle_bind import OracleModel, Scale, load_oracle

TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.POINTER(ctypes.c_int8),
                            ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64)
# attn norm, q, q after RoPE, ctx, o, attn res, mlp norm, gate, up, act, down, mlp res
ORDER = [0, 6, 11, 1, 7, 2, 3, 8, 9, 4, 10, 5]


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


def _chunk_trace(lib, sm, chunks):
    """Records of the last chunk: {(layer, site): [rows in token order]}."""
    om = OracleModel(lib, sm)
    seq = om.new_seq()
    for c in chunks[:-1]:
        assert seq.prefill(c) == (0, len(c))
    recs = {}

    def hook(u, l, site, codes, n, m, e):
        recs.setdefault((l, site), []).append((np.ctypeslib.as_array(codes, shape=(n,)).copy(), (m, e)))

    cb = TRACE_FN(hook)
    lib.or_set_trace(cb, None)
    try:
        assert seq.prefill(chunks[-1]) == (0, len(chunks[-1]))
    finally:
        lib.or_set_trace(ctypes.cast(None, TRACE_FN), None)
    return recs, seq


def test_chunk_trace_every_site_and_split_invariant():
    sm, _ = synthetic("small")
    lib = load_oracle()
    lib.or_set_trace.argtypes = [TRACE_FN, ctypes.c_void_p]
    prompt = [3, 1, 4, 1, 5, 9, 2]
    whole, seq = _chunk_trace(lib, sm, [prompt])
    L = sm.config.layers
    assert sorted(whole) == sorted((l, s) for l in range(L) for s in ORDER)
    assert all(len(v) == len(prompt) for v in whole.values())
    # the last layer's residual rows are the chunk's committed rows; the last one the stream state
    assert np.array_equal(whole[(L - 1, 5)][-1][0], seq.hidden)
    assert whole[(L - 1, 5)][-1][1] == (seq.state.scale.m, seq.state.scale.e)
    split, _ = _chunk_trace(lib, sm, [prompt[:5], prompt[5:]])
    for key, rows in split.items():
        assert len(rows) == 2
        for k in range(2):
            assert np.array_equal(rows[k][0], whole[key][5 + k][0]), key
            assert rows[k][1] == whole[key][5 + k][1], key
