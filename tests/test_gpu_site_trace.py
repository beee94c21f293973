"""Per-site intermediate parity of the decode layer loop: with layer_budget 1 every
sslm_decode_step runs one layer, and sslm_hip_debug_site exposes the codes and carried scale the
HIP path computed at the attention RMSNorm, the attention context funnel, the attention residual,
the MLP RMSNorm and the MLP activation of that layer.  They must equal the oracle's per-site trace
(the records of include/superslm/trace_hook.h:36-112; the oracle is pinned to the compiled
reference by tokens, KV and blobs elsewhere) for every layer, sequence and site, so a parity
failure is located to its layer and site."""
import ctypes

import numpy as np
import pytest

import baseline_workloads as W
from conftest import synthetic
from oracle_bind import OracleModel, load_oracle
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu

SITES = {0: "attention rmsnorm", 1: "attention context", 2: "attention residual", 3: "mlp rmsnorm",
         4: "mlp activation"}
TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.POINTER(ctypes.c_int8),
                            ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64)


def _oracle_trace(sm, prompt, tokens):
    """The oracle's records at budget 1: a list over layer calls of {site: (codes, (m, e))}."""
    lib = load_oracle()
    lib.or_set_trace.argtypes = [TRACE_FN, ctypes.c_void_p]
    om = OracleModel(lib, sm)
    seq = om.new_seq()
    assert seq.prefill(prompt) == (0, len(prompt))
    assert seq.decode_step(1)[0] == 0  # logits only: the prompt's last row
    calls = []

    def hook(user, layer, site, codes, n, m, e):
        if site in SITES:
            calls[-1][site] = (np.ctypeslib.as_array(codes, shape=(n,)).copy(), (m, e))

    cb = TRACE_FN(hook)
    lib.or_set_trace(cb, None)
    try:
        for _ in range(tokens * sm.config.layers):
            calls.append({})
            assert seq.decode_step(1)[0] == 0
    finally:
        lib.or_set_trace(ctypes.cast(None, TRACE_FN), None)
    return calls


def _check(sm, art, hip_lib, prompts, tokens):
    c = sm.config
    width = {0: c.hidden, 1: c.hidden, 2: c.hidden, 3: c.hidden, 4: c.inter}
    want = [_oracle_trace(sm, p, tokens) for p in prompts]
    L = hip_lib.lib
    L.sslm_hip_debug_site.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                      ctypes.c_void_p]
    L.sslm_hip_debug_site.restype = ctypes.c_int32
    model = Model(hip_lib, art)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for s, p in zip(seqs, prompts):
        s.prefill(p)
    model.decode_step(seqs, 1)  # logits only
    for call in range(tokens * c.layers):
        model.decode_step(seqs, 1)
        for r in range(len(prompts)):
            for site, name in SITES.items():
                codes = np.zeros(width[site], dtype=np.int8)
                me = np.zeros(2, dtype=np.int64)
                assert L.sslm_hip_debug_site(model.handle, site, r, codes.ctypes.data, me.ctypes.data) == width[site]
                wc, wme = want[r][call][site]
                where = f"sequence {r}, token {call // c.layers}, layer {call % c.layers}, {name}"
                assert (int(me[0]), int(me[1])) == wme, f"{where}: scale {tuple(me)} != {wme}"
                bad = np.nonzero(codes != wc)[0]
                assert bad.size == 0, f"{where}: codes differ at {bad[:8]}: {codes[bad[:8]]} != {wc[bad[:8]]}"
    for s in seqs:
        s.release()
    pool.close()
    model.close()


@pytest.mark.parametrize("name", ["small", "medium"])
def test_sites_match_oracle_toy(name, hip_lib):
    sm, art = synthetic(name)
    rng = np.random.default_rng(77)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (6, 3, 11)]
    print(f"case site trace {name}", flush=True)
    _check(sm, art, hip_lib, prompts, tokens=2)


@pytest.mark.timeout(600)
def test_sites_match_oracle_15b(hip_lib):
    """BASELINE configuration 1's shape: two sequences, one token through all 28 layers."""
    sm = W.model_15b()
    rng = np.random.default_rng(78)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (4, 2)]
    print("case site trace 1.5B", flush=True)
    _check(sm, sm.to_array(), hip_lib, prompts, tokens=1)
