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


# ---- every site of every layer: prefill spans and whole-depth decode (sslm_hip_debug_capture) ----
# capture site -> oracle trace site (capture site 6 is q after RoPE, the oracle's site 11)
CAPTURE = {0: 0, 1: 1, 2: 2, 3: 3, 4: 4, 5: 5, 6: 11, 7: 7, 8: 8, 9: 9, 10: 10}
CAPTURE_NAMES = {0: "attention rmsnorm", 1: "attention context", 2: "attention residual", 3: "mlp rmsnorm",
                 4: "mlp activation", 5: "mlp residual", 6: "q after RoPE", 7: "o_proj funnel", 8: "gate funnel",
                 9: "up funnel", 10: "down funnel"}


def _bind_capture(L):
    L.sslm_hip_debug_capture.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    L.sslm_hip_debug_capture.restype = ctypes.c_int
    L.sslm_hip_debug_capture_read.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_void_p, ctypes.c_void_p]
    L.sslm_hip_debug_capture_read.restype = ctypes.c_int32


def _compare_capture(L, model, c, want, rows, what):
    """want[(layer, oracle site)][row] = (codes, (m, e)) for rows 0..rows-1 of the captured launch."""
    width = {s: (c.inter if s in (4, 8, 9) else c.hidden) for s in CAPTURE}
    for layer in range(c.layers):
        for site, osite in CAPTURE.items():
            for r in range(rows):
                codes = np.zeros(width[site], dtype=np.int8)
                me = np.zeros(2, dtype=np.int64)
                assert L.sslm_hip_debug_capture_read(model.handle, layer, site, r, codes.ctypes.data,
                                                     me.ctypes.data) == width[site]
                wc, wme = want[(layer, osite)][r]
                where = f"{what}: row {r}, layer {layer}, {CAPTURE_NAMES[site]}"
                assert (int(me[0]), int(me[1])) == wme, f"{where}: scale {tuple(me)} != {wme}"
                bad = np.nonzero(codes != wc)[0]
                assert bad.size == 0, f"{where}: codes differ at {bad[:8]}: {codes[bad[:8]]} != {wc[bad[:8]]}"


def _oracle_chunk_records(sm, chunks):
    """The oracle's records of the last chunk: {(layer, site): [rows in token order]}."""
    lib = load_oracle()
    lib.or_set_trace.argtypes = [TRACE_FN, ctypes.c_void_p]
    seq = OracleModel(lib, sm).new_seq()
    for ch in chunks[:-1]:
        assert seq.prefill(ch) == (0, len(ch))
    recs = {}

    def hook(user, layer, site, codes, n, m, e):
        recs.setdefault((layer, site), []).append((np.ctypeslib.as_array(codes, shape=(n,)).copy(), (m, e)))

    cb = TRACE_FN(hook)
    lib.or_set_trace(cb, None)
    try:
        assert seq.prefill(chunks[-1]) == (0, len(chunks[-1]))
    finally:
        lib.or_set_trace(ctypes.cast(None, TRACE_FN), None)
    return recs


def _check_prefill(sm, art, hip_lib, chunks, what):
    c = sm.config
    want = _oracle_chunk_records(sm, chunks)
    L = hip_lib.lib
    _bind_capture(L)
    model = Model(hip_lib, art)
    assert L.sslm_hip_debug_capture(model.handle, max(len(ch) for ch in chunks)) == 0
    pool = model.pool(1)
    seq = pool.seq()
    for ch in chunks:
        assert seq.prefill(ch, chunk_budget=len(ch)) == len(ch)
    _compare_capture(L, model, c, want, len(chunks[-1]), what)
    assert L.sslm_hip_debug_capture(model.handle, 0) == 0
    seq.release()
    pool.close()
    model.close()


@pytest.mark.parametrize("name", ["small", "medium"])
def test_prefill_sites_match_oracle_toy(name, hip_lib):
    """Every site of every layer of a prefill span, token by token: a 13-token prompt in one span,
    and the same prompt as 9 + 4 (the second span's rows)."""
    sm, art = synthetic(name)
    rng = np.random.default_rng(91)
    prompt = rng.integers(0, sm.config.vocab, size=13)
    print(f"case prefill site capture {name}", flush=True)
    _check_prefill(sm, art, hip_lib, [prompt], f"{name} one span")
    _check_prefill(sm, art, hip_lib, [prompt[:9], prompt[9:]], f"{name} second span")


@pytest.mark.timeout(900)
def test_prefill_sites_match_oracle_15b(hip_lib):
    """The 1.5B shape: a 64-token chunk, 28 layers x 11 sites x 64 tokens (the prefill GEMM,
    tiled attention, q landing, residual and SiLU kernels at their real shapes)."""
    sm = W.model_15b()
    rng = np.random.default_rng(92)
    prompt = rng.integers(0, sm.config.vocab, size=64)
    print("case prefill site capture 1.5B", flush=True)
    _check_prefill(sm, sm.to_array(), hip_lib, [prompt], "1.5B 64-token chunk")


def _oracle_decode_records(sm, prompt):
    """The oracle's records of one whole-depth decode call after `prompt` and its logits call."""
    lib = load_oracle()
    lib.or_set_trace.argtypes = [TRACE_FN, ctypes.c_void_p]
    seq = OracleModel(lib, sm).new_seq()
    assert seq.prefill(prompt) == (0, len(prompt))
    assert seq.decode_step(sm.config.layers)[0] == 0  # logits only
    recs = {}

    def hook(user, layer, site, codes, n, m, e):
        recs.setdefault((layer, site), []).append((np.ctypeslib.as_array(codes, shape=(n,)).copy(), (m, e)))

    cb = TRACE_FN(hook)
    lib.or_set_trace(cb, None)
    try:
        assert seq.decode_step(sm.config.layers)[0] == 0
    finally:
        lib.or_set_trace(ctypes.cast(None, TRACE_FN), None)
    return recs


@pytest.mark.parametrize("name", ["small", "medium"])
def test_decode_sites_match_oracle_whole_depth(name, hip_lib):
    """A batched decode call at layer budget L (every layer in one call, the fused decode attention,
    the packed decode GEMVs): every site of every layer for each of three sequences."""
    sm, art = synthetic(name)
    c = sm.config
    rng = np.random.default_rng(93)
    prompts = [rng.integers(0, c.vocab, size=n) for n in (5, 2, 8)]
    want_each = [_oracle_decode_records(sm, p) for p in prompts]
    want = {k: [w[k][0] for w in want_each] for k in want_each[0]}
    L = hip_lib.lib
    _bind_capture(L)
    model = Model(hip_lib, art)
    assert L.sslm_hip_debug_capture(model.handle, len(prompts)) == 0
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for s, p in zip(seqs, prompts):
        s.prefill(p)
    model.decode_step(seqs, c.layers)  # logits only
    print(f"case decode site capture {name}", flush=True)
    model.decode_step(seqs, c.layers)
    _compare_capture(L, model, c, want, len(prompts), f"{name} decode")
    assert L.sslm_hip_debug_capture(model.handle, 0) == 0
    for s in seqs:
        s.release()
    pool.close()
    model.close()
