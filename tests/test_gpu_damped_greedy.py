"""Damped-greedy decoding (SSLM_DECODE_MODE_DAMPED_GREEDY: top-k i-exp renormalization, anti-LM
n-gram penalty; src/damped_greedy_topk.cpp, src/damped_greedy_antilm.cpp, src/sslm_abi.cpp:
2004-2035, 2301-2384, 2462-2485) against the compiled reference: defaults, parameter
validation, tokens, KV and the anti-LM history carried by the SSB3 blob."""
import ctypes

import numpy as np
import pytest

from superslm_amd.sslm import Model
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic, with_flags, with_weight_rows

pytestmark = pytest.mark.gpu

_ART = {}


def damped_artifact(name, scale=1.0 / 20000):
    """A synthetic artifact with the damped-greedy constants section (flag bit 1)."""
    key = (name, scale)
    if key not in _ART:
        sm = build_synthetic(CONFIGS[name], seed=7, damped_logit_scale=scale)
        _ART[key] = (sm, sm.to_bytes())
    return _ART[key]


def _fields(p):
    return (p.layer_budget, p.struct_size, p.mode, p.alpha_q15, p.anti_lm_max_order, p.top_k, p.q_ln2, p.q_b,
            p.q_c)


def test_damped_params_init_matches_reference(hip_lib, ref_lib):
    sm, art = damped_artifact("tiny")
    got = {}
    for lib in (ref_lib, hip_lib):
        m = Model(lib, art)
        got[lib.path] = [(st, _fields(p)) for st, p in (m.decode_params(1, 1, raw=True),
                                                         m.decode_params(sm.config.layers, 1, raw=True),
                                                         m.decode_params(1, 0, raw=True))]
        m.close()
    r, h = got[ref_lib.path], got[hip_lib.path]
    assert r[0][0] == 0 and r[0][1][6] > 0
    assert h == r


def _run(lib, art, prompts, steps, budget, params_fn, save=False):
    model = Model(lib, art)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for sq, p in zip(seqs, prompts):
        sq.prefill(p)
    params = params_fn(model, budget)
    toks = [model.decode_step(seqs, budget, params=params) for _ in range(steps)]
    kv = [pool.kv_block(i).copy() for i in range(len(prompts))]
    blobs = [sq.save() for sq in seqs] if save else None
    for sq in seqs:
        sq.release()
    pool.close()
    model.close()
    return toks, kv, blobs


def _damped(model, budget):
    return model.decode_params(budget, 1)


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_damped_decode_matches_reference(name, hip_lib, ref_lib):
    sm, art = damped_artifact(name)
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (4, 9, 2)]
    L = sm.config.layers
    for budget in sorted({1, L}):
        steps = 8 * L // budget
        print(f"case damped {name} budget={budget}", flush=True)
        r = _run(ref_lib, art, prompts, steps, budget, _damped, save=True)
        h = _run(hip_lib, art, prompts, steps, budget, _damped, save=True)
        assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
        for i in range(len(prompts)):
            assert np.array_equal(h[1][i], r[1][i]), f"KV of sequence {i} differs"
            assert h[2][i] == r[2][i], f"blob of sequence {i} differs (anti-LM history)"
        if name == "small":  # its greedy continuations repeat, so the anti-LM penalty bites
            g = _run(ref_lib, art, prompts, steps, budget, lambda m, b: m.decode_params(b, 0))
            assert g[0] != r[0], "damping changed no token: the test would not see it"


def _run_raw(lib, art, prompts, steps, budget, top_k):
    """Decode with damped greedy at `top_k`: per step (status, tokens), then every KV block."""
    model = Model(lib, art)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for sq, p in zip(seqs, prompts):
        sq.prefill(p)
    out = []
    for _ in range(steps):
        params = model.decode_params(budget, 1)
        params.top_k = top_k
        out.append(model.decode_step(seqs, budget, raw=True, params=params))
    kv = [pool.kv_block(i).copy() for i in range(len(prompts))]
    for sq in seqs:
        sq.release()
    pool.close()
    model.close()
    return out, kv


@pytest.mark.parametrize("tied", [False, True])
@pytest.mark.parametrize("top_k", [1, 37, 1024, 1500])
def test_damped_candidate_sets_match_reference(top_k, tied, hip_lib, ref_lib):
    """The device's top-k candidate set (k <= 1024; above that whole rows come back) against the
    reference's partial sort, on a 4096-token vocabulary; `tied`: the LM head's rows repeat every
    64, so every logit value occurs 64 times and the cut at k falls inside runs of equal logits
    (ordered by index)."""
    sm, art = damped_artifact("medium")
    if tied:
        head = sm.weights["lm_head"]
        art = with_weight_rows(sm, "lm_head", {r: head[r % 64] for r in range(64, sm.config.vocab)})
    rng = np.random.default_rng(top_k)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (5, 3)]
    L = sm.config.layers
    print(f"case damped top_k={top_k} tied={tied}", flush=True)
    r = _run_raw(ref_lib, art, prompts, 6, L, top_k)
    h = _run_raw(hip_lib, art, prompts, 6, L, top_k)
    assert h[0] == r[0], f"statuses / tokens differ: hip {h[0]} ref {r[0]}"
    for i in range(len(prompts)):
        assert np.array_equal(h[1][i], r[1][i]), f"KV of sequence {i} differs"


def test_damped_restore_continues_like_reference(hip_lib, ref_lib):
    sm, art = damped_artifact("tiny")
    prompt = np.random.default_rng(8).integers(0, sm.config.vocab, size=6)
    L = sm.config.layers
    r = _run(ref_lib, art, [prompt], 5, L, _damped, save=True)
    blob = r[2][0]
    assert int.from_bytes(blob[108:112], "little") == 2  # the anti-LM order travels
    outs = {}
    for lib in (ref_lib, hip_lib):
        model = Model(lib, art)
        pool = model.pool(1)
        seq = pool.restore(blob)
        p = model.decode_params(L, 1)
        outs[lib.path] = [model.decode_step([seq], L, params=p)[0] for _ in range(5)], seq.save()
        seq.release()
        pool.close()
        model.close()
    assert outs[hip_lib.path] == outs[ref_lib.path]


def test_damped_param_rejections_match_reference(hip_lib, ref_lib):
    from conftest import synthetic
    sm, art = damped_artifact("tiny")
    _, plain = synthetic("tiny")
    V, L = sm.config.vocab, sm.config.layers
    cases = [("alpha<0", "alpha_q15", -1), ("alpha 2^20", "alpha_q15", 1 << 20), ("order 0", "anti_lm_max_order", 0),
             ("top_k 0", "top_k", 0), ("top_k>V", "top_k", V + 1), ("top_k V", "top_k", V), ("mode 2", "mode", 2),
             ("q_ln2 0", "q_ln2", 0), ("q_c<0", "q_c", -1), ("ok", None, None)]
    statuses = {}
    for lib in (ref_lib, hip_lib):
        res = {}
        model = Model(lib, art)
        pool = model.pool(1)
        seq = pool.seq()
        seq.prefill([1, 2, 3])
        for label, field, value in cases:
            p = model.decode_params(L, 1)
            if field:
                setattr(p, field, value)
            st, _ = model.decode_step([seq], L, raw=True, params=p)
            res[label] = st
        seq.release()
        pool.close()
        model.close()
        # no constants in the artifact
        m2 = Model(lib, plain)
        res["init without constants"] = m2.decode_params(L, 1, raw=True)[0]
        pool2 = m2.pool(1)
        s2 = pool2.seq()
        s2.prefill([1, 2, 3])
        p = m2.decode_params(L, 0)
        p.mode, p.alpha_q15, p.anti_lm_max_order, p.top_k = 1, 1000, 2, 4
        p.q_ln2, p.q_b, p.q_c = 1000, 2000, 3000
        res["decode without constants"] = m2.decode_step([s2], L, raw=True, params=p)[0]
        s2.release()
        pool2.close()
        m2.close()
        # flag bit 1 set but no constants section: the artifact is rejected
        flagged = with_flags(plain, 2)
        buf = ctypes.create_string_buffer(flagged, len(flagged))
        h = ctypes.c_void_p()
        res["flag without section"] = lib.lib.sslm_model_map(buf, len(flagged), ctypes.byref(h))
        statuses[lib.path] = res
    print(statuses[ref_lib.path], flush=True)
    assert statuses[hip_lib.path] == statuses[ref_lib.path]
    assert statuses[ref_lib.path]["ok"] == 0
