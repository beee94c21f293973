"""The C oracle against the reference compiled from its own sources (oracle/_ref, built by
oracle/Makefile where the reference tree exists; these tests skip elsewhere).

Pins what the golden vectors leave open: the composed funnel scale (CombineCarriedScale's
left fold), IExpScaleConstants over random scales, LandingRescale's branches, the RMSNorm,
MlpAct and residual sites, bias reconcile, the SiLU lookup, and whole-model prefill/decode
(tokens and every KV byte) at several layer budgets and chunk splits."""
import ctypes
import os

import numpy as np
import pytest

from conftest import synthetic
from oracle_bind import REF_SO, OracleModel, load_oracle

i64p = ctypes.POINTER(ctypes.c_int64)
i32p = ctypes.POINTER(ctypes.c_int32)
i8p = ctypes.POINTER(ctypes.c_int8)
u64p = ctypes.POINTER(ctypes.c_uint64)
intp = ctypes.POINTER(ctypes.c_int)

pytestmark = pytest.mark.skipif(not os.path.exists(REF_SO), reason="compiled reference (oracle/_ref) not built")


class Scale(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int64), ("e", ctypes.c_int64)]


def _p(a, t):
    return a.ctypes.data_as(t)


@pytest.fixture(scope="module")
def libs():
    ref = ctypes.CDLL(REF_SO)
    orc = load_oracle()
    S = Scale
    for name, res, args in [
        ("ref_requant_chain", ctypes.c_int, [i64p, ctypes.c_size_t, i64p, ctypes.c_size_t, ctypes.c_int64,
                                             ctypes.c_int64, i8p, i64p]),
        ("ref_reciprocal", ctypes.c_int64, [ctypes.c_int64]),
        ("ref_iexp_scale_constants", ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, i64p]),
        ("ref_softmax_row", ctypes.c_int, [i64p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                           i64p]),
        ("ref_check_softmax_width", ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t]),
        ("ref_landing_rescale", ctypes.c_int64, [ctypes.c_int64] * 5 + [u64p, intp]),
        ("ref_rmsnorm", ctypes.c_int, [i8p, i32p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64, i8p, i64p]),
        ("ref_mlp_act", ctypes.c_int, [i8p, ctypes.c_int64, ctypes.c_int64, i8p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64, i8p, i64p]),
        ("ref_residual", ctypes.c_int, [i8p, ctypes.c_int64, ctypes.c_int64, i8p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64, i8p, i64p]),
        ("ref_silu_sigmoid", ctypes.c_int32, [ctypes.c_int8, ctypes.c_int64, ctypes.c_int]),
        ("ref_silu_table", ctypes.c_void_p, []),
        ("ref_apply_fold", ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
        ("ref_apply_amp_fold", ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
        ("ref_bias_reconcile_wide", ctypes.c_int, [ctypes.c_int64] * 4 + [i64p]),
        ("ref_rope_pair", None, [ctypes.c_int32] * 4 + [i64p]),
    ]:
        fn = getattr(ref, name)
        fn.restype, fn.argtypes = res, args
    for name, res, args in [
        ("or_requant_chain", ctypes.c_int, [i64p, ctypes.c_size_t, ctypes.POINTER(S), ctypes.c_size_t, S, i8p,
                                            ctypes.POINTER(S)]),
        ("or_reciprocal", ctypes.c_int64, [ctypes.c_int64]),
        ("or_iexp_scale_constants", ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                                   ctypes.c_int64, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                                   i64p, i64p, i64p]),
        ("or_iexp_pinned", None, [i64p, i64p, i64p]),
        ("or_softmax_row_q15", ctypes.c_int, [i64p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_int64, i64p]),
        ("or_check_softmax_width", ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t]),
        ("or_landing_rescale", ctypes.c_int64, [ctypes.c_int64] * 5 + [u64p, intp]),
        ("or_rmsnorm_site", ctypes.c_int, [i8p, i32p, ctypes.c_size_t, S, i8p, ctypes.POINTER(S)]),
        ("or_mlp_act_site", ctypes.c_int, [i8p, S, i8p, S, ctypes.c_size_t, i32p, S, i8p, ctypes.POINTER(S)]),
        ("or_residual_site", ctypes.c_int, [i8p, S, i8p, S, ctypes.c_size_t, S, i8p, ctypes.POINTER(S)]),
        ("or_silu_sigmoid_q15", ctypes.c_int32, [i32p, ctypes.c_int8, ctypes.c_int64, ctypes.c_int]),
        ("or_apply_fold", ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
        ("or_apply_amp_fold", ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
        ("or_bias_reconcile_wide", ctypes.c_int, [ctypes.c_int64] * 4 + [i64p]),
        ("or_rope_pair", None, [ctypes.c_int32] * 4 + [i64p, i64p]),
    ]:
        fn = getattr(orc, name)
        fn.restype, fn.argtypes = res, args
    table = np.ctypeslib.as_array(ctypes.cast(ref.ref_silu_table(), i32p), shape=(1025,)).copy()
    return ref, orc, table


def rand_scale(rng, canonical=True):
    if canonical or rng.random() < 0.8:
        m = int(rng.integers(1 << 30, 1 << 31))
    else:
        m = int(rng.choice([0, 1, -5, (1 << 31) - 1, 1 << 31, -(1 << 31), 1 << 32, 12345]))
    return m, int(rng.integers(-80, 10))


def test_requant_chain_fuzz(libs):
    ref, orc, _ = libs
    rng = np.random.default_rng(1)
    for it in range(3000):
        n = int(rng.integers(1, 40))
        mag = int(rng.choice([1, 100, 1 << 20, 1 << 31, (1 << 31) + 1, 1 << 40]))
        row = rng.integers(-mag, mag + 1, size=n, dtype=np.int64)
        if rng.random() < 0.05:
            row[:] = 0
        n_in = int(rng.integers(0, 3))
        inc = [rand_scale(rng, canonical=rng.random() < 0.9) for _ in range(n_in)]
        site = rand_scale(rng, canonical=rng.random() < 0.95)
        inc_arr = np.array(inc or [(0, 0)], dtype=np.int64).ravel()
        c_ref, me_ref = np.zeros(n, np.int8), np.zeros(2, np.int64)
        st_ref = ref.ref_requant_chain(_p(row, i64p), n, _p(inc_arr, i64p), n_in, site[0], site[1],
                                       _p(c_ref, i8p), _p(me_ref, i64p))
        c_or, sc = np.zeros(n, np.int8), Scale()
        inc_s = (Scale * max(1, n_in))(*[Scale(*x) for x in inc])
        st_or = orc.or_requant_chain(_p(row, i64p), n, inc_s, n_in, Scale(*site), _p(c_or, i8p), ctypes.byref(sc))
        assert st_or == st_ref, (it, row.tolist(), inc, site)
        if st_ref == 0:
            assert np.array_equal(c_or, c_ref), it
            assert (sc.m, sc.e) == tuple(me_ref), it


def test_reciprocal_full_domain(libs):
    ref, orc, _ = libs
    rng = np.random.default_rng(2)
    dns = np.concatenate([rng.integers(1 << 30, 1 << 31, size=20000), rng.integers(-(1 << 31), 1 << 31, size=4000),
                          [1 << 30, (1 << 31) - 1, (1 << 30) + 1, 0, -1, -(1 << 31)]])
    for dn in dns:
        assert orc.or_reciprocal(int(dn)) == ref.ref_reciprocal(int(dn)), dn


def test_iexp_scale_constants_and_softmax_rows(libs):
    ref, orc, _ = libs
    rng = np.random.default_rng(3)
    ln2, bq, ca = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    orc.or_iexp_pinned(ctypes.byref(ln2), ctypes.byref(bq), ctypes.byref(ca))
    accepted = 0
    for it in range(2000):
        m, e = int(rng.integers(1 << 30, 1 << 31)), int(rng.integers(-75, -20))
        r3 = np.zeros(3, np.int64)
        st_ref = ref.ref_iexp_scale_constants(m, e, _p(r3, i64p))
        q = [ctypes.c_int64() for _ in range(3)]
        st_or = orc.or_iexp_scale_constants(m, e, ln2.value, 30, bq.value, 30, ca.value, 30,
                                            *[ctypes.byref(x) for x in q])
        assert (st_or == 0) == (st_ref == 0), (m, e)
        if st_ref != 0:
            continue
        assert [x.value for x in q] == r3.tolist(), (m, e)
        width = int(rng.integers(1, 300))
        assert orc.or_check_softmax_width(r3[1], r3[2], width) == ref.ref_check_softmax_width(r3[1], r3[2], width)
        if ref.ref_check_softmax_width(r3[1], r3[2], width) != 0:
            continue
        scores = rng.integers(-(1 << 20), 1 << 20, size=width, dtype=np.int64)
        scores -= scores.max()
        p_ref, p_or = np.zeros(width, np.int64), np.zeros(width, np.int64)
        ok_ref = ref.ref_softmax_row(_p(scores, i64p), width, *[int(x) for x in r3], _p(p_ref, i64p))
        ok_or = orc.or_softmax_row_q15(_p(scores, i64p), width, *[int(x) for x in r3], _p(p_or, i64p))
        assert bool(ok_or) == bool(ok_ref), (m, e)
        if ok_ref:
            assert np.array_equal(p_or, p_ref), (m, e)
            accepted += 1
    assert accepted > 200


def test_landing_rescale_branches(libs):
    ref, orc, _ = libs
    rng = np.random.default_rng(4)
    for it in range(20000):
        branch = int(rng.choice([rng.integers(-127, 128), rng.integers(-(1 << 31), 1 << 31),
                                 rng.integers(-(1 << 62), 1 << 62)]))
        m_a = int(rng.choice([rng.integers(1 << 30, 1 << 31), -int(rng.integers(1 << 30, 1 << 31)),
                              rng.integers(-(1 << 40), 1 << 40)]))
        r_t = int(rng.choice([rng.integers((1 << 31) + 1, (1 << 32) + 1), rng.integers(1, 1 << 40)]))
        e_a, e_t = int(rng.integers(-200, 200)), int(rng.integers(-200, 200))
        if rng.random() < 0.01:
            e_a = int(rng.choice([-(1 << 62), 1 << 62]))
        s1, s2 = ctypes.c_uint64(0), ctypes.c_uint64(0)
        x1, x2 = ctypes.c_int(0), ctypes.c_int(0)
        v_ref = ref.ref_landing_rescale(branch, m_a, r_t, e_a, e_t, ctypes.byref(s1), ctypes.byref(x1))
        v_or = orc.or_landing_rescale(branch, m_a, r_t, e_a, e_t, ctypes.byref(s2), ctypes.byref(x2))
        assert (v_or, s2.value, x2.value) == (v_ref, s1.value, x1.value), (branch, m_a, r_t, e_a, e_t)


def test_row_sites(libs):
    """RMSNorm, MlpAct and residual sites on random rows and scales."""
    ref, orc, table = libs
    rng = np.random.default_rng(5)
    for it in range(600):
        n = int(rng.integers(1, 300))
        h = rng.integers(-127, 128, size=n).astype(np.int8)
        if rng.random() < 0.05:
            h[:] = 0
        g = rng.integers(-(1 << 17), 1 << 17, size=n).astype(np.int32)
        site = rand_scale(rng, canonical=rng.random() < 0.95)
        o_ref, me = np.zeros(n, np.int8), np.zeros(2, np.int64)
        st_ref = ref.ref_rmsnorm(_p(h, i8p), _p(g, i32p), n, site[0], site[1], _p(o_ref, i8p), _p(me, i64p))
        o_or, sc = np.zeros(n, np.int8), Scale()
        st_or = orc.or_rmsnorm_site(_p(h, i8p), _p(g, i32p), n, Scale(*site), _p(o_or, i8p), ctypes.byref(sc))
        assert st_or == st_ref, it
        if st_ref == 0:
            assert np.array_equal(o_or, o_ref) and (sc.m, sc.e) == tuple(me), it

        up = rng.integers(-127, 128, size=n).astype(np.int8)
        gs, us = rand_scale(rng, rng.random() < 0.9), rand_scale(rng)
        gs = (gs[0], int(rng.integers(-40, 4)))
        st_ref = ref.ref_mlp_act(_p(h, i8p), gs[0], gs[1], _p(up, i8p), us[0], us[1], n, site[0], site[1],
                                 _p(o_ref, i8p), _p(me, i64p))
        st_or = orc.or_mlp_act_site(_p(h, i8p), Scale(*gs), _p(up, i8p), Scale(*us), n, _p(table, i32p),
                                    Scale(*site), _p(o_or, i8p), ctypes.byref(sc))
        assert st_or == st_ref, it
        if st_ref == 0:
            assert np.array_equal(o_or, o_ref) and (sc.m, sc.e) == tuple(me), it

        bs, ss = rand_scale(rng, rng.random() < 0.9), rand_scale(rng, rng.random() < 0.9)
        st_ref = ref.ref_residual(_p(h, i8p), bs[0], bs[1], _p(up, i8p), ss[0], ss[1], n, site[0], site[1],
                                  _p(o_ref, i8p), _p(me, i64p))
        st_or = orc.or_residual_site(_p(h, i8p), Scale(*bs), _p(up, i8p), Scale(*ss), n, Scale(*site),
                                     _p(o_or, i8p), ctypes.byref(sc))
        assert st_or == st_ref, it
        if st_ref == 0:
            assert np.array_equal(o_or, o_ref) and (sc.m, sc.e) == tuple(me), it


def test_scalar_sites(libs):
    """SiLU lookup, WSC1 / amplifying folds, bias reconcile and RoPE pairs."""
    ref, orc, table = libs
    rng = np.random.default_rng(6)
    for it in range(20000):
        code = int(rng.integers(-128, 128))
        m, e = int(rng.integers(1 << 30, 1 << 31)), int(rng.integers(-60, 5))
        assert orc.or_silu_sigmoid_q15(_p(table, i32p), code, m, e) == ref.ref_silu_sigmoid(code, m, e)
        acc = int(rng.integers(-(1 << 40), 1 << 40))
        ident, mult = int(rng.random() < 0.1), int(rng.integers(1 << 30, 1 << 31))
        shift, ex = int(rng.integers(0, 32)), int(rng.integers(-31, 32))
        assert orc.or_apply_fold(acc, ident, mult, shift) == ref.ref_apply_fold(acc, ident, mult, shift)
        assert orc.or_apply_amp_fold(acc, ident, mult, ex) == ref.ref_apply_amp_fold(acc, ident, mult, ex)
        b = int(rng.integers(-(1 << 40), 1 << 40))
        r_a, e_a = int(rng.integers((1 << 31) + 1, (1 << 32) + 1)), int(rng.integers(-120, 10))
        o1, o2 = np.zeros(1, np.int64), np.zeros(1, np.int64)
        k1 = ref.ref_bias_reconcile_wide(b, 30, r_a, e_a, _p(o1, i64p))
        k2 = orc.or_bias_reconcile_wide(b, 30, r_a, e_a, _p(o2, i64p))
        assert bool(k1) == bool(k2) and (not k1 or o1[0] == o2[0]), (b, r_a, e_a)
        x, y = int(rng.integers(-(1 << 31), 1 << 31)), int(rng.integers(-(1 << 31), 1 << 31))
        c, s = int(rng.integers(-(1 << 30), (1 << 30) + 1)), int(rng.integers(-(1 << 30), (1 << 30) + 1))
        r2 = np.zeros(2, np.int64)
        ref.ref_rope_pair(x, y, c, s, _p(r2, i64p))
        ox, oy = ctypes.c_int64(), ctypes.c_int64()
        orc.or_rope_pair(x, y, c, s, ctypes.byref(ox), ctypes.byref(oy))
        assert (ox.value, oy.value) == tuple(r2)


def _ref_run(lib, art, prompt, steps, budget, chunk=None):
    from superslm_amd.sslm import Model
    model = Model(lib, art)
    pool = model.pool(1)
    seq = pool.seq()
    done = 0
    while done < len(prompt):
        done += seq.prefill(prompt[done:], chunk_budget=chunk)
    toks = []
    while len(toks) < steps:
        out = model.decode_step([seq], budget)[0]
        if out >= 0:
            toks.append(out)
    kv = pool.kv_block(0).copy()
    seq.release()
    pool.close()
    model.close()
    return toks, kv


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_whole_model_matches_reference(name, oracle_lib, ref_lib):
    """Oracle layer loops, chunked prefill and head against the reference's sslm_* ABI on a
    seeded synthetic artifact: tokens and KV bytes, every layer budget tried."""
    sm, art = synthetic(name)
    om = OracleModel(oracle_lib, sm)
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, sm.config.vocab, size=13)
    L = sm.config.layers
    for budget in sorted({1, L, max(1, L - 1)}):
        seq = om.new_seq()
        assert seq.prefill(prompt) == (0, len(prompt))
        toks = []
        while len(toks) < 5:
            st, t = seq.decode_step(budget)
            assert st == 0
            if t >= 0:
                toks.append(t)
        r_toks, r_kv = _ref_run(ref_lib, art, prompt, 5, budget)
        assert toks == r_toks, (budget, toks, r_toks)
        assert np.array_equal(seq.kv, r_kv), budget
