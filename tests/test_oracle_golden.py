"""The C oracle against the golden vectors of the reference's own unit tests
(tests/golden/reference_fixtures.json, extracted by tests/golden/make_fixtures.py).

Each table names the reference fixture it comes from; a mismatch here means the oracle
restates the reference's arithmetic wrongly, before any GPU result is compared with it."""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

from oracle_bind import load_oracle

HERE = os.path.dirname(os.path.abspath(__file__))
FX = json.load(open(os.path.join(HERE, "golden", "reference_fixtures.json")))

c_i64p = ctypes.POINTER(ctypes.c_int64)
c_i8p = ctypes.POINTER(ctypes.c_int8)


class Scale(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int64), ("e", ctypes.c_int64)]


@pytest.fixture(scope="module")
def orc():
    L = load_oracle()
    sig = {
        "or_srdhm": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32]),
        "or_rdbpot32": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int]),
        "or_mbqm": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int]),
        "or_clz64": (ctypes.c_int, [ctypes.c_uint64]),
        "or_max_abs_wide": (ctypes.c_int64, [c_i64p, ctypes.c_size_t]),
        "or_normalize_scale": (ctypes.c_int64, [ctypes.c_int64, ctypes.POINTER(ctypes.c_int)]),
        "or_reciprocal": (ctypes.c_int64, [ctypes.c_int64]),
        "or_requant_code_wide": (ctypes.c_int8, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int]),
        "or_isqrt": (ctypes.c_int64, [ctypes.c_int64]),
        "or_iexp_construct": (ctypes.c_int, [ctypes.c_int64] * 4 + [c_i64p, c_i64p]),
        "or_iexp_evaluate": (ctypes.c_int64, [ctypes.c_int64] * 3),
        "or_iexp_scale_constants": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                                   ctypes.c_int64, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                                   c_i64p, c_i64p, c_i64p]),
        "or_iexp_pinned": (None, [c_i64p, c_i64p, c_i64p]),
        "or_rope_pair": (None, [ctypes.c_int32] * 4 + [c_i64p, c_i64p]),
        "or_check_softmax_width": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t]),
        "or_landing_rescale": (ctypes.c_int64, [ctypes.c_int64] * 5 + [ctypes.POINTER(ctypes.c_uint64),
                                                                       ctypes.POINTER(ctypes.c_int)]),
        "or_gemm_i8": (None, [c_i8p, c_i8p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, c_i64p]),
        "or_requant_chain": (ctypes.c_int, [c_i64p, ctypes.c_size_t, ctypes.POINTER(Scale), ctypes.c_size_t, Scale,
                                            c_i8p, ctypes.POINTER(Scale)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def i64(a):
    a = np.ascontiguousarray(a, dtype=np.int64)
    return a, a.ctypes.data_as(c_i64p)


def i8(a):
    a = np.ascontiguousarray(a, dtype=np.int8)
    return a, a.ctypes.data_as(c_i8p)


def gemm(orc, acts, wgts, m, k, n):
    a, ap = i8(acts)
    w, wp = i8(wgts)
    out = np.zeros(m * n, dtype=np.int64)
    orc.or_gemm_i8(ap, wp, m, k, n, out.ctypes.data_as(c_i64p))
    return out


# --- tests/sslm_intmath_fixtures.h ------------------------------------------------------
def test_srdhm(orc):
    for c in FX["srdhm"]:
        assert orc.or_srdhm(c["a"], c["b"]) == c["expected"], c["label"]


def test_rdbpot(orc):
    for c in FX["rdbpot"]:
        assert orc.or_rdbpot32(c["x"], c["exponent"]) == c["expected"], c["label"]


def test_mbqm(orc):
    for c in FX["mbqm"]:
        assert orc.or_mbqm(c["x"], c["multiplier"], c["shift"]) == c["expected"], c["label"]


def test_clz64(orc):
    for c in FX["clz64"]:
        assert orc.or_clz64(c["n"]) == c["expected"], c["label"]


def test_max_abs(orc):
    for c in FX["max_abs"] + FX["max_abs_wide"]:
        a, p = i64(c["data"])
        assert orc.or_max_abs_wide(p, len(a)) == c["expected"], c["label"]


def test_normalize_scale(orc):
    for c in FX["normalize_scale"]:
        s = ctypes.c_int()
        assert orc.or_normalize_scale(c["d_prime"], ctypes.byref(s)) == c["expected_dn"], c["label"]
        assert s.value == c["expected_s"], c["label"]


def test_reciprocal(orc):
    for c in FX["reciprocal_named"] + FX["reciprocal_dense"]:
        assert orc.or_reciprocal(c["dn"]) == c["expected_r"], c


def test_requant(orc):
    for c in FX["requant"] + FX["requant_wide"]:
        assert orc.or_requant_code_wide(c["x_i"], c["r"], c["s"]) == c["expected"], c["label"]


def _funnel_steps(orc, xs):
    a, p = i64(xs)
    d = orc.or_max_abs_wide(p, len(a))
    s = ctypes.c_int()
    dn = orc.or_normalize_scale(max(d, 1), ctypes.byref(s))
    r = orc.or_reciprocal(dn)
    codes = [orc.or_requant_code_wide(int(x), r, s.value) for x in a]
    return d, dn, s.value, r, codes


def test_requant_pipeline(orc):
    """D' -> NormalizeScale -> DynamicScaleReciprocal -> per-element codes (the funnel's
    element half)."""
    for c in FX["pipeline"]:
        d, dn, s, r, codes = _funnel_steps(orc, c["xs"])
        assert (d, dn, s, r) == (c["expected_d_prime"], c["expected_dn"], c["expected_s"], c["expected_r"]), c["label"]
        assert codes == c["expected_codes"], c["label"]


def test_isqrt(orc):
    for c in FX["isqrt"]:
        assert orc.or_isqrt(c["n"]) == c["expected_root"], c["label"]


def test_iexp(orc):
    for c in FX["iexp"]:
        z, b = ctypes.c_int64(), ctypes.c_int64()
        st = orc.or_iexp_construct(c["q"], c["q_ln2"], c["q_b"], c["q_c"], ctypes.byref(z), ctypes.byref(b))
        assert st in (0, 1), c["label"]
        assert orc.or_iexp_evaluate(z.value, b.value, c["q_c"]) == c["expected"], c["label"]


def test_rope_pair(orc):
    for c in FX["rope"]:
        x, y = ctypes.c_int64(), ctypes.c_int64()
        orc.or_rope_pair(c["x"], c["y"], c["cos_q30"], c["sin_q30"], ctypes.byref(x), ctypes.byref(y))
        assert (x.value, y.value) == (c["expected_x"], c["expected_y"]), c["label"]


# --- tests/sslm_iexp_domain_fixtures.h, sslm_s3_1_c30_iexp_domain_sweep_fixtures.h ----------
IEXP_DOMAIN = {"kOk": 0, "kNotRepresentable": 1, "kBadQ": 2, "kBadQLn2": 3, "kBadQB": 4}


def test_iexp_construct(orc):
    for c in FX["iexp_construct"]:
        z, b = ctypes.c_int64(), ctypes.c_int64()
        st = orc.or_iexp_construct(c["q"], c["q_ln2"], c["q_b"], c["q_c"], ctypes.byref(z), ctypes.byref(b))
        assert st == IEXP_DOMAIN[c["expected_domain"]], c["label"]
        if st in (0, 1):
            assert (z.value, b.value) == (c["expected_z"], c["expected_base"]), c["label"]
            assert orc.or_iexp_evaluate(z.value, b.value, c["q_c"]) == c["expected_value"], c["label"]


def test_iexp_in_domain(orc):
    for c in FX["iexp_domain"]:
        z, b = ctypes.c_int64(), ctypes.c_int64()
        st = orc.or_iexp_construct(c["q"], c["q_ln2"], c["q_b"], c["q_c"], ctypes.byref(z), ctypes.byref(b))
        assert (st == 0) == c["expected_in_domain"], c["label"]


def test_iexp_scale_constants_sweep(orc):
    """IExpScaleConstants over the (m, e) sweep: where the fixture's derivation succeeds the
    oracle's triple equals it, and the q = 0 domain verdict matches."""
    ln2, bq, ca = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    orc.or_iexp_pinned(ctypes.byref(ln2), ctypes.byref(bq), ctypes.byref(ca))
    checked = 0
    for c in FX["iexp_scale_sweep"]:
        q = [ctypes.c_int64() for _ in range(3)]
        st = orc.or_iexp_scale_constants(c["m"], c["e"], ln2.value, 30, bq.value, 30, ca.value, 30,
                                         *[ctypes.byref(x) for x in q])
        if not c["derivation_ok"]:
            continue
        assert st == 0, c
        assert [x.value for x in q] == [c["q_ln2"], c["q_b"], c["q_c"]], c
        z, b = ctypes.c_int64(), ctypes.c_int64()
        dom = orc.or_iexp_construct(0, c["q_ln2"], c["q_b"], c["q_c"], ctypes.byref(z), ctypes.byref(b))
        assert (dom == 0) == c["expected_in_domain"], c
        checked += 1
    assert checked > 100


# --- tests/sslm_s3_3_fixtures.h, sslm_s3_3_rope_application_site_fixtures.h ---------------
def test_softmax_width_gate(orc):
    """Accept iff the row peak M = q_b^2 + q_c is within 2^47 and width * M fits int64 (the
    verdict rule of the reference's test, test_main.cpp:10755-10760), band witness included."""
    for c in FX["softmax_width"] + FX["softmax_width_band"]:
        assert c["row_max"] == c["q_b"] ** 2 + c["q_c"]
        ok = orc.or_check_softmax_width(c["q_b"], c["q_c"], c["width"]) == 0
        expect = c["ok_under_2pow47"] and (c["row_max"] <= 0 or c["width"] <= (2 ** 63 - 1) // c["row_max"])
        assert ok == expect, c["label"]


def test_landing_composite(orc):
    for c in FX["landing"]:
        sat, exc = ctypes.c_uint64(0), ctypes.c_int(0)
        raw = orc.or_landing_rescale(c["branch_code"], c["m_b"], c["r_h"], c["e_b"], c["e_h"], ctypes.byref(sat),
                                     ctypes.byref(exc))
        assert raw == c["correct_raw"], c["label"]
        assert max(-127, min(127, raw)) == c["correct"], c["label"]


def test_rope_application_site(orc):
    for c in FX["rope_site"]:
        out = []
        for i in range(64):
            x, y = ctypes.c_int64(), ctypes.c_int64()
            orc.or_rope_pair(c["row"][2 * i], c["row"][2 * i + 1], c["cos_row"][i], c["sin_row"][i], ctypes.byref(x),
                             ctypes.byref(y))
            out += [max(-127, min(127, x.value)), max(-127, min(127, y.value))]
        assert out == c["expected_out"], c["label"]


# --- tests/sslm_matmul_fixtures.h, tests/matmul_golden_pin.h ------------------------------
def test_matmul_rows_and_tails(orc):
    for c in FX["matmul_rows"] + FX["matmul_tail"]:
        got = gemm(orc, c["activations"], c["weights"], 1, c["in_channels"], c["out_channels"])
        assert got.tolist() == c["expected"], c["label"]


def test_matmul_multirow(orc):
    for c in FX["matmul_multirow"]:
        got = gemm(orc, c["activations"], c["weights"], c["num_tokens"], c["in_channels"], c["out_channels"])
        assert got.tolist() == c["expected"], c["label"]


def test_matmul_uniform(orc):
    for c in FX["matmul_uniform"]:
        k = c["in_channels"]
        got = gemm(orc, np.full(k, c["act_value"]), np.full(k, c["wgt_value"]), 1, k, 1)
        assert int(got[0]) == c["expected"], c["label"]


def test_matmul_composition(orc):
    """GEMM -> int32 row -> funnel element half, against independently built goldens."""
    for c in FX["matmul_composition"]:
        got = gemm(orc, c["activations"], c["weights"], 1, c["in_channels"], c["out_channels"])
        assert got.tolist() == c["golden_i32"], c["label"]
        d, dn, s, r, codes = _funnel_steps(orc, c["golden_i32"])
        assert (d, dn, s, r) == (c["expected_d_prime"], c["expected_dn"], c["expected_s"], c["expected_r"]), c["label"]
        assert codes == c["expected_codes"], c["label"]


def _lcg_bytes(seed, n):
    out = np.empty(n, dtype=np.uint8)
    x = seed
    mask = (1 << 64) - 1
    for i in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) & mask
        out[i] = x >> 56
    return out


def test_matmul_golden_hash(orc):
    """The reference's cross-platform matmul golden: 13 cases (real 1.5B shapes, tails, K up to
    4,194,305 past int32) whose int64 accumulators, scalar row-0 dot and narrowed int32 rows
    hash to one pinned SHA-256 (matmul_golden_pin.h; stream layout test_main.cpp:7261-7313)."""
    assert _lcg_bytes(1, 16).tolist() == FX["matmul_golden_lcg_probe"]
    stream = bytearray()
    for c in FX["matmul_golden"]:
        m, k, n = c["num_tokens"], c["in_channels"], c["out_channels"]
        if c["kind"] == 1:
            acts = np.tile(np.where(np.arange(k) % 2 == 0, 127, -127), m)
            jk = np.add.outer(np.arange(n), np.arange(k))
            wgts = np.where(jk % 2 == 0, 127, -128).ravel()
        elif c["kind"] in (2, 3):
            acts = np.full(m * k, 127 if c["kind"] == 2 else -127)
            wgts = np.full(n * k, -128)
        else:
            b = _lcg_bytes(c["seed"], m * k + n * k)
            acts = (b[:m * k].astype(np.int64) % 255) - 127
            wgts = b[m * k:].astype(np.int64) - 128
        wide = gemm(orc, acts, wgts, m, k, n)
        stream += wide.astype("<i8").tobytes()
        stream += np.int64(int(np.dot(acts[:k].astype(np.int64), wgts[:k].astype(np.int64)))).astype("<i8").tobytes()
        if c["int32_safe"]:
            stream += wide[:n].astype("<i4").tobytes()
    assert len(stream) == FX["matmul_golden_total_bytes"]
    assert hashlib.sha256(bytes(stream)).hexdigest() == FX["matmul_golden_sha256"]


# --- tests/silu_lut_golden_table.h ----------------------------------------------------------
def test_silu_table_generator():
    """The artifact writer's SIL1 table is the reference's canonical sigmoid table."""
    from superslm_amd.sslm_artifact import sigmoid_lut
    assert np.asarray(sigmoid_lut()).tolist() == FX["silu_table"]
