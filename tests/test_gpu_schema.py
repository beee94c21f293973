"""SCM1 schema masks (include/superslm/schema_masks.h; src/sslm_abi.cpp:1193-1264, 1420-1560,
1791-1818, 2301-2440, 2506-2534) against the compiled reference: the schema table verbs, binding
rules, schema-content prefill along the DFA, masked greedy and damped decoding with the walk
(including the -2 dead end), the binding carried by the SSB3 blob, and malformed tables."""
import ctypes

import numpy as np
import pytest

from superslm_amd.sslm import SPAN_SCHEMA_CONTENT, Model
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic, scm1

pytestmark = pytest.mark.gpu

SCHEMAS = [("cycle", {0: {5: 1, 6: 1, 7: 1}, 1: {5: 1, 8: 2, 9: 2}, 2: {10: 0}}, [2]),
           ("dead_end", {0: {3: 1, 4: 1}}, [1]),
           ("wide", {0: {t: 0 for t in range(100, 300)}}, [0])]
_ART = {}


def schema_artifact(name="tiny"):
    if name not in _ART:
        sm = build_synthetic(CONFIGS[name], seed=7, damped_logit_scale=1.0 / 20000, schemas=SCHEMAS)
        _ART[name] = (sm, sm.to_bytes())
    return _ART[name]


def test_schema_table_verbs_match_reference(hip_lib, ref_lib):
    sm, art = schema_artifact()
    res = {}
    for lib in (ref_lib, hip_lib):
        m = Model(lib, art)
        r = [m.schema_count()]
        for nm in ("cycle", "dead_end", "wide", "nope", "cycl"):
            r.append(m.schema(nm)[0])
        for i in (0, 1, 2, 3, -1):
            r.append(m.schema_name(i))
            r.append(m.schema_name(i, 4))
            r.append(m.schema_name(i, 64))
        res[lib.path] = r
        m.close()
    print(res[ref_lib.path], flush=True)
    assert res[hip_lib.path] == res[ref_lib.path]


def _script(lib, art, schema, L, budget, mode, steps=10):
    """Bind `schema`, prefill a prompt and a schema-content span, decode; everything observable."""
    m = Model(lib, art)
    pool = m.pool(2)
    seq, other = pool.seq(), pool.seq()
    log = []
    st, h = m.schema(schema)
    log.append(("bind", seq.set_schema(h)))
    log.append(("span unbound", other.prefill([1, 2], raw=True, kind=SPAN_SCHEMA_CONTENT)))
    other.prefill([1, 2])
    log.append(("bind after prompt", other.set_schema(h)))
    log.append(("prompt", seq.prefill([11, 12, 13], raw=True)))
    table = dict((n, t) for n, t, _ in SCHEMAS)[schema]
    path = []
    w = 0
    while len(path) < 3 and table.get(w):
        tok = sorted(table[w])[0]
        path.append(tok)
        w = table[w][tok]
    log.append(("span", seq.prefill(path + [2], raw=True, kind=SPAN_SCHEMA_CONTENT)))  # 2 has no transition
    log.append(("stats", m.stats(seq)))
    log.append(("blob", seq.save()))
    p = m.decode_params(budget, mode)
    # (status, token): a dead end answers -2, and a token left at the last layer by it is refused
    # on the call after (the layer loop's guard), with the output untouched
    toks = [m.decode_step([seq], budget, raw=True, params=p) for _ in range(steps * L // budget)]
    log.append(("tokens", toks))
    log.append(("stats after", m.stats(seq)))
    log.append(("kv", pool.kv_block(0).tobytes()))
    log.append(("blob after", seq.save()))
    seq.release()
    other.release()
    pool.close()
    m.close()
    return log


@pytest.mark.parametrize("schema", ["cycle", "dead_end", "wide"])
def test_schema_prefill_decode_match_reference(schema, hip_lib, ref_lib):
    sm, art = schema_artifact()
    L = sm.config.layers
    for mode in (0, 1):
        for budget in sorted({1, L}):
            print(f"case schema {schema} mode={mode} budget={budget}", flush=True)
            r = _script(ref_lib, art, schema, L, budget, mode)
            h = _script(hip_lib, art, schema, L, budget, mode)
            for (k, rv), (_, hv) in zip(r, h):
                assert hv == rv, f"{k} differs: hip {hv if k != 'kv' else '...'} ref {rv if k != 'kv' else '...'}"
            if schema == "dead_end":
                assert any(-2 in t for _, t in dict(r)["tokens"])


def test_schema_restore_matches_reference(hip_lib, ref_lib):
    sm, art = schema_artifact()
    L = sm.config.layers
    blob = dict(_script(ref_lib, art, "cycle", L, L, 0, steps=2))["blob after"]
    assert blob[40:48] != bytes(8)  # the schema name hash travels
    outs = {}
    for lib in (ref_lib, hip_lib):
        m = Model(lib, art)
        pool = m.pool(1)
        seq = pool.restore(blob)
        outs[lib.path] = ([m.decode_step([seq], L)[0] for _ in range(4)], m.stats(seq), seq.save())
        seq.release()
        pool.close()
        m.close()
    assert outs[hip_lib.path] == outs[ref_lib.path]


def test_malformed_schema_tables_rejected_like_reference(hip_lib, ref_lib):
    vocab = CONFIGS["tiny"].vocab
    good = scm1(vocab, SCHEMAS)
    bad = {
        "magic": b"SCM2" + good[4:],
        "version": good[:4] + (2).to_bytes(4, "little") + good[8:],
        "vocab": good[:12] + (vocab + 1).to_bytes(4, "little") + good[16:],
        "reserved": good[:20] + (1).to_bytes(4, "little") + good[24:],
        "truncated": good[:-8],
        "duplicate name": scm1(vocab, [SCHEMAS[0], SCHEMAS[0]]),
    }
    # a mask bit without its transition: flip token 300's bit in the "wide" schema's page
    off = int.from_bytes(good[24 + 2 * 56 + 24:24 + 2 * 56 + 32], "little")
    flipped = bytearray(good)
    flipped[off + 300 // 8] |= 1 << (300 % 8)
    bad["mask mismatch"] = bytes(flipped)
    from superslm_amd import sslm_artifact as A
    arts = {}
    for label, sec in list(bad.items()) + [("good", good)]:
        orig = A.scm1  # the writer's SchemaMasks payload replaced by the raw section under test
        A.scm1 = lambda v, sch, _sec=sec: _sec
        try:
            arts[label] = build_synthetic(CONFIGS["tiny"], seed=7, schemas=SCHEMAS).to_bytes()
        finally:
            A.scm1 = orig
    statuses = {}
    for lib in (ref_lib, hip_lib):
        res = {}
        for label, art in arts.items():
            buf = ctypes.create_string_buffer(art, len(art))
            h = ctypes.c_void_p()
            res[label] = lib.lib.sslm_model_map(buf, len(art), ctypes.byref(h))
            if res[label] == 0:
                lib.lib.sslm_model_unmap(h)
        statuses[lib.path] = res
    print(statuses[ref_lib.path], flush=True)
    assert statuses[hip_lib.path] == statuses[ref_lib.path]
    assert statuses[ref_lib.path]["good"] == 0


def _mixed(lib, art, L, budget, mode, n=3):
    """One decode batch of `n` sequences cycling through: bound to "cycle", unbound, bound to
    "wide"."""
    m = Model(lib, art)
    pool = m.pool(n)
    seqs = [pool.seq() for _ in range(n)]
    names = ("cycle", None, "wide")
    prompts = ([11, 12], [13, 14, 15], [16])
    for i, sq in enumerate(seqs):
        if names[i % 3]:
            assert sq.set_schema(m.schema(names[i % 3])[1]) == 0
        sq.prefill([t + i for t in prompts[i % 3]])
    p = m.decode_params(budget, mode)
    toks = [m.decode_step(seqs, budget, raw=True, params=p) for _ in range(6 * L // budget)]
    out = (toks, [m.stats(sq) for sq in seqs], [sq.save() for sq in seqs],
           [pool.kv_block(i).tobytes() for i in range(n)])
    for sq in seqs:
        sq.release()
    pool.close()
    m.close()
    return out


def test_mixed_schema_batch_matches_reference(hip_lib, ref_lib):
    sm, art = schema_artifact()
    L = sm.config.layers
    for mode in (0, 1):
        for budget in sorted({1, L}):
            print(f"case mixed mode={mode} budget={budget}", flush=True)
            r = _mixed(ref_lib, art, L, budget, mode)
            h = _mixed(hip_lib, art, L, budget, mode)
            assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
            assert h[1] == r[1] and h[2] == r[2] and h[3] == r[3]


def test_wide_mixed_schema_batch_matches_reference(hip_lib, ref_lib):
    """72 sequences in one call: the LM head runs as a tiled GEMM (more than 64 tokens) with the
    schema masks applied in its argmax epilogue."""
    sm, art = schema_artifact()
    L = sm.config.layers
    for mode in (0, 1):
        print(f"case wide mixed mode={mode}", flush=True)
        r = _mixed(ref_lib, art, L, L, mode, n=72)
        h = _mixed(hip_lib, art, L, L, mode, n=72)
        assert h[0] == r[0], "tokens differ"
        assert h[1] == r[1] and h[2] == r[2] and h[3] == r[3]


def test_mid_mixed_schema_batch_matches_reference(hip_lib, ref_lib):
    """24 sequences in one call: the LM head runs on the packed copy with two 16-token row groups
    (k_gemv_head<2, ...>), the schema masks applied in its argmax epilogue."""
    sm, art = schema_artifact()
    L = sm.config.layers
    for mode in (0, 1):
        print(f"case mid mixed mode={mode}", flush=True)
        r = _mixed(ref_lib, art, L, L, mode, n=24)
        h = _mixed(hip_lib, art, L, L, mode, n=24)
        assert h[0] == r[0], "tokens differ"
        assert h[1] == r[1] and h[2] == r[2] and h[3] == r[3]
