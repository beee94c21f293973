"""The synthetic SCM1 (schema masks) and damped-greedy constants sections, checked on the CPU
against the compiled reference: its loader accepts them, resolves the schemas by name, walks the
DFA on schema-content spans, and derives the damped-greedy decode parameters; corrupted tables
are refused.  (The GPU library is compared with the reference in the gpu-marked tests.)"""
import ctypes

import numpy as np

from superslm_amd.sslm import SPAN_SCHEMA_CONTENT, Model
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic, scm1, with_flags

SCHEMAS = [("cycle", {0: {5: 1, 6: 1, 7: 1}, 1: {5: 1, 8: 2, 9: 2}, 2: {10: 0}}, [2]),
           ("dead_end", {0: {3: 1, 4: 1}}, [1])]


def test_reference_accepts_synthetic_schemas_and_damped_constants(ref_lib):
    sm = build_synthetic(CONFIGS["tiny"], seed=7, damped_logit_scale=1.0 / 20000, schemas=SCHEMAS)
    m = Model(ref_lib, sm.to_bytes())
    assert m.schema_count() == 2
    assert m.schema("cycle")[0] == 0 and m.schema("dead_end")[0] == 0 and m.schema("x")[0] != 0
    assert m.schema_name(1, 64) == (0, b"dead_end")
    st, p = m.decode_params(1, 1, raw=True)
    assert st == 0 and p.top_k == 6 and p.anti_lm_max_order == 2 and p.q_ln2 > 0
    pool = m.pool(1)
    seq = pool.seq()
    assert seq.set_schema(m.schema("cycle")[1]) == 0
    st, n = seq.prefill([5, 8, 10, 7, 2], raw=True, kind=SPAN_SCHEMA_CONTENT)
    assert (st, n) == (23, 4)  # SSLM_SCHEMA_SPAN_UNREACHABLE after the walk 0-5->1-8->2-10->0-7->1
    assert m.stats(seq)[1][2:] == (4, 1, 0)  # 4 forced tokens, one block, state 1 not accepting
    tok = m.decode_step([seq], 1, params=m.decode_params(1, 0))[0]
    assert tok in (5, 8, 9)  # the mask of state 1
    seq.release()
    pool.close()
    m.close()


def test_reference_rejects_corrupt_schema_tables(ref_lib):
    from superslm_amd import sslm_artifact as A
    good = scm1(CONFIGS["tiny"].vocab, SCHEMAS)
    for label, sec in (("magic", b"XCM1" + good[4:]), ("vocab", good[:12] + (7).to_bytes(4, "little") + good[16:]),
                       ("good", good)):
        orig = A.scm1
        A.scm1 = lambda v, s, _sec=sec: _sec
        try:
            art = build_synthetic(CONFIGS["tiny"], seed=7, schemas=SCHEMAS).to_bytes()
        finally:
            A.scm1 = orig
        buf = ctypes.create_string_buffer(art, len(art))
        h = ctypes.c_void_p()
        st = ref_lib.lib.sslm_model_map(buf, len(art), ctypes.byref(h))
        assert (st == 0) == (label == "good"), label
        if st == 0:
            ref_lib.lib.sslm_model_unmap(h)
    flagged = with_flags(build_synthetic(CONFIGS["tiny"], seed=7).to_bytes(), 2)  # flag without section
    buf = ctypes.create_string_buffer(flagged, len(flagged))
    h = ctypes.c_void_p()
    assert ref_lib.lib.sslm_model_map(buf, len(flagged), ctypes.byref(h)) != 0
