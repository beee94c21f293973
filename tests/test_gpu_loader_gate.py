"""Loader value gate: malformed and out-of-domain artifacts through sslm_model_map of both
libraries.  The reference rejects over degrading (src/artifact.cpp:229-410 container checks,
src/model.cpp:940-1180 typed sections and value domains, docs/sslm_format.md); every case here
must get the reference's status from the HIP backend too, and a model that maps must run."""
import struct

import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import SslmError, Model
from superslm_amd.sslm_artifact import CONFIGS, build_synthetic, with_flags

pytestmark = pytest.mark.gpu

HEADER = 64
DESC = 40


def _sections(art):
    count = struct.unpack_from("<I", art, 12)[0]
    out = {}
    for i in range(count):
        typ, dt, off, size = struct.unpack_from("<IIQQ", art, HEADER + i * DESC)
        out.setdefault(typ, (i, off, size))
    return out


def _patch(art, off, fmt, value, rehash=True):
    b = bytearray(art)
    struct.pack_into(fmt, b, off, value)
    b = bytes(b)
    return with_flags(b, struct.unpack_from("<I", b, 16)[0]) if rehash else b


def _cfg(art, field_off, value):
    _, off, _ = _sections(art)[0]
    return _patch(art, off + field_off, "<I", value)


def _edited(fn, name="tiny"):
    def edit(m):
        fn(m)
    return build_synthetic(CONFIGS[name], seed=7, edit=edit).to_bytes()


def _set(d, key, row, col, value):
    a = np.array(d[key])
    a[row, col] = value
    d[key] = a


def cases():
    _, art = synthetic("tiny")
    secs = _sections(art)
    w_idx, w_off, w_size = secs[2]
    yield "valid", art
    yield "bad sha", bytes(art[:w_off + 100]) + bytes([art[w_off + 100] ^ 1]) + bytes(art[w_off + 101:])
    yield "truncated", art[:-100]
    yield "short header", art[:40]
    yield "bad magic", _patch(art, 0, "<4s", b"SSLX")
    yield "bad version", _patch(art, 4, "<I", 3)
    yield "section beyond file", _patch(art, HEADER + w_idx * DESC + 8, "<Q", len(art) + 64)
    yield "section size beyond file", _patch(art, HEADER + w_idx * DESC + 16, "<Q", w_size + len(art))
    yield "cfg hidden 0", _cfg(art, 8, 0)
    yield "cfg head_dim odd", _cfg(art, 24, 31)
    yield "cfg tie 2", _cfg(art, 40, 2)
    yield "cfg kv int16", _cfg(art, 44, 1)
    yield "cfg kv precision 2", _cfg(art, 44, 2)
    yield "cfg kv block 0", _cfg(art, 48, 0)
    yield "cfg reserved", _cfg(art, 64, 1)
    yield "cfg vocab mismatch", _cfg(art, 32, 513)
    yield "cfg layers 3", _cfg(art, 12, 3)
    yield "cfg heads 3", _cfg(art, 16, 3)
    yield "wsc1 shift 32", _edited(lambda m: _set(m.folds, "layer0.q_proj", 0, 2, 32))
    yield "wsc1 shift -1", _edited(lambda m: _set(m.folds, "layer1.down_proj", 5, 2, -1))
    yield "wsc1 identity 2", _edited(lambda m: _set(m.folds, "layer0.o_proj", 3, 0, 2))
    yield "wsc1 mult negative", _edited(lambda m: _set(m.folds, "layer0.gate_proj", 1, 1, -5))

    def landing(key, idx, value):
        def f(m):
            v = list(m.landing[key])
            v[idx] = value
            m.landing[key] = tuple(v)
        return f
    yield "kvc1 R 2^31", _edited(landing("layer0.k_head0", 2, 1 << 31))
    yield "kvc1 R above 2^32", _edited(landing("layer1.v_head1", 2, (1 << 32) + 1))
    yield "kvc1 landing m below 2^30", _edited(landing("layer0.v_head0", 0, (1 << 30) - 1))

    def rope(v):
        def f(m):
            m.rope_cos = m.rope_cos.copy()
            m.rope_cos[3, 1] = v
        return f
    yield "rop1 above 2^30", _edited(rope((1 << 30) + 1))
    yield "rop1 below -2^30", _edited(rope(-(1 << 30) - 1))

    def const(key, value):
        def f(m):
            m.consts[key] = value
        return f
    yield "site mantissa below 2^30", _edited(const("layer0.q_proj", ((1 << 30) - 1, -40)))
    yield "site mantissa 2^31", _edited(const("layer1.mlp_act", (1 << 31, -40)))
    yield "embed site exponent", _edited(const("embed", (1 << 30, 100)))

    def silu(i, v):
        def f(m):
            m.silu = m.silu.copy()
            m.silu[i] = v
        return f
    yield "sil1 node out of range", _edited(silu(0, -1))
    yield "sil1 last node", _edited(silu(1024, 1 << 16))


def _map_status(lib, art):
    try:
        model = Model(lib, art)
    except SslmError as e:
        return e.status, None
    return 0, model


@pytest.fixture(scope="module")
def statuses(hip_lib, ref_lib):
    out = {}
    for name, art in cases():
        print(f"case loader {name}", flush=True)
        row = []
        for lib in (ref_lib, hip_lib):
            st, model = _map_status(lib, art)
            if model is not None:  # a model that maps must run a token
                pool = model.pool(1)
                seq = pool.seq()
                st = seq.prefill([1, 2, 3], raw=True)[0]
                row.append(("mapped", st, model.decode_step([seq], 2, raw=True), model.block_size))
                seq.release()
                pool.close()
                model.close()
            else:
                row.append(("rejected", st))
        out[name] = row
    return out


# Deliberate divergence: the reference never checks the embedding / LM-head tensor shapes
# against CFG1's vocab (src/sslm_abi.cpp:637-663), so with vocab above the tensor's rows it maps
# the artifact and then reads past the tensor for ids at or beyond its rows.  This backend uploads
# each tensor by its manifest shape and refuses such an artifact (SSLM_ARTIFACT_REJECTED).
DIVERGENT = {"cfg vocab mismatch"}


def test_loader_statuses_match_reference(statuses):
    bad = {k: v for k, v in statuses.items() if v[0] != v[1] and k not in DIVERGENT}
    assert not bad, f"status differs (reference, hip): {bad}"
    for k in DIVERGENT:
        assert statuses[k][0][0] == "mapped" and statuses[k][1] == ("rejected", 4), statuses[k]


def test_loader_rejects_the_reference_rejects(statuses):
    rejected = [k for k, v in statuses.items() if v[0][0] == "rejected"]
    assert len(rejected) >= 20, rejected
    assert statuses["valid"][0][0] == "mapped"
