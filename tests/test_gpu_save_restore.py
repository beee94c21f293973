"""Sequence save/restore (SSB3 blob, src/sslm_abi.cpp:2585-2987) against the compiled reference.

Blobs must be byte-identical in every resting state (fresh, after prefill, mid-token, between
decode steps). A restored sequence must continue exactly as the reference's restored sequence
does, whether the HIP backend restores its own blob or the reference's. Malformed blobs must be
refused with the reference's status, in the reference's check order."""
import ctypes
import struct

import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu


def _states(lib, art, prompt, L):
    """Blobs of one sequence at each resting state, in order."""
    model = Model(lib, art)
    pool = model.pool(1)
    seq = pool.seq()
    blobs = {"fresh": seq.save()}
    seq.prefill(prompt)
    blobs["prefill"] = seq.save()  # ready for logits: the first decode call runs no layers
    assert model.decode_step([seq], 1)[0] >= 0
    blobs["between"] = seq.save()  # resting between decode steps, the next token to embed
    if L > 1:
        assert model.decode_step([seq], 1)[0] == -1  # first layer of the next token
        blobs["mid"] = seq.save()
    while model.decode_step([seq], L)[0] < 0:
        pass
    blobs["between2"] = seq.save()
    st, need = seq.save_size()
    seq.release()
    pool.close()
    model.close()
    return blobs, (st, need)


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_save_blobs_match_reference(name, hip_lib, ref_lib):
    sm, art = synthetic(name)
    prompt = np.random.default_rng(3).integers(0, sm.config.vocab, size=9)
    L = sm.config.layers
    print(f"case save {name}", flush=True)
    r, r_size = _states(ref_lib, art, prompt, L)
    h, h_size = _states(hip_lib, art, prompt, L)
    assert h_size == r_size  # SSLM_BUFFER_TOO_SMALL and the required size
    for k in r:
        assert len(h[k]) == len(r[k]), k
        if h[k] != r[k]:
            diff = np.nonzero(np.frombuffer(h[k], np.uint8) != np.frombuffer(r[k], np.uint8))[0]
            pytest.fail(f"blob '{k}' differs at {diff[:8]} ({len(diff)} bytes)")


def _continue(lib, art, blob, L, budget, steps):
    """Restore `blob` into a fresh pool and decode `steps` tokens at `budget` layers per call."""
    model = Model(lib, art)
    pool = model.pool(1)
    seq = pool.restore(blob)
    toks = []
    while len(toks) < steps:
        out = model.decode_step([seq], budget)[0]
        if out >= 0:
            toks.append(out)
    kv = pool.kv_block(0).copy()
    again = seq.save()
    seq.release()
    pool.close()
    model.close()
    return toks, kv, again


@pytest.mark.parametrize("name", ["tiny", "small"])
def test_restore_continues_like_reference(name, hip_lib, ref_lib):
    sm, art = synthetic(name)
    prompt = np.random.default_rng(4).integers(0, sm.config.vocab, size=7)
    L = sm.config.layers
    r_blobs, _ = _states(ref_lib, art, prompt, L)
    h_blobs, _ = _states(hip_lib, art, prompt, L)
    for state in ("prefill", "between", "mid", "between2"):
        for budget in sorted({1, L}):
            print(f"case restore {name} {state} budget={budget}", flush=True)
            r = _continue(ref_lib, art, r_blobs[state], L, budget, 3)
            h_own = _continue(hip_lib, art, h_blobs[state], L, budget, 3)
            h_ref = _continue(hip_lib, art, r_blobs[state], L, budget, 3)
            for h in (h_own, h_ref):
                assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
                assert np.array_equal(h[1], r[1]), "KV differs"
                assert h[2] == r[2], "re-saved blob differs"


def _mutations(blob, other_blob, H, cap, L):
    """(label, bytes) of malformed or foreign blobs derived from a valid mid-token SSB3 blob."""
    b = bytearray(blob)

    def with_(off, fmt, v):
        x = bytearray(b)
        struct.pack_into(fmt, x, off, v)
        return bytes(x)

    ssb2 = bytearray(b[:108] + b[120:])
    ssb2[0:4] = b"SSB2"
    yield "short", bytes(b[:3])
    yield "magic", b"SSB1" + bytes(b[4:])
    yield "header only", bytes(b[:120])
    yield "model hash", bytes(other_blob[:36]) + bytes(b[36:])
    yield "kv precision", with_(36, "<I", 1)
    yield "schema hash", with_(40, "<Q", 12345)
    yield "walk state", with_(48, "<I", 0)
    yield "context over cap", with_(60, "<q", cap + 1)
    yield "negative context", with_(60, "<q", -1)
    yield "layer over depth", with_(68, "<I", L + 1)
    yield "negative anti-LM order", with_(108, "<i", -1)
    yield "history without order", with_(112, "<Q", 1)
    yield "history over context", bytes(with_(108, "<i", 2)[:112]) + struct.pack("<Q", 10 ** 6) + bytes(b[120:])
    yield "block count", bytes(b[:120 + H]) + struct.pack("<I", 2) + bytes(b[124 + H:])
    yield "truncated block", bytes(b[:-1])
    yield "ssb2", bytes(ssb2)
    yield "ssb2 truncated", bytes(ssb2[:-5])
    yield "valid", bytes(b)


def test_restore_rejections_match_reference(hip_lib, ref_lib):
    sm, art = synthetic("tiny")
    _, other = synthetic("tiny", seed=8)
    prompt = np.random.default_rng(5).integers(0, sm.config.vocab, size=5)
    c = sm.config
    r_blobs, _ = _states(ref_lib, art, prompt, c.layers)
    other_blobs, _ = _states(ref_lib, other, prompt, c.layers)
    for lib in (ref_lib, hip_lib):
        lib.statuses = {}
        model = Model(lib, art)
        pool = model.pool(1)
        for label, blob in _mutations(r_blobs["mid"], other_blobs["mid"], c.hidden, c.context_cap, c.layers):
            st, seq = pool.restore(blob, raw=True)
            lib.statuses[label] = st
            if seq is not None:
                seq.release()
        # a pool of another mapping of the same artifact (same hash, another model handle)
        m2 = Model(lib, art)
        p2 = m2.pool(1)
        blob = r_blobs["mid"]
        buf = ctypes.create_string_buffer(blob, len(blob))
        h = ctypes.c_void_p()
        lib.statuses["pool of another model"] = lib.lib.sslm_seq_restore(
            model.handle, ctypes.byref(p2.handle), buf, len(blob), ctypes.byref(h))
        # an exhausted pool
        held = pool.seq()
        st, seq = pool.restore(r_blobs["mid"], raw=True)
        lib.statuses["pool exhausted"] = st
        held.release()
        p2.close()
        m2.close()
        pool.close()
        model.close()
    print(ref_lib.statuses, flush=True)
    assert hip_lib.statuses == ref_lib.statuses
    assert ref_lib.statuses["valid"] == 0 and ref_lib.statuses["ssb2"] == 0
    assert ref_lib.statuses["pool of another model"] != 0 and ref_lib.statuses["pool exhausted"] != 0
