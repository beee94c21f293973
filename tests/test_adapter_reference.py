"""Synthetic LoRA adapters (superslm_amd/sslm_artifact.py build_adapter) against the compiled
reference (oracle/_ref): the reference's own loader must accept them (which validates the
writer: ADP1 record, tensor names and shapes, fold domains), reject them for another base, and
their deltas must change the forward (so the GPU parity tests compare a non-trivial path)."""
import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import Model, SslmError
from superslm_amd.sslm_artifact import build_adapter

SSLM_ARTIFACT_REJECTED = 4  # include/sslm_hip.h (reference sslm_abi.h:96-152)
SSLM_ADAPTER_MODEL_MISMATCH = 5


def _decode(ref_lib, art, adapter_bytes, prompt, steps, L):
    model = Model(ref_lib, art)
    ad = model.adapter(adapter_bytes) if adapter_bytes is not None else None
    pool = model.pool(1)
    seq = pool.seq()
    if ad:
        seq.set_adapter(ad)
    seq.prefill(prompt)
    toks = []
    while len(toks) < steps:
        out = model.decode_step([seq], L)[0]
        if out >= 0:
            toks.append(out)
    kv = pool.kv_block(0).copy()
    seq.release()
    pool.close()
    if ad:
        ad.release()
    model.close()
    return toks, kv


@pytest.mark.parametrize("targets", [("q_proj", "v_proj"), ("q_proj", "o_proj", "gate_proj", "up_proj",
                                                            "down_proj", "k_proj", "v_proj")])
def test_reference_accepts_and_applies_adapter(ref_lib, targets):
    sm, art = synthetic("tiny")
    adapter = build_adapter(sm, rank=8, targets=targets, seed=5)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, sm.config.vocab, size=9)
    base = _decode(ref_lib, art, None, prompt, 4, sm.config.layers)
    with_ad = _decode(ref_lib, art, adapter, prompt, 4, sm.config.layers)
    assert not np.array_equal(base[1], with_ad[1]), "the adapter left every KV byte unchanged"


def test_reference_rejects_adapter_of_another_base(ref_lib):
    sm, art = synthetic("tiny")
    sm2, _ = synthetic("tiny", seed=8)
    other = build_adapter(sm2, rank=4, seed=1)
    model = Model(ref_lib, art)
    try:
        with pytest.raises(SslmError) as e:
            model.adapter(other)
        assert e.value.status == SSLM_ADAPTER_MODEL_MISMATCH
        bad = bytearray(build_adapter(sm, rank=4, seed=1))
        with pytest.raises(SslmError) as e:
            model.adapter(bytes(bad[:-7]))  # truncated container
        assert e.value.status == SSLM_ARTIFACT_REJECTED
    finally:
        model.close()
