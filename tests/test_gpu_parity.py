"""HIP backend vs the compiled reference and the C oracle, through the sslm_* C ABI.

Bit-exact bar: every produced token, every KV byte (the reference's own block layout) after
prefill and after decode, at every layer budget and chunk split tried."""
import ctypes

import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu


def _run(lib, artifact, prompt, steps, budget, chunk=None):
    model = Model(lib, artifact)
    pool = model.pool(1)
    seq = pool.seq()
    consumed = seq.prefill(prompt, chunk_budget=chunk)
    kv_after_prefill = pool.kv_block(0).copy()
    toks = []
    while len(toks) < steps:
        out = model.decode_step([seq], budget)[0]
        if out >= 0:
            toks.append(out)
    kv = pool.kv_block(0).copy()
    seq.release()
    pool.close()
    model.close()
    return consumed, kv_after_prefill, toks, kv


@pytest.mark.parametrize("name", ["tiny", "small", "medium"])
def test_prefill_decode_matches_reference(name, hip_lib, ref_lib):
    sm, art = synthetic(name)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, sm.config.vocab, size=20)
    L = sm.config.layers
    for budget in sorted({L, 1, max(1, L - 1)}):  # small: 2 of 3 layers per call as well
        print(f"case {name} budget={budget}", flush=True)
        r = _run(ref_lib, art, prompt, 6, budget)
        h = _run(hip_lib, art, prompt, 6, budget)
        assert h[0] == r[0]
        assert np.array_equal(h[1], r[1]), "KV after prefill differs"
        assert h[2] == r[2], f"tokens differ: hip {h[2]} ref {r[2]}"
        assert np.array_equal(h[3], r[3]), "KV after decode differs"


def test_chunk_split_invariance(hip_lib, ref_lib):
    sm, art = synthetic("tiny")
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, sm.config.vocab, size=17)
    r = _run(ref_lib, art, prompt, 4, sm.config.layers)
    for chunk in (1, 5, 17):
        print(f"case chunk={chunk}", flush=True)
        model = Model(hip_lib, art)
        pool = model.pool(1)
        seq = pool.seq()
        done = 0
        while done < len(prompt):
            done += seq.prefill(prompt[done:], chunk_budget=chunk)
        toks = []
        while len(toks) < 4:
            out = model.decode_step([seq], sm.config.layers)[0]
            if out >= 0:
                toks.append(out)
        assert toks == r[2]
        assert np.array_equal(pool.kv_block(0), r[3])
        seq.release()
        pool.close()
        model.close()


def _run_batch(lib, artifact, prompts, steps, budget):
    model = Model(lib, artifact)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for sq, p in zip(seqs, prompts):
        sq.prefill(p)
    toks = [model.decode_step(seqs, budget) for _ in range(steps)]
    kv = [pool.kv_block(i).copy() for i in range(len(prompts))]
    for sq in seqs:
        sq.release()
    pool.close()
    model.close()
    return toks, kv


@pytest.mark.parametrize("name", ["small", "medium"])
def test_batched_decode_matches_reference(name, hip_lib, ref_lib):
    """Several sequences of different lengths decoded together (one GEMV row per sequence, token
    groups on concurrent streams)."""
    sm, art = synthetic(name)
    rng = np.random.default_rng(23)
    # 13 sequences: split over several concurrent token groups (tracks) of at least 4 tokens
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (3, 9, 1, 14, 6, 2, 11, 5, 7, 4, 8, 12, 10)]
    L = sm.config.layers
    for budget in sorted({L, 1}):
        print(f"case batch {name} budget={budget}", flush=True)
        r = _run_batch(ref_lib, art, prompts, 4 * L // budget, budget)
        h = _run_batch(hip_lib, art, prompts, 4 * L // budget, budget)
        assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
        for i in range(len(prompts)):
            assert np.array_equal(h[1][i], r[1][i]), f"KV of sequence {i} differs"


@pytest.mark.parametrize("name,n", [("small", 150), ("medium", 90)])
def test_long_prefill_chunk_matches_reference(name, n, hip_lib, ref_lib):
    """Prefill chunks of more than 64 tokens run the tiled MFMA GEMM (split-K partial planes for
    the narrow projections); every KV byte and the following tokens must still match."""
    sm, art = synthetic(name)
    rng = np.random.default_rng(31)
    prompt = rng.integers(0, sm.config.vocab, size=n)
    L = sm.config.layers
    print(f"case long prefill {name} n={n}", flush=True)
    r = _run(ref_lib, art, prompt, 3, L)
    h = _run(hip_lib, art, prompt, 3, L)
    assert h[0] == r[0]
    assert np.array_equal(h[1], r[1]), "KV after prefill differs"
    assert h[2] == r[2], f"tokens differ: hip {h[2]} ref {r[2]}"
    assert np.array_equal(h[3], r[3]), "KV after decode differs"


ALL_PROJ = ("q_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "k_proj", "v_proj")


def _run_lora(lib, artifact, adapter_blobs, prompts, script, budget):
    """Sequences with adapters (index into `adapter_blobs` or None) decoded together; `script` is a
    list of (step count, {sequence: adapter index or None}) phases -- the attachments change
    between tokens, as sslm_seq_set_adapter allows.  Returns every phase's tokens and the KV."""
    model = Model(lib, artifact)
    ads = [model.adapter(b) for b in adapter_blobs]
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    toks = []
    for phase, (steps, attach) in enumerate(script):
        for i, a in attach.items():
            seqs[i].set_adapter(ads[a] if a is not None else None)
        if phase == 0:
            for sq, p in zip(seqs, prompts):
                sq.prefill(p)
        for _ in range(steps):
            toks.append(model.decode_step(seqs, budget))
    kv = [pool.kv_block(i).copy() for i in range(len(prompts))]
    for sq in seqs:
        sq.release()
    pool.close()
    for a in ads:
        a.release()
    model.close()
    return toks, kv


@pytest.mark.parametrize("name,targets,rank", [("small", ("q_proj", "v_proj"), 16), ("tiny", ALL_PROJ, 8),
                                               ("medium", ALL_PROJ, 16)])
def test_lora_adapter_matches_reference(name, targets, rank, hip_lib, ref_lib):
    """LoRA side-GEMMs (u = amp_fold(A.x), delta = amp_fold(B.u)) on the adapted projections,
    with a swap between tokens: adapter 0 on every sequence, then sequence 0 detached and
    sequence 1 moved to adapter 1, mixed with an unadapted sequence in the same batch."""
    from superslm_amd.sslm_artifact import build_adapter
    sm, art = synthetic(name)
    blobs = [build_adapter(sm, rank=rank, targets=targets, seed=s) for s in (5, 6)]
    rng = np.random.default_rng(41)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (7, 12, 4)]
    L = sm.config.layers
    for budget in sorted({L, 1}):
        # phases end on token boundaries (the first call after prefill only produces logits;
        # a token takes L / budget calls), where sslm_seq_set_adapter accepts a swap
        script = [(1 + 2 * (L // budget), {0: 0, 1: 0, 2: None}), (2 * (L // budget), {0: None, 1: 1})]
        print(f"case lora {name} targets={len(targets)} rank={rank} budget={budget}", flush=True)
        r = _run_lora(ref_lib, art, blobs, prompts, script, budget)
        h = _run_lora(hip_lib, art, blobs, prompts, script, budget)
        assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
        for i in range(len(prompts)):
            assert np.array_equal(h[1][i], r[1][i]), f"KV of sequence {i} differs"


@pytest.mark.parametrize("name,n", [("small", 90)])
def test_lora_long_prefill_matches_reference(name, n, hip_lib, ref_lib):
    """A prefill chunk of more than 64 tokens with every projection adapted (the tiled GEMM with
    the LoRA epilogue, the batched u side-GEMM)."""
    from superslm_amd.sslm_artifact import build_adapter
    sm, art = synthetic(name)
    blob = build_adapter(sm, rank=16, targets=ALL_PROJ, seed=9)
    rng = np.random.default_rng(43)
    prompt = rng.integers(0, sm.config.vocab, size=n)
    L = sm.config.layers
    print(f"case lora long prefill {name} n={n}", flush=True)
    script = [(3, {0: 0})]
    r = _run_lora(ref_lib, art, [blob], [prompt], script, L)
    h = _run_lora(hip_lib, art, [blob], [prompt], script, L)
    assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
    assert np.array_equal(h[1][0], r[1][0]), "KV differs"


def test_adapter_map_rejections_match_reference(hip_lib, ref_lib):
    """sslm_adapter_map statuses: another base's adapter, a truncated container."""
    from superslm_amd.sslm import SslmError
    from superslm_amd.sslm_artifact import build_adapter
    sm, art = synthetic("tiny")
    sm2, _ = synthetic("tiny", seed=8)
    good = build_adapter(sm, rank=4, seed=1)
    cases = {"other base": build_adapter(sm2, rank=4, seed=1), "truncated": good[:-7]}
    statuses = {}
    for lib_name, lib in (("ref", ref_lib), ("hip", hip_lib)):
        model = Model(lib, art)
        for case, blob in cases.items():
            try:
                model.adapter(blob).release()
                statuses[(lib_name, case)] = 0
            except SslmError as e:
                statuses[(lib_name, case)] = e.status
        model.close()
    for case in cases:
        assert statuses[("hip", case)] == statuses[("ref", case)] != 0, (case, statuses)


def test_option_g_flag_matches_reference(hip_lib, ref_lib):
    """Artifact flag bit 0 (Option-G fused K landing, src/artifact.cpp:511-513).  The reference's
    C ABI never enables it: prefill passes option_g_fused_k_landing = false
    (src/sslm_abi.cpp:1535-1540) and decode runs the RunLayerLoop overload that fixes it to false
    (forward_sites.cpp:2018-2031).  Both libraries accept the flagged artifact and run the
    plain landing; tokens and KV must agree."""
    from superslm_amd.sslm_artifact import with_flags
    sm, plain = synthetic("tiny")
    art = with_flags(plain, 1)
    assert art[16] == 1 and art[32:64] != plain[32:64]
    prompt = np.random.default_rng(12).integers(0, sm.config.vocab, size=11)
    L = sm.config.layers
    for budget in sorted({1, L}):
        print(f"case option-g budget={budget}", flush=True)
        r = _run(ref_lib, art, prompt, 5, budget)
        h = _run(hip_lib, art, prompt, 5, budget)
        p = _run(hip_lib, plain, prompt, 5, budget)
        assert h[0] == r[0]
        assert np.array_equal(h[1], r[1]), "KV after prefill differs"
        assert h[2] == r[2], f"tokens differ: hip {h[2]} ref {r[2]}"
        assert np.array_equal(h[3], r[3]), "KV after decode differs"
        assert h[2] == p[2] and np.array_equal(h[3], p[3])  # the flag changes nothing at the ABI


@pytest.mark.parametrize("waves", ["4", "8"])
def test_tiled_prefill_attention_matches_reference(waves, hip_lib, ref_lib, monkeypatch):
    """Prefill attention runs over 16-token query tiles in 4- or 8-wave blocks (the grid size picks
    one; SSLM_HIP_TILED_WAVES forces it): ragged last tiles and chunks that start mid-sequence
    (D = 128) must leave every KV byte and the following tokens as the reference does."""
    monkeypatch.setenv("SSLM_HIP_TILED_WAVES", waves)
    sm, art = synthetic("medium")
    rng = np.random.default_rng(77)
    prompt = rng.integers(0, sm.config.vocab, size=90)  # the context cap is 96
    L = sm.config.layers
    r = _run(ref_lib, art, prompt, 3, L)
    for chunk in (90, 37):
        print(f"case tiled attention waves={waves} chunk={chunk}", flush=True)
        model = Model(hip_lib, art)
        pool = model.pool(1)
        seq = pool.seq()
        done = 0
        while done < len(prompt):
            done += seq.prefill(prompt[done:], chunk_budget=chunk)
        kv = pool.kv_block(0).copy()
        toks = []
        while len(toks) < 3:
            out = model.decode_step([seq], L)[0]
            if out >= 0:
                toks.append(out)
        assert np.array_equal(kv, r[1]), "KV after prefill differs"
        assert toks == r[2], f"tokens differ: hip {toks} ref {r[2]}"
        seq.release()
        pool.close()
        model.close()


@pytest.mark.parametrize("halves", ["1", "2"])
@pytest.mark.parametrize("name", ["tiny", "small", "medium"])
def test_grouped_decode_attention_matches_reference(name, halves, hip_lib, ref_lib, monkeypatch):
    """Decode attention forced to one block per (sequence, KV head), the group's query heads the
    rows of the MFMA tiles (G = 2, 4, 4; D = 32, 64, 128), or two blocks per group each taking half
    of its heads (halves "2"): tokens and every KV byte as the reference, at budget 1 and at the
    full depth, decoding past the prompt."""
    monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", "1")
    monkeypatch.setenv("SSLM_HIP_GROUP_HALVES", halves)
    sm, art = synthetic(name)
    rng = np.random.default_rng(23)
    prompt = rng.integers(0, sm.config.vocab, size=40)
    L = sm.config.layers
    for budget in sorted({1, L}):
        print(f"case grouped attention {name} halves={halves} budget={budget}", flush=True)
        r = _run(ref_lib, art, prompt, 8, budget)
        h = _run(hip_lib, art, prompt, 8, budget)
        assert np.array_equal(h[1], r[1]), "KV after prefill differs"
        assert h[2] == r[2], f"tokens differ: hip {h[2]} ref {r[2]}"
        assert np.array_equal(h[3], r[3]), "KV after decode differs"
