"""BASELINE.json configurations 1-4 as parity workloads at their real shapes.

Each workload drives one sslm_* library through the C ABI and returns what it observed: output
tokens, and SHA-256 digests of KV blocks (the reference layout) and SSB3 sequence blobs.  The
same functions run the compiled reference (tests/golden/make_workload_fixtures.py records its
results in tests/golden/workload_fixtures.json) and the HIP backend (tests/test_gpu_workloads.py
compares against that file), so the GPU box needs no CPU reference run at these sizes.

Shapes (sslm_artifact.CONFIGS): "qwen1.5b" (hidden 1536, intermediate 8960, 28 layers, 12 / 2
heads, head_dim 128, vocab 151,936) and "qwen7b" (hidden 3584, intermediate 18944, 28 layers, 28
/ 4 heads).  Weights are seeded uniform int8 codes; prompts are seeded uniform token ids.
"""
from __future__ import annotations

import hashlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from superslm_amd.sslm import Model
from superslm_amd.sslm_artifact import CONFIGS, build_adapter, build_synthetic

SEED_15B = 1515
SEED_7B = 7007
C1_BATCH, C1_PROMPT, C1_CALLS = 16, 32, 8
C2_PROMPT, C2_TOKENS = 512, 128
C3_PROMPT, C3_TOKENS, C3_BASE_TOKENS = 64, 64, 16
C4_PROMPT, C4_TOKENS = 128, 8

_CACHE = {}


def model_15b():
    if "15b" not in _CACHE:
        _CACHE["15b"] = build_synthetic(CONFIGS["qwen1.5b"], seed=SEED_15B)
    return _CACHE["15b"]


def model_7b():
    return build_synthetic(CONFIGS["qwen7b"], seed=SEED_7B)


def sha(data) -> str:
    if isinstance(data, np.ndarray):
        data = data.tobytes()
    return hashlib.sha256(data).hexdigest()


def artifact_hash(sm) -> str:
    """The artifact's own integrity SHA-256 (header bytes 32..64)."""
    return bytes(sm.to_array()[32:64]).hex()


def _decode_tokens(model, seq, budget, n_tokens, first_is_logits=True):
    """Greedy tokens produced by repeated decode calls at `budget` layers per call."""
    toks = []
    while len(toks) < n_tokens:
        t = model.decode_step([seq], budget)[0]
        if t >= 0:
            toks.append(t)
    return toks


def c2_prompt(vocab):
    return np.random.default_rng(2002).integers(0, vocab, size=C2_PROMPT)


def run_c2(lib, sm, chunks, budget):
    """Configuration 2: a 512-token prompt prefilled in `chunks` (list of chunk budgets, cycled
    until the prompt is consumed), then 128 greedy tokens at `budget` layers per call."""
    model = Model(lib, sm.to_array())
    pool = model.pool(1)
    seq = pool.seq()
    prompt = c2_prompt(sm.config.vocab)
    done, k = 0, 0
    while done < len(prompt):
        done += seq.prefill(prompt[done:], chunk_budget=chunks[k % len(chunks)])
        k += 1
    out = {"kv_after_prefill": sha(pool.kv_block(0)), "blob_after_prefill": sha(seq.save())}
    out["tokens"] = _decode_tokens(model, seq, budget, C2_TOKENS)
    out["kv_after_decode"] = sha(pool.kv_block(0))
    out["blob_after_decode"] = sha(seq.save())
    seq.release()
    pool.close()
    model.close()
    return out


def c3_adapters(sm):
    return [build_adapter(sm, rank=16, targets=("q_proj", "v_proj"), seed=s) for s in (31, 32)]


def run_c3(lib, sm, budget):
    """Configuration 3: rank-16 adapters on q_proj and v_proj of all 28 layers.  Adapter A on a
    sequence: 64-token prefill, 64 greedy tokens; the sequence is released and A unmapped; adapter
    B on a new sequence: the same prompt and tokens; finally a sequence with no adapter (the base
    weights untouched: its tokens are the base model's)."""
    model = Model(lib, sm.to_array())
    blobs = c3_adapters(sm)
    prompt = np.random.default_rng(3003).integers(0, sm.config.vocab, size=C3_PROMPT)
    out = {}
    pool = model.pool(1)
    for name, blob, n_tok in (("adapter_a", blobs[0], C3_TOKENS), ("adapter_b", blobs[1], C3_TOKENS),
                              ("base", None, C3_BASE_TOKENS)):
        ad = model.adapter(blob) if blob is not None else None
        seq = pool.seq()
        if ad is not None:
            seq.set_adapter(ad)
        seq.prefill(prompt)
        toks = _decode_tokens(model, seq, budget, n_tok)
        out[name] = {"tokens": toks, "kv": sha(pool.kv_block(0))}
        seq.set_adapter(None)
        seq.release()
        if ad is not None:
            ad.release()
    pool.close()
    model.close()
    return out


def c1_prompts(vocab):
    rng = np.random.default_rng(1001)
    return [rng.integers(0, vocab, size=C1_PROMPT) for _ in range(C1_BATCH)]


def run_c1(lib, sm, batched, threads=1):
    """Configuration 1: 16 sequences with 32-token prompts, then 8 decode calls over the batch
    (28 layers + LM head per call; the first call produces the prompts' next tokens).  `batched`:
    one sslm_decode_step over all 16 per call; otherwise one call per sequence (the reference
    runs its batch sequence by sequence, so the results are the same), spread over `threads`."""
    model = Model(lib, sm.to_array())
    L = sm.config.layers
    pool = model.pool(C1_BATCH)
    seqs = [pool.seq() for _ in range(C1_BATCH)]
    prompts = c1_prompts(sm.config.vocab)
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda sp: sp[0].prefill(sp[1]), zip(seqs, prompts)))
        toks = []
        for _ in range(C1_CALLS):
            if batched:
                toks.append(model.decode_step(seqs, L))
            else:
                toks.append(list(ex.map(lambda s: model.decode_step([s], L)[0], seqs)))
    out = {"tokens": toks, "kv": [sha(pool.kv_block(i)) for i in range(C1_BATCH)]}
    for s in seqs:
        s.release()
    pool.close()
    model.close()
    return out


def run_c1_solo(lib, sm):
    """Configuration 1 at M = 1: the first sequence of the batch alone, 8 decode calls."""
    model = Model(lib, sm.to_array())
    pool = model.pool(1)
    seq = pool.seq()
    seq.prefill(c1_prompts(sm.config.vocab)[0])
    toks = [model.decode_step([seq], sm.config.layers)[0] for _ in range(C1_CALLS)]
    out = {"tokens": toks, "kv": sha(pool.kv_block(0))}
    seq.release()
    pool.close()
    model.close()
    return out


def c4_prompt(vocab):
    return np.random.default_rng(4004).integers(0, vocab, size=C4_PROMPT)


def run_c4(lib, sm, budget, chunk):
    """Configuration 4's shape (7B) at a length the CPU reference affords: one sequence, a
    128-token prompt in chunks of `chunk`, then 8 greedy tokens at `budget` layers per call."""
    model = Model(lib, sm.to_array())
    pool = model.pool(1)
    seq = pool.seq()
    prompt = c4_prompt(sm.config.vocab)
    done = 0
    while done < len(prompt):
        done += seq.prefill(prompt[done:], chunk_budget=chunk)
    out = {"kv_after_prefill": sha(pool.kv_block(0))}
    out["tokens"] = _decode_tokens(model, seq, budget, C4_TOKENS)
    out["kv_after_decode"] = sha(pool.kv_block(0))
    seq.release()
    pool.close()
    model.close()
    return out
