"""BASELINE configurations 1-4 at their real shapes: the HIP backend against the compiled
reference's recorded results (tests/golden/workload_fixtures.json, made by
tests/golden/make_workload_fixtures.py from oracle/_ref on the same seeded artifacts and prompts).

Bit-exact bar: every output token, and SHA-256 of every KV block and sequence blob.  Configuration
2 runs its 512-token prompt as one chunk, as 200 + 312 and as 17-token chunks, decoding 128 tokens
at layer budgets 28, 4 and 1 respectively; configuration 4's full workload (32 sequences x
2048-token prompts) is beyond the CPU reference, so it is checked on the GPU through properties
the reference guarantees: a 2048-token chunk equals four 512-token chunks, a batched decode
equals a solo decode, and budget 1 equals budget 28."""
import json
import os

import numpy as np
import pytest

import baseline_workloads as W
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "workload_fixtures.json")


@pytest.fixture(scope="module")
def fx():
    return json.load(open(FIXTURES))


@pytest.fixture(scope="module")
def sm15(fx):
    sm = W.model_15b()
    assert W.artifact_hash(sm) == fx["artifact_15b"], "the synthetic 1.5B artifact is not the fixtures' one"
    return sm


def _need(fx, key):
    if key not in fx:
        pytest.fail(f"{key} missing from workload_fixtures.json: run tests/golden/make_workload_fixtures.py")
    return fx[key]


@pytest.mark.timeout(600)
def test_config1_batch_and_solo(fx, sm15, hip_lib):
    want = _need(fx, "c1")
    print("case config1 batch of 16", flush=True)
    got = W.run_c1(hip_lib, sm15, batched=True)
    assert got["tokens"] == want["tokens"]
    assert got["kv"] == want["kv"]
    print("case config1 solo", flush=True)
    solo = W.run_c1_solo(hip_lib, sm15)
    assert solo == _need(fx, "c1_solo")
    assert solo["tokens"] == [t[0] for t in want["tokens"]]  # M = 1 equals row 0 of the batch


@pytest.mark.timeout(600)
@pytest.mark.parametrize("chunks,budget", [([512], 28), ([200, 312], 4), ([17], 1)])
def test_config2_chunks_and_budgets(chunks, budget, fx, sm15, hip_lib):
    want = _need(fx, "c2")
    print(f"case config2 chunks={chunks} budget={budget}", flush=True)
    got = W.run_c2(hip_lib, sm15, chunks, budget)
    assert got["kv_after_prefill"] == want["kv_after_prefill"], "KV after prefill differs"
    assert got["blob_after_prefill"] == want["blob_after_prefill"]
    assert got["tokens"] == want["tokens"]
    assert got["kv_after_decode"] == want["kv_after_decode"], "KV after decode differs"
    assert got["blob_after_decode"] == want["blob_after_decode"]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("budget", [28, 4])
def test_config3_lora_swap(budget, fx, sm15, hip_lib):
    want = _need(fx, "c3")
    print(f"case config3 budget={budget}", flush=True)
    got = W.run_c3(hip_lib, sm15, budget)
    for k in ("adapter_a", "adapter_b", "base"):
        assert got[k]["tokens"] == want[k]["tokens"], k
        assert got[k]["kv"] == want[k]["kv"], k


@pytest.fixture(scope="module")
def sm7(fx):
    _need(fx, "c4")
    sm = W.model_7b()
    assert W.artifact_hash(sm) == fx["artifact_7b"], "the synthetic 7B artifact is not the fixtures' one"
    yield sm
    sm.image = None


@pytest.mark.timeout(900)
@pytest.mark.parametrize("budget,chunk,grouped", [(28, 128, ""), (1, 50, ""), (28, 128, "1"), (28, 128, "1h")])
def test_config4_shape_against_reference(budget, chunk, grouped, fx, sm7, hip_lib, monkeypatch):
    """grouped "1": decode attention as one block per (sequence, KV head) with its 7 query heads
    as the MFMA rows; "1h": two blocks per (sequence, KV head), 4 and 3 of its heads (the form
    batches of long rows take by themselves)."""
    want = fx["c4"]
    if grouped:
        monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", "1")
        monkeypatch.setenv("SSLM_HIP_GROUP_HALVES", "2" if grouped == "1h" else "1")
    print(f"case config4 7B budget={budget} chunk={chunk} grouped={grouped}", flush=True)
    got = W.run_c4(hip_lib, sm7, budget, chunk)
    assert got == want


@pytest.mark.timeout(900)
def test_config4_full_size_properties(sm7, hip_lib):
    """32 sequences with 2048-token prompts (one chunk each) decoded together at budget 28 for 256
    greedy steps (contexts grow to 2304 positions, as configuration 4 states), and a 33rd sequence
    with sequence 0's prompt in four 512-token chunks decoded alone at budget 1: its KV after
    prefill, its 256 tokens and its final KV equal sequence 0's.  The batch's decode attention runs
    one block per (sequence, KV head), the solo sequence's one block per query head."""
    B, ctx, steps = 32, 2048, 256
    L = sm7.config.layers
    model = Model(hip_lib, sm7.to_array())
    pool = model.pool(B + 1)
    rng = np.random.default_rng(4096)
    prompts = [rng.integers(0, sm7.config.vocab, size=ctx) for _ in range(B)]
    seqs = [pool.seq() for _ in range(B)]
    print("case config4 full size: prefill", flush=True)
    for s, p in zip(seqs, prompts):
        assert s.prefill(p, chunk_budget=ctx) == ctx
    solo = pool.seq()
    done = 0
    while done < ctx:
        done += solo.prefill(prompts[0][done:], chunk_budget=512)
    kv0 = W.sha(pool.kv_block(0))
    assert W.sha(pool.kv_block(B)) == kv0, "2048-token chunk and 4 x 512 chunks leave different KV"
    print("case config4 full size: decode", flush=True)
    batch_toks = [model.decode_step(seqs, L) for _ in range(steps)]
    solo_toks = []
    while len(solo_toks) < steps:
        t = model.decode_step([solo], 1)[0]
        if t >= 0:
            solo_toks.append(t)
    assert solo_toks == [t[0] for t in batch_toks], (solo_toks, batch_toks)
    assert W.sha(pool.kv_block(B)) == W.sha(pool.kv_block(0)), "batched budget-28 and solo budget-1 KV differ"
    for s in seqs + [solo]:
        s.release()
    pool.close()
    model.close()
