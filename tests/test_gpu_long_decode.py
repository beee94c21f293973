"""Batched decode over long attention rows (1,000-1,500 positions, a 1,536-position cap): tokens,
every KV byte and the blobs must equal the compiled reference (src/sslm_abi.cpp:1989-2434) for
rows of different lengths in one batch, at layer budgets 1 and L, and for rows that grow past
1,024 positions while decoding."""
import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu


def _run(lib, art, prompts, calls, budget):
    model = Model(lib, art)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for s, p in zip(seqs, prompts):
        done = 0
        while done < len(p):
            done += s.prefill(p[done:], chunk_budget=512)
    toks = [model.decode_step(seqs, budget) for _ in range(calls)]
    kv = [pool.kv_block(i).copy() for i in range(len(prompts))]
    blobs = [s.save() for s in seqs]
    for s in seqs:
        s.release()
    pool.close()
    model.close()
    return toks, kv, blobs


@pytest.mark.parametrize("grouped", ["0", "1"])
@pytest.mark.parametrize("lengths,budget,calls", [((1100, 1500, 1023), 2, 6), ((1100, 1500, 1023), 1, 9),
                                                  ((1020, 1018), 2, 12)])
def test_long_rows_match_reference(lengths, budget, calls, grouped, hip_lib, ref_lib, monkeypatch):
    """grouped "1" forces decode attention to one block per (sequence, KV head), "0" to one block
    per query head."""
    monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", grouped)
    sm, art = synthetic("long")
    rng = np.random.default_rng(sum(lengths) + budget)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in lengths]
    print(f"case long decode lengths={lengths} budget={budget} grouped={grouped}", flush=True)
    r = _run(ref_lib, art, prompts, calls, budget)
    h = _run(hip_lib, art, prompts, calls, budget)
    assert h[0] == r[0], f"tokens differ: hip {h[0]} ref {r[0]}"
    for i in range(len(prompts)):
        assert np.array_equal(h[1][i], r[1][i]), f"KV of sequence {i} differs"
        assert h[2][i] == r[2][i], f"blob of sequence {i} differs"
