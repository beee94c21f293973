"""Long prefill spans and forward refusals: the HIP backend against the compiled reference.

The reference's prefill (src/sslm_abi.cpp:1417-1545) embeds every admitted token, runs one batched
layer loop over all of them and commits nothing when a step refuses; admission stops at the first
out-of-range id or at the context cap; decode (src/sslm_abi.cpp:1989-2434) leaves a refused
sequence at its last committed layer.  Each case compares the status, `consumed`, the output
tokens and the SSB3 blob (context length, layer index, current token, hidden scale, saturation
count and the whole KV block) with the reference, then keeps decoding from the state the refusal
left and compares again.  The argmax cases pin the lowest-index tie break (forward_sites.cpp:
2427-2441) with exactly tied LM-head rows, within one 16-column tile and across tiles."""
import struct

import numpy as np
import pytest

from conftest import synthetic
from superslm_amd.sslm import Model

pytestmark = pytest.mark.gpu

CURRENT_TOKEN_OFFSET = 72  # SSB3 header field (src/sslm_abi.cpp:2585-2618)


def _script(lib, art, steps):
    """Runs `steps` against one fresh sequence and returns what each step observed.
    Steps: ("prefill", tokens, chunk_budget) -> (status, consumed);
           ("decode", budget) -> (status, out token);
           ("save",) -> blob; ("kv",) -> KV block;
           ("restore_patched", offset, fmt, value) -> status (re-create the sequence from its own
           blob with one header field changed)."""
    model = Model(lib, art)
    pool = model.pool(1)
    seq = pool.seq()
    out = []
    for st in steps:
        kind = st[0]
        if kind == "prefill":
            out.append(seq.prefill(st[1], chunk_budget=st[2], raw=True))
        elif kind == "decode":
            s, toks = model.decode_step([seq], st[1], raw=True)
            out.append((s, toks[0]))
        elif kind == "save":
            out.append(seq.save())
        elif kind == "kv":
            out.append(pool.kv_block(0).copy())
        elif kind == "restore_patched":
            blob = bytearray(seq.save())
            struct.pack_into(st[2], blob, st[1], st[3])
            seq.release()
            s, seq = pool.restore(bytes(blob), raw=True)
            out.append(s)
            assert seq is not None
        else:
            raise ValueError(kind)
    seq.release()
    pool.close()
    model.close()
    return out


def _compare(h, r, steps):
    for i, (a, b, st) in enumerate(zip(h, r, steps)):
        if isinstance(b, (bytes, np.ndarray)):
            a8 = np.frombuffer(a, np.uint8) if isinstance(a, bytes) else a.view(np.uint8)
            b8 = np.frombuffer(b, np.uint8) if isinstance(b, bytes) else b.view(np.uint8)
            assert a8.size == b8.size, f"step {i} {st[0]}: sizes {a8.size} vs {b8.size}"
            diff = np.nonzero(a8 != b8)[0]
            assert diff.size == 0, f"step {i} {st[0]}: {diff.size} bytes differ, first at {diff[:6]}"
        else:
            assert a == b, f"step {i} {st[:2] if st[0] != 'prefill' else st[0]}: hip {a} ref {b}"


def _decode_until(n_tokens, budget, L):
    """decode steps that yield n_tokens whole tokens at `budget` layers per call (one logits call
    after a prefill, then ceil(L / budget) calls per token)."""
    per = -(-L // budget)
    return [("decode", budget)] * (1 + n_tokens * per)


def _run_both(hip_lib, ref_lib, art, steps, label):
    print(f"case {label}", flush=True)
    r = _script(ref_lib, art, steps)
    h = _script(hip_lib, art, steps)
    _compare(h, r, steps)
    return h, r


@pytest.mark.parametrize("chunk", [1100, 600, 512])
def test_long_prefill_span_matches_reference(chunk, hip_lib, ref_lib):
    """A 1100-token prompt in spans of `chunk` tokens: one launch sequence of 1100 tokens, or
    spans of 600 + 500 / 512 + 512 + 76; every KV byte, the blob and the next tokens."""
    sm, art = synthetic("long")
    prompt = np.random.default_rng(101).integers(0, sm.config.vocab, size=1100)
    L = sm.config.layers
    steps = []
    for b in range(0, len(prompt), chunk):
        steps.append(("prefill", prompt[b:], chunk))
    steps += [("kv",), ("save",)] + _decode_until(3, L, L) + [("save",)]
    h, r = _run_both(hip_lib, ref_lib, art, steps, f"long prefill chunk={chunk}")
    assert all(x == (0, min(chunk, 1100 - i * chunk)) for i, x in enumerate(h[:len(steps) - 1]) if steps[i][0] == "prefill")


def _zero_embed_model(token):
    sm, _ = synthetic("long")
    from superslm_amd.sslm_artifact import with_weight_rows
    return sm, with_weight_rows(sm, "embed", {token: np.zeros(sm.config.hidden, np.int8)})


def test_refusal_in_second_span_commits_nothing(hip_lib, ref_lib):
    """A token whose embedding row is all zeros is refused by the forward (the reference's
    RMSNorm site rejects the zero row).  Placed at index 700 of an 1100-token prefill -- past the
    first 512 tokens -- the whole call must commit nothing: status, consumed 0, the blob (context
    length 0, the untouched KV block) as the reference's; the same sequence then prefills a clean
    prompt and decodes as the reference does."""
    bad = 5
    sm, art = _zero_embed_model(bad)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, sm.config.vocab, size=1100)
    prompt[prompt == bad] = bad + 1
    clean = prompt.copy()
    prompt[700] = bad
    L = sm.config.layers
    steps = [("prefill", clean[:40], 64), ("save",), ("prefill", prompt, 1100), ("save",), ("kv",),
             ("prefill", prompt, 512), ("save",),
             ("prefill", clean[40:900], 900), ("save",)] + _decode_until(2, L, L) + [("save",)]
    h, r = _run_both(hip_lib, ref_lib, art, steps, "zero-embed refusal at index 700")
    assert h[2][0] != 0 and h[2][1] == 0, h[2]  # refused, nothing consumed
    assert h[1] == h[3], "a refused prefill changed the sequence"


def test_multi_span_prefill_matches_reference(monkeypatch, hip_lib, ref_lib):
    """The multi-span commit path (spans of at most 256 tokens forced by SSLM_HIP_PREFILL_SPAN, so
    an 1100-token prefill runs as five launch sequences): a clean 1100-token prompt prefills and
    decodes as the reference's single batched call does, and the zero-embedding refusal at index
    700 -- in the third span, after two spans have landed K/V rows and clamp counts -- commits
    nothing: status, consumed, the blob and the whole KV block equal the reference's."""
    monkeypatch.setenv("SSLM_HIP_PREFILL_SPAN", "256")
    bad = 5
    sm, art = _zero_embed_model(bad)
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, sm.config.vocab, size=1100)
    prompt[prompt == bad] = bad + 1
    clean = prompt.copy()
    prompt[700] = bad
    L = sm.config.layers
    print("case multi-span prefill: clean", flush=True)
    steps = [("prefill", clean, 1100), ("save",), ("kv",)] + _decode_until(2, L, L) + [("save",)]
    _run_both(hip_lib, ref_lib, art, steps, "multi-span clean prefill")
    print("case multi-span prefill: refusal in the third span", flush=True)
    steps = [("prefill", clean[:40], 64), ("save",), ("prefill", prompt, 1100), ("save",), ("kv",),
             ("prefill", clean[40:300], 300), ("save",), ("kv",)] + _decode_until(2, L, L) + [("save",)]
    h, _ = _run_both(hip_lib, ref_lib, art, steps, "multi-span refusal at index 700")
    assert h[2][0] != 0 and h[2][1] == 0, h[2]  # refused, nothing consumed
    assert h[1] == h[3], "a refused multi-span prefill changed the sequence"


def test_admission_stops_match_reference(hip_lib, ref_lib):
    """Admission pre-scan (src/sslm_abi.cpp:1451-1510): an out-of-range id at index 700 admits
    the 700 tokens before it; a prompt crossing the context cap admits the headroom."""
    sm, art = synthetic("long")
    V, cap = sm.config.vocab, sm.config.context_cap
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, V, size=1000)
    prompt[700] = V + 3
    L = sm.config.layers
    tail = rng.integers(0, V, size=cap)
    steps = [("prefill", prompt, 1000), ("save",)] + _decode_until(1, L, L) + [
        ("prefill", tail[:cap - 700 - 2 + 40], 2000), ("save",), ("kv",),
        ("prefill", tail[:5], 5)]
    h, _ = _run_both(hip_lib, ref_lib, art, steps, "admission: id out of range, cap crossed")
    assert h[0] == (15, 700), h[0]  # SSLM_TOKEN_ID_OUT_OF_RANGE, 700 admitted


def _bias_edit(layer, scale):
    def edit(m):
        m.biases[f"layer{layer}.q_proj"] = (m.biases[f"layer{layer}.q_proj"] * scale).astype(np.int64)
    return edit


@pytest.mark.parametrize("grouped", ["0", "1"])
def test_numeric_refusal_at_later_layer(grouped, hip_lib, ref_lib, monkeypatch):
    """A q bias pushed far out of range at layer 1 makes the q|k|v funnel refuse there (layer 0
    runs normally): prefill refuses and commits nothing; a sliced decode (budget 1) commits layer
    0 and refuses at layer 1, leaving the sequence at layer 1, as the reference does.  Decode
    attention (where the q funnel runs) as one block per query head ("0") and one per KV head
    ("1")."""
    monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", grouped)
    from superslm_amd.sslm_artifact import CONFIGS, build_synthetic
    sm = build_synthetic(CONFIGS["small"], seed=7, edit=_bias_edit(1, 1 << 34))
    art = sm.to_bytes()
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, sm.config.vocab, size=30)
    L = sm.config.layers
    steps = [("prefill", prompt, 30), ("save",), ("kv",)]
    h, _ = _run_both(hip_lib, ref_lib, art, steps, "numeric refusal at layer 1 (prefill)")
    assert h[0][0] != 0, h[0]
    # decode: a fresh sequence restored with a pending token (SSB3 current_token) runs layer 0
    # at budget 1, then refuses at layer 1 and stays there
    steps = [("restore_patched", CURRENT_TOKEN_OFFSET, "<i", 3), ("decode", 1), ("save",), ("decode", 1),
             ("save",), ("kv",), ("decode", 1), ("save",), ("decode", L), ("save",)]
    h, _ = _run_both(hip_lib, ref_lib, art, steps, "numeric refusal at layer 1 (decode, budget 1)")
    assert h[1] == (0, -1) and h[3][0] != 0, (h[1], h[3])


def test_decode_refusal_from_restored_token(hip_lib, ref_lib):
    """A sequence restored with the zero-embedding token as its pending token (SSB3 current_token)
    refuses that token's forward at layer 0, at budget 1 and at budget L."""
    bad = 5
    sm, art = _zero_embed_model(bad)
    rng = np.random.default_rng(10)
    prompt = rng.integers(0, sm.config.vocab, size=12)
    prompt[prompt == bad] = bad + 1
    L = sm.config.layers
    for budget in (1, L):
        steps = [("prefill", prompt, 12), ("decode", L), ("save",),
                 ("restore_patched", CURRENT_TOKEN_OFFSET, "<i", bad), ("save",),
                 ("decode", budget), ("save",), ("decode", budget), ("save",)]
        h, _ = _run_both(hip_lib, ref_lib, art, steps, f"decode refusal from restored token budget={budget}")
        assert h[5][0] != 0, h[5]


@pytest.mark.parametrize("period", [2, 40])
def test_argmax_tie_break_lowest_index(period, hip_lib, ref_lib):
    """LM-head rows repeated with period `period` (row j = row j % period): every logit ties with
    its copies, within one 16-column tile (period 2) and across tiles (period 40); the argmax must
    be the lowest index, the reference's tie break."""
    from superslm_amd.sslm_artifact import with_weight_rows
    sm, _ = synthetic("tiny")
    head = np.array(sm.weights["lm_head"])
    art = with_weight_rows(sm, "lm_head", {j: head[j % period] for j in range(period, sm.config.vocab)})
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, sm.config.vocab, size=9)
    L = sm.config.layers
    steps = [("prefill", prompt, 9)] + _decode_until(6, L, L) + [("kv",)]
    h, _ = _run_both(hip_lib, ref_lib, art, steps, f"argmax ties period={period}")
    toks = [x[1] for x in h[1:-1]]
    assert all(t < period for t in toks), toks


def _batch_script(lib, art, prompts, bad_index, bad_token, budget, calls):
    """Three sequences prefilled, one decode call; then sequence `bad_index` is re-created from its
    blob with `bad_token` pending, and `calls` batched decode calls follow.  Returns each call's
    (status, out tokens) -- the out array is pre-filled with 777 so untouched entries show -- and
    every sequence's blob after each call."""
    import ctypes
    model = Model(lib, art)
    pool = model.pool(len(prompts))
    seqs = [pool.seq() for _ in prompts]
    for s, p in zip(seqs, prompts):
        s.prefill(p)
    model.decode_step(seqs, _LAYERS[0])
    blob = bytearray(seqs[bad_index].save())
    struct.pack_into("<i", blob, CURRENT_TOKEN_OFFSET, bad_token)
    seqs[bad_index].release()
    seqs[bad_index] = pool.restore(bytes(blob))
    rec = []
    for _ in range(calls):
        n = len(seqs)
        arr = (ctypes.c_void_p * n)(*[s.handle.value for s in seqs])
        out = (ctypes.c_int32 * n)(*([777] * n))
        p = model.decode_params(budget)
        st = lib.lib.sslm_decode_step(model.handle, arr, n, ctypes.byref(p), None, out)
        rec.append((st, list(out), [s.save() for s in seqs]))
    for s in seqs:
        s.release()
    pool.close()
    model.close()
    return rec


_LAYERS = [None]  # layer count of the model under test


@pytest.mark.parametrize("grouped", ["0", "1"])
@pytest.mark.parametrize("budget", [1, 2])
def test_batched_decode_stops_at_first_refusal(budget, grouped, hip_lib, ref_lib, monkeypatch):
    """A batch of three whose middle sequence refuses its pending token at layer 0: the first
    sequence advances, the refusing one and the one after it are left as they were (outputs
    untouched, blobs unchanged), status as the reference's -- every call, at budget 1 and 2, with
    decode attention as one block per query head ("0") and one per KV head ("1")."""
    monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", grouped)
    bad = 5
    sm, art = _zero_embed_model(bad)
    _LAYERS[0] = sm.config.layers
    rng = np.random.default_rng(13)
    prompts = [rng.integers(0, sm.config.vocab, size=n) for n in (6, 9, 4)]
    for p in prompts:
        p[p == bad] = bad + 1
    print(f"case batched refusal budget={budget}", flush=True)
    r = _batch_script(ref_lib, art, prompts, 1, bad, budget, 3)
    h = _batch_script(hip_lib, art, prompts, 1, bad, budget, 3)
    for c, (hh, rr) in enumerate(zip(h, r)):
        assert hh[0] == rr[0] != 0, (c, hh[0], rr[0])
        assert hh[1] == rr[1], (c, hh[1], rr[1])
        for i in range(3):
            assert hh[2][i] == rr[2][i], f"call {c}: blob of sequence {i} differs"


ATTN_MODES = {"head": "0", "group": "1"}


@pytest.mark.parametrize("shift", [40, -40])
@pytest.mark.parametrize("mode", list(ATTN_MODES))
def test_attention_refusal_in_decode(mode, shift, hip_lib, ref_lib, monkeypatch):
    """Layer 1's second K head scale shifted by 2^shift: the i-exp constants of that KV group's
    heads refuse (the loader accepts the artifact).  A sequence restored with a pending token
    commits layer 0 at budget 1, then refuses at layer 1's attention, call after call, with the
    reference's status, K/V rows and saturation count (every KV group lands before attention);
    decode attention as one block per query head and one per (sequence, KV group)."""
    monkeypatch.setenv("SSLM_HIP_GROUPED_ATTN", ATTN_MODES[mode])
    from superslm_amd.sslm_artifact import CONFIGS, build_synthetic

    def edit(m):
        km, ke = m.consts["layer1.softmax_khead1"]
        m.consts["layer1.softmax_khead1"] = (km, ke + shift)
    sm = build_synthetic(CONFIGS["tiny"], seed=7, edit=edit)
    L = sm.config.layers
    # (a fresh sequence's blob with a pending token: a prefill refused at the attention stage
    # leaves staged K/V past the committed context that differs by design)
    steps = [("restore_patched", CURRENT_TOKEN_OFFSET, "<i", 3),
             ("decode", 1), ("save",), ("decode", 1), ("save",), ("decode", 1), ("save",), ("decode", L), ("save",)]
    h, _ = _run_both(hip_lib, ref_lib, sm.to_bytes(), steps, f"attention refusal {mode} shift={shift}")
    assert h[1] == (0, -1) and h[3][0] != 0, (h[1], h[3])
