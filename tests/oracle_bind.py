"""ctypes binding of the C oracle (oracle/libsslm_oracle.so) -- test infrastructure.

`OracleModel` builds the oracle's plain-struct model from a SyntheticModel's arrays and drives
the ABI-level sequence semantics of the reference's sslm_prefill / sslm_decode_step
(src/sslm_abi.cpp:1417-1567 and :1989-2434): prefill embeds every admitted token, runs the
chunked loop and hands the last hidden row to the next decode step, which then only computes
logits; a decode step otherwise embeds the current token at layer 0, runs up to `layer_budget`
layers, and produces a token once the last layer has committed.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(os.path.dirname(HERE), "oracle", "libsslm_oracle.so")
REF_SO = os.path.join(os.path.dirname(HERE), "oracle", "_ref", "libsuperslm_ref.so")

P = ctypes.c_void_p
i8p = ctypes.POINTER(ctypes.c_int8)
i32p = ctypes.POINTER(ctypes.c_int32)
i64p = ctypes.POINTER(ctypes.c_int64)

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class Scale(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int64), ("e", ctypes.c_int64)]


class LoraProj(ctypes.Structure):
    _fields_ = [("a", i8p), ("b", i8p), ("u_fold", i32p), ("d_fold", i32p)]


class Layer(ctypes.Structure):
    _fields_ = [("w", i8p * 7), ("fold", i32p * 7), ("ctx_fold", i32p), ("bias", i64p * 3),
                ("attn_gain", i32p), ("mlp_gain", i32p), ("kv_r_t_k", i64p), ("kv_e_t_k", i64p),
                ("kv_r_t_v", i64p), ("kv_e_t_v", i64p), ("khead_m", i64p), ("khead_e", i64p),
                ("attn_norm_sc", Scale), ("q_sc", Scale), ("ctx_sc", Scale), ("o_sc", Scale),
                ("attn_res_sc", Scale), ("mlp_norm_sc", Scale), ("gate_sc", Scale), ("up_sc", Scale),
                ("act_sc", Scale), ("down_sc", Scale), ("mlp_res_sc", Scale),
                ("lora_rank", ctypes.c_uint32), ("lora", ctypes.POINTER(LoraProj) * 7)]


class ModelS(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_uint32), ("layers", ctypes.c_uint32), ("heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32), ("inter", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("context_cap", ctypes.c_int64), ("layer", ctypes.POINTER(Layer)),
                ("embed", i8p), ("head", i8p), ("final_gain", i32p), ("embed_sc", Scale), ("final_sc", Scale),
                ("rope_cos", i64p), ("rope_sin", i64p), ("silu_table", i32p)]


class SeqS(ctypes.Structure):
    _fields_ = [("hidden", i8p), ("scale", Scale), ("layer_index", ctypes.c_uint32),
                ("kv_saturation_count", ctypes.c_uint64), ("context_length", ctypes.c_int64)]


def load_oracle():
    lib = ctypes.CDLL(ORACLE_SO)
    lib.or_run_layer_loop.argtypes = [ctypes.POINTER(ModelS), ctypes.POINTER(SeqS), ctypes.c_uint32, i8p]
    lib.or_run_chunk.argtypes = [ctypes.POINTER(ModelS), i8p, ctypes.POINTER(Scale), ctypes.c_size_t,
                                 ctypes.c_int64, i8p, ctypes.POINTER(ctypes.c_uint64)]
    lib.or_embed_entry.argtypes = [ctypes.POINTER(ModelS), ctypes.c_int32, i8p, ctypes.POINTER(Scale)]
    lib.or_final_logits.argtypes = [ctypes.POINTER(ModelS), i8p, i32p]
    lib.or_argmax.argtypes = [i32p, ctypes.c_size_t]
    lib.or_argmax.restype = ctypes.c_int32
    lib.or_project_row.argtypes = [i8p, Scale, ctypes.c_size_t, ctypes.c_size_t, i8p, i32p, i64p,
                                   ctypes.c_void_p, ctypes.c_uint32, Scale, i8p, ctypes.POINTER(Scale)]
    lib.or_kv_block_bytes.argtypes = [ctypes.POINTER(ModelS)]
    lib.or_kv_block_bytes.restype = ctypes.c_size_t
    return lib


def _p(arr, t):
    return arr.ctypes.data_as(t)


class OracleModel:
    """The oracle's view of a SyntheticModel (and optionally one adapter)."""

    def __init__(self, lib, sm, adapter=None):
        self.lib = lib
        self.sm = sm
        c = sm.config
        self.keep = []
        self.layers = (Layer * c.layers)()
        for l in range(c.layers):
            L = self.layers[l]
            p = f"layer{l}"
            for j, name in enumerate(PROJ):
                w = np.ascontiguousarray(sm.weights[f"{p}.{name}"])
                f = np.ascontiguousarray(sm.folds[f"{p}.{name}"], dtype=np.int32)
                self.keep += [w, f]
                L.w[j] = _p(w, i8p)
                L.fold[j] = _p(f, i32p)
            cf = np.ascontiguousarray(sm.folds[f"{p}.ctx_fold"], dtype=np.int32)
            self.keep.append(cf)
            L.ctx_fold = _p(cf, i32p)
            for j, name in enumerate(("q_proj", "k_proj", "v_proj")):
                b = sm.biases.get(f"{p}.{name}")
                if b is not None:
                    b = np.ascontiguousarray(b, dtype=np.int64)
                    self.keep.append(b)
                    L.bias[j] = _p(b, i64p)
            ag = sm.weights[f"{p}.attn_norm.gain"].astype(np.int32)
            mg = sm.weights[f"{p}.mlp_norm.gain"].astype(np.int32)
            self.keep += [ag, mg]
            L.attn_gain, L.mlp_gain = _p(ag, i32p), _p(mg, i32p)
            nkv = c.kv_heads
            rk = np.array([sm.landing[f"{p}.k_head{h}"][2] for h in range(nkv)], dtype=np.int64)
            ek = np.array([sm.landing[f"{p}.k_head{h}"][1] for h in range(nkv)], dtype=np.int64)
            rv = np.array([sm.landing[f"{p}.v_head{h}"][2] for h in range(nkv)], dtype=np.int64)
            ev = np.array([sm.landing[f"{p}.v_head{h}"][1] for h in range(nkv)], dtype=np.int64)
            km = np.array([sm.consts[f"{p}.softmax_khead{h}"][0] for h in range(nkv)], dtype=np.int64)
            ke = np.array([sm.consts[f"{p}.softmax_khead{h}"][1] for h in range(nkv)], dtype=np.int64)
            self.keep += [rk, ek, rv, ev, km, ke]
            L.kv_r_t_k, L.kv_e_t_k, L.kv_r_t_v, L.kv_e_t_v = (_p(a, i64p) for a in (rk, ek, rv, ev))
            L.khead_m, L.khead_e = _p(km, i64p), _p(ke, i64p)
            for fld, key in (("attn_norm_sc", "attn_norm"), ("q_sc", "q_proj"), ("ctx_sc", "attn_ctx"),
                             ("o_sc", "o_proj"), ("attn_res_sc", "attn_residual"), ("mlp_norm_sc", "mlp_norm"),
                             ("gate_sc", "gate_proj"), ("up_sc", "up_proj"), ("act_sc", "mlp_act"),
                             ("down_sc", "down_proj"), ("mlp_res_sc", "mlp_residual")):
                setattr(L, fld, Scale(*sm.consts[f"{p}.{key}"]))
            if adapter is not None:
                L.lora_rank = adapter.rank
                for j, name in enumerate(PROJ):
                    key = f"{p}.{name}"
                    if key in adapter.a:
                        a = np.ascontiguousarray(adapter.a[key])
                        b = np.ascontiguousarray(adapter.b[key])
                        uf = np.ascontiguousarray(adapter.u_fold[key], dtype=np.int32)
                        df = np.ascontiguousarray(adapter.d_fold[key], dtype=np.int32)
                        lp = LoraProj(_p(a, i8p), _p(b, i8p), _p(uf, i32p), _p(df, i32p))
                        self.keep += [a, b, uf, df, lp]
                        L.lora[j] = ctypes.pointer(lp)
        self.embed = np.ascontiguousarray(sm.weights["embed"])
        self.head = np.ascontiguousarray(sm.weights["embed"] if c.tie_embeddings else sm.weights["lm_head"])
        self.fgain = sm.weights["final_norm.gain"].astype(np.int32)
        self.cos = np.ascontiguousarray(sm.rope_cos, dtype=np.int64)
        self.sin = np.ascontiguousarray(sm.rope_sin, dtype=np.int64)
        self.silu = np.ascontiguousarray(sm.silu, dtype=np.int32)
        self.m = ModelS(c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.inter, c.vocab, c.context_cap,
                        ctypes.cast(self.layers, ctypes.POINTER(Layer)), _p(self.embed, i8p),
                        _p(self.head, i8p), _p(self.fgain, i32p), Scale(*sm.consts["embed"]),
                        Scale(*sm.consts["final_norm"]), _p(self.cos, i64p), _p(self.sin, i64p),
                        _p(self.silu, i32p))
        self.block_bytes = lib.or_kv_block_bytes(ctypes.byref(self.m))

    def new_seq(self) -> "OracleSeq":
        return OracleSeq(self)


class OracleSeq:
    """ABI-level state of one sequence (src/sslm_abi.cpp sslm_seq_s fields that matter)."""

    def __init__(self, om: OracleModel):
        self.om = om
        c = om.sm.config
        self.hidden = np.zeros(c.hidden, dtype=np.int8)
        self.kv = np.zeros(om.block_bytes, dtype=np.int8)
        self.state = SeqS(_p(self.hidden, i8p), Scale(0, 0), 0, 0, 0)
        self.current_token = -1
        self.ready_for_logits = False

    def prefill(self, tokens) -> tuple[int, int]:
        """Returns (oracle status, consumed).  Admission as src/sslm_abi.cpp:1451-1480: stop at
        the first out-of-range id or at the context cap."""
        om, c = self.om, self.om.sm.config
        tokens = [int(t) for t in tokens]
        admit = len(tokens)
        for i, t in enumerate(tokens):
            if t < 0 or t >= c.vocab:
                admit = i
                break
        head_room = c.context_cap - self.state.context_length
        admit = max(0, min(admit, head_room))
        if admit == 0:
            return 0, 0
        H = c.hidden
        chunk = np.zeros(admit * H, dtype=np.int8)
        scales = (Scale * admit)()
        for i in range(admit):
            st = om.lib.or_embed_entry(ctypes.byref(om.m), tokens[i], _p(chunk[i * H:], i8p), ctypes.byref(scales[i]))
            if st:
                return st, 0
        sat = ctypes.c_uint64(self.state.kv_saturation_count)
        st = om.lib.or_run_chunk(ctypes.byref(om.m), _p(chunk, i8p), scales, admit, self.state.context_length,
                                 _p(self.kv, i8p), ctypes.byref(sat))
        self.state.kv_saturation_count = sat.value
        if st:
            return st, 0
        self.hidden[:] = chunk[(admit - 1) * H:]
        self.state.scale = Scale(scales[admit - 1].m, scales[admit - 1].e)
        self.state.layer_index = 0
        self.state.context_length += admit
        self.current_token = tokens[admit - 1]
        self.ready_for_logits = True
        return 0, admit

    def decode_step(self, layer_budget: int) -> tuple[int, int]:
        """Returns (oracle status, token or -1 while mid-token)."""
        om, c = self.om, self.om.sm.config
        if self.ready_for_logits:
            self.ready_for_logits = False
        else:
            if self.state.layer_index == 0:
                sc = Scale()
                st = om.lib.or_embed_entry(ctypes.byref(om.m), self.current_token, _p(self.hidden, i8p),
                                           ctypes.byref(sc))
                if st:
                    return st, -1
                self.state.scale = sc
            st = om.lib.or_run_layer_loop(ctypes.byref(om.m), ctypes.byref(self.state), layer_budget,
                                          _p(self.kv, i8p))
            if st:
                return st, -1
            if self.state.layer_index < c.layers:
                return 0, -1
        logits = np.zeros(c.vocab, dtype=np.int32)
        st = om.lib.or_final_logits(ctypes.byref(om.m), _p(self.hidden, i8p), _p(logits, i32p))
        if st:
            return st, -1
        tok = int(om.lib.or_argmax(_p(logits, i32p), c.vocab))
        self.current_token = tok
        self.state.layer_index = 0
        return 0, tok


def project_rows(lib, a, w, fold, in_scale, site):
    """Oracle GEMM -> WSC1 fold -> funnel for every row of `a` (forward_sites.cpp:1114-1170).
    Returns (codes [m, n], scales [(m, e)] per row, statuses)."""
    m, k = a.shape
    n = w.shape[0]
    a = np.ascontiguousarray(a)
    w = np.ascontiguousarray(w)
    fold = np.ascontiguousarray(fold, dtype=np.int32)
    codes = np.zeros((m, n), dtype=np.int8)
    scales, sts = [], []
    for t in range(m):
        out_sc = Scale()
        st = lib.or_project_row(_p(a[t], i8p), Scale(*in_scale), k, n, _p(w, i8p), _p(fold, i32p), None, None, 0,
                                Scale(*site), _p(codes[t], i8p), ctypes.byref(out_sc))
        scales.append((out_sc.m, out_sc.e))
        sts.append(st)
    return codes, scales, sts
