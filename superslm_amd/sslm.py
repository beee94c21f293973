"""ctypes binding of the sslm_* C ABI (reference include/superslm/sslm_abi.h and
include/superslm/sslm_abi_functions*.inc).

The same binding drives any library that exports the ABI: the HIP backend
(superslm_amd/libsslm_hip.so) and, in the tests, the compiled reference.  Statuses are the
reference's sslm_status values (sslm_abi.h:96-152); a non-OK status raises SslmError unless the
caller asks for the raw code.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

SSLM_OK = 0
STATUS_NAMES = [
    "SSLM_OK", "SSLM_INVALID_ARGUMENT", "SSLM_BUFFER_TOO_SMALL", "SSLM_MISALIGNED_BUFFER",
    "SSLM_ARTIFACT_REJECTED", "SSLM_ADAPTER_MODEL_MISMATCH", "SSLM_RESTORE_MODEL_MISMATCH",
    "SSLM_RESTORE_KV_MISMATCH", "SSLM_MODEL_HAS_LIVE_SEQUENCES", "SSLM_POOL_HAS_LIVE_HANDLES",
    "SSLM_ADAPTER_HAS_LIVE_SEQUENCES", "SSLM_ADAPTER_SWAP_MIDTOKEN_REJECTED",
    "SSLM_SEQ_RESET_MIDTOKEN_REJECTED", "SSLM_PREFIX_FROZEN_REJECTED", "SSLM_KV_POOL_EXHAUSTED",
    "SSLM_TOKEN_ID_OUT_OF_RANGE", "SSLM_CONTEXT_CAP_EXCEEDED", "SSLM_TOKEN_ID_UNMAPPED",
    "SSLM_SCHEMA_NOT_FOUND", "SSLM_SCHEMA_BIND_REJECTED", "SSLM_SCHEMA_SPAN_UNBOUND",
    "SSLM_PREFIX_SCHEMA_MISMATCH", "SSLM_RESTORE_SCHEMA_MISMATCH", "SSLM_SCHEMA_SPAN_UNREACHABLE",
    "SSLM_SCHEMA_UNSATISFIABLE", "SSLM_ALLOCATION_FAILED", "SSLM_NUMERIC_STEP_REFUSED",
]
ABI_ALIGNMENT = 64
SPAN_PROMPT = 0
SPAN_SCHEMA_CONTENT = 1


class SslmError(RuntimeError):
    def __init__(self, where: str, status: int):
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"{where}: {name}")
        self.status = status


class DecodeParams(ctypes.Structure):
    """sslm_decode_params (sslm_abi.h:207-224)."""
    _fields_ = [("layer_budget", ctypes.c_int32), ("struct_size", ctypes.c_uint32),
                ("mode", ctypes.c_int32), ("alpha_q15", ctypes.c_int32),
                ("anti_lm_max_order", ctypes.c_int32), ("top_k", ctypes.c_int32),
                ("q_ln2", ctypes.c_int64), ("q_b", ctypes.c_int64), ("q_c", ctypes.c_int64)]


class StatsOut(ctypes.Structure):
    """sslm_stats_out (sslm_abi.h:232-238)."""
    _fields_ = [("decode_step_ceiling", ctypes.c_int64), ("decode_step_actual", ctypes.c_int64),
                ("forced_token_count", ctypes.c_int64), ("kv_blocks_resident", ctypes.c_int32),
                ("schema_accepting", ctypes.c_int32)]


class Config(ctypes.Structure):
    """sslm_config (sslm_abi.h:40-46)."""
    _fields_ = [("max_batch", ctypes.c_int32), ("max_chunk_budget", ctypes.c_int32),
                ("max_layer_budget", ctypes.c_int32), ("reserved", ctypes.c_uint32)]


def _aligned_buffer(nbytes: int):
    raw = np.zeros(nbytes + ABI_ALIGNMENT, dtype=np.uint8)
    off = (-raw.ctypes.data) % ABI_ALIGNMENT
    return raw, raw.ctypes.data + off


class SslmLib:
    """One loaded sslm_* library."""

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path = path
        self.lib = ctypes.CDLL(path)
        L = self.lib
        vp, sz, i32, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint32
        pvp = ctypes.POINTER(ctypes.c_void_p)
        pi32 = ctypes.POINTER(ctypes.c_int32)

        def sig(name, res, *args):
            f = getattr(L, name)
            f.restype = res
            f.argtypes = list(args)

        sig("sslm_model_map", ctypes.c_int, vp, sz, pvp)
        sig("sslm_model_unmap", ctypes.c_int, vp)
        sig("sslm_kv_block_size", sz, vp)
        sig("sslm_kv_pool_overhead_size", sz, vp, u32)
        sig("sslm_kv_pool_create", ctypes.c_int, vp, vp, sz, u32, pvp)
        sig("sslm_kv_pool_destroy", ctypes.c_int, vp)
        sig("sslm_workspace_size", sz, vp, ctypes.POINTER(Config))
        sig("sslm_workspace_create", ctypes.c_int, vp, ctypes.POINTER(Config), vp, sz, pvp)
        sig("sslm_workspace_destroy", ctypes.c_int, vp)
        sig("sslm_seq_create", ctypes.c_int, vp, pvp, pvp)
        sig("sslm_seq_release", ctypes.c_int, vp)
        sig("sslm_seq_reset", ctypes.c_int, vp)
        sig("sslm_prefill", ctypes.c_int, vp, vp, pi32, i32, i32, ctypes.c_int, vp, pi32)
        sig("sslm_decode_step", ctypes.c_int, vp, pvp, i32, ctypes.POINTER(DecodeParams), vp, pi32)
        sig("sslm_decode_step_v2", ctypes.c_int, vp, pvp, i32, ctypes.POINTER(DecodeParams), vp, pi32)
        sig("sslm_decode_params_init", ctypes.c_int, vp, i32, i32, ctypes.POINTER(DecodeParams))
        sig("sslm_seq_set_adapter", ctypes.c_int, vp, vp)
        sig("sslm_adapter_map", ctypes.c_int, vp, sz, vp, pvp)
        sig("sslm_adapter_release", ctypes.c_int, vp)
        sig("sslm_seq_save", ctypes.c_int, vp, vp, ctypes.POINTER(sz))
        sig("sslm_seq_restore", ctypes.c_int, vp, pvp, vp, sz, pvp)
        sig("sslm_schema_lookup", ctypes.c_int, vp, ctypes.c_char_p, pvp)
        sig("sslm_schema_count", sz, vp)
        sig("sslm_schema_name", ctypes.c_int, vp, i32, vp, ctypes.POINTER(sz))
        sig("sslm_seq_set_schema", ctypes.c_int, vp, vp)
        sig("sslm_stats", ctypes.c_int, vp, vp, ctypes.POINTER(StatsOut))
        self.has_peek = hasattr(L, "sslm_g5_test_only_peek_kv_block_bytes")
        if self.has_peek:
            sig("sslm_g5_test_only_peek_kv_block_bytes", ctypes.c_int, vp, u32, vp, sz)

    def check(self, where: str, st: int):
        if st != SSLM_OK:
            raise SslmError(where, st)


class Model:
    """A mapped artifact.  Keeps the artifact bytes alive (the ABI requires it)."""

    def __init__(self, lib: SslmLib, artifact):
        """`artifact`: bytes, or a uint8 numpy array (mapped in place, no copy)."""
        self.lib = lib
        if isinstance(artifact, np.ndarray):
            self._bytes = np.ascontiguousarray(artifact, dtype=np.uint8)
            ptr, size = self._bytes.ctypes.data, self._bytes.nbytes
        else:
            self._bytes = ctypes.create_string_buffer(artifact, len(artifact))
            ptr, size = ctypes.addressof(self._bytes), len(artifact)
        h = ctypes.c_void_p()
        lib.check("sslm_model_map", lib.lib.sslm_model_map(ctypes.c_void_p(ptr), size, ctypes.byref(h)))
        self.handle = h
        self.block_size = lib.lib.sslm_kv_block_size(h)

    def pool(self, blocks: int) -> "KvPool":
        return KvPool(self, blocks)

    def decode_params(self, layer_budget: int, mode: int = 0, raw: bool = False):
        """sslm_decode_params_init (mode 0 greedy, 1 damped greedy); with `raw` the status too."""
        p = DecodeParams()
        st = self.lib.lib.sslm_decode_params_init(self.handle, mode, layer_budget, ctypes.byref(p))
        if raw:
            return st, p
        self.lib.check("sslm_decode_params_init", st)
        return p

    def decode_step(self, seqs, layer_budget: int, raw: bool = False, params: DecodeParams | None = None,
                    v2: bool = False):
        """One sslm_decode_step, or sslm_decode_step_v2 when `params` (or `v2`) is given."""
        n = len(seqs)
        arr = (ctypes.c_void_p * n)(*[s.handle.value for s in seqs])
        out = (ctypes.c_int32 * n)()
        p = params if params is not None else self.decode_params(layer_budget)
        # sslm_decode_step_v2 reads the whole struct (the v1 verb reads only layer_budget)
        verb = self.lib.lib.sslm_decode_step_v2 if v2 or params is not None else self.lib.lib.sslm_decode_step
        st = verb(self.handle, arr, n, ctypes.byref(p), None, out)
        if raw:
            return st, list(out)
        self.lib.check("sslm_decode_step", st)
        return list(out)

    def adapter(self, artifact) -> "Adapter":
        return Adapter(self, artifact)

    def schema_count(self) -> int:
        return self.lib.lib.sslm_schema_count(self.handle)

    def schema(self, name):
        """sslm_schema_lookup: (status, handle or None)."""
        h = ctypes.c_void_p()
        st = self.lib.lib.sslm_schema_lookup(self.handle, name if name is None else name.encode(), ctypes.byref(h))
        return st, (h if st == SSLM_OK else None)

    def schema_name(self, index: int, size: int | None = None):
        """sslm_schema_name with a buffer of `size` bytes (None: the sizing call): (status, name
        bytes or the required size)."""
        n = ctypes.c_size_t(size or 0)
        if size is None:
            st = self.lib.lib.sslm_schema_name(self.handle, index, None, ctypes.byref(n))
            return st, n.value
        buf = ctypes.create_string_buffer(size)
        st = self.lib.lib.sslm_schema_name(self.handle, index, buf, ctypes.byref(n))
        return st, buf.raw[:n.value] if st == SSLM_OK else n.value

    def stats(self, seq) -> tuple:
        out = StatsOut()
        st = self.lib.lib.sslm_stats(self.handle, seq.handle, ctypes.byref(out))
        return st, (out.decode_step_ceiling, out.decode_step_actual, out.forced_token_count,
                    out.kv_blocks_resident, out.schema_accepting)

    def close(self):
        if self.handle:
            self.lib.check("sslm_model_unmap", self.lib.lib.sslm_model_unmap(self.handle))
            self.handle = None


class Adapter:
    """A mapped LoRA adapter artifact (sslm_adapter_map).  Keeps its bytes alive."""

    def __init__(self, model: Model, artifact):
        self.model = model
        self._bytes = ctypes.create_string_buffer(bytes(artifact), len(artifact))
        h = ctypes.c_void_p()
        self.status = model.lib.lib.sslm_adapter_map(ctypes.addressof(self._bytes), len(artifact),
                                                     model.handle, ctypes.byref(h))
        model.lib.check("sslm_adapter_map", self.status)
        self.handle = h

    def release(self):
        if self.handle:
            self.model.lib.check("sslm_adapter_release", self.model.lib.lib.sslm_adapter_release(self.handle))
            self.handle = None


class KvPool:
    def __init__(self, model: Model, blocks: int):
        lib = model.lib
        self.model = model
        size = blocks * model.block_size + lib.lib.sslm_kv_pool_overhead_size(model.handle, blocks)
        self._raw, addr = _aligned_buffer(size)
        h = ctypes.c_void_p()
        lib.check("sslm_kv_pool_create",
                  lib.lib.sslm_kv_pool_create(model.handle, ctypes.c_void_p(addr), size, blocks, ctypes.byref(h)))
        self.handle = h

    def kv_block(self, index: int = 0) -> np.ndarray:
        """One KV block in the reference layout [layer][K|V][kv_head][context_cap][head_dim]
        (forward_sites.cpp:1227-1269); a sequence owns exactly one block."""
        m = self.model
        out = np.zeros(m.block_size, dtype=np.int8)
        m.lib.check("peek_kv", m.lib.lib.sslm_g5_test_only_peek_kv_block_bytes(
            self.handle, index, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def seq(self) -> "Seq":
        return Seq(self)

    def restore(self, blob: bytes, raw: bool = False):
        """sslm_seq_restore of a saved sequence blob into this pool: a Seq, or with `raw` the
        status and the Seq (None unless the status is SSLM_OK)."""
        m = self.model
        buf = ctypes.create_string_buffer(bytes(blob), len(blob))
        h = ctypes.c_void_p()
        st = m.lib.lib.sslm_seq_restore(m.handle, ctypes.byref(self.handle), buf, len(blob), ctypes.byref(h))
        seq = Seq(self, handle=h) if st == SSLM_OK else None
        if raw:
            return st, seq
        m.lib.check("sslm_seq_restore", st)
        return seq

    def close(self):
        if self.handle:
            self.model.lib.check("sslm_kv_pool_destroy", self.model.lib.lib.sslm_kv_pool_destroy(self.handle))
            self.handle = None


class Seq:
    def __init__(self, pool: KvPool, handle=None):
        lib = pool.model.lib
        self.pool = pool
        if handle is not None:  # a restored sequence
            self.handle = handle
            return
        h = ctypes.c_void_p()
        lib.check("sslm_seq_create", lib.lib.sslm_seq_create(pool.model.handle, ctypes.byref(pool.handle),
                                                              ctypes.byref(h)))
        self.handle = h

    def set_schema(self, schema) -> int:
        """sslm_seq_set_schema (None unbinds); returns the status."""
        return self.pool.model.lib.lib.sslm_seq_set_schema(self.handle, schema)

    def prefill(self, tokens, chunk_budget: int | None = None, raw: bool = False, kind: int = SPAN_PROMPT):
        m = self.pool.model
        arr = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        consumed = ctypes.c_int32(0)
        budget = chunk_budget if chunk_budget is not None else max(1, len(arr))
        st = m.lib.lib.sslm_prefill(m.handle, self.handle, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                    len(arr), budget, kind, None, ctypes.byref(consumed))
        if raw:
            return st, consumed.value
        m.lib.check("sslm_prefill", st)
        return consumed.value

    def set_adapter(self, adapter):
        m = self.pool.model
        m.lib.check("sslm_seq_set_adapter",
                    m.lib.lib.sslm_seq_set_adapter(self.handle, adapter.handle if adapter else None))

    def save_size(self):
        """The two-call sizing form: (status, required size) of sslm_seq_save with no buffer."""
        n = ctypes.c_size_t(0)
        st = self.pool.model.lib.lib.sslm_seq_save(self.handle, None, ctypes.byref(n))
        return st, n.value

    def save(self) -> bytes:
        lib = self.pool.model.lib
        n = ctypes.c_size_t(0)
        lib.lib.sslm_seq_save(self.handle, None, ctypes.byref(n))
        buf = ctypes.create_string_buffer(n.value)
        lib.check("sslm_seq_save", lib.lib.sslm_seq_save(self.handle, buf, ctypes.byref(n)))
        return buf.raw[:n.value]

    def release(self):
        if self.handle:
            self.pool.model.lib.check("sslm_seq_release", self.pool.model.lib.lib.sslm_seq_release(self.handle))
            self.handle = None
