"""The C-ABI library loads without a GPU and exports every symbol include/sslm_hip.h declares."""
import ctypes
import os
import re

from conftest import HIP_SO, ROOT


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "sslm_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:sslm|sslm_hip)_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for s in ("sslm_model_map", "sslm_prefill", "sslm_decode_step", "sslm_kv_pool_create", "sslm_seq_create",
              "sslm_adapter_map", "sslm_seq_set_adapter", "sslm_hip_gemm_requant"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(HIP_SO)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_resolves(hip_lib):
    assert hip_lib.lib is not None
