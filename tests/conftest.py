import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HIP_SO = os.path.join(ROOT, "superslm_amd", "libsslm_hip.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP backend)")


@pytest.fixture(scope="session")
def ref_lib():
    from oracle_bind import REF_SO
    from superslm_amd.sslm import SslmLib
    if not os.path.exists(REF_SO):
        pytest.skip("compiled reference (oracle/_ref) not built")
    return SslmLib(REF_SO)


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle_bind import load_oracle
    return load_oracle()


@pytest.fixture(scope="session")
def hip_lib():
    from superslm_amd.sslm import SslmLib
    if not os.path.exists(HIP_SO):
        raise RuntimeError("libsslm_hip.so is not built: run __graft_entry__.build()")
    return SslmLib(HIP_SO)


_MODELS = {}


def synthetic(name, seed=7):
    from superslm_amd.sslm_artifact import CONFIGS, build_synthetic
    key = (name, seed)
    if key not in _MODELS:
        sm = build_synthetic(CONFIGS[name], seed=seed)
        _MODELS[key] = (sm, sm.to_bytes())
    return _MODELS[key]
