"""superslm_amd/build.sh fails loudly: a source that does not compile makes the script (and so
__graft_entry__.build()) exit non-zero and leaves no library behind, even when an earlier build
left objects and a library in place.  Runs on stub sources in a temporary copy (no GPU)."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

STUB_OK = 'extern "C" int stub_%s(void) { return 0; }\n'


def _tree(tmp_path, broken):
    pkg = tmp_path / "pkg"
    (pkg / "csrc").mkdir(parents=True)
    shutil.copy(os.path.join(ROOT, "superslm_amd", "build.sh"), pkg / "build.sh")
    for name in ("kernels.hip", "runtime.cpp", "artifact.cpp", "noalloc.hip"):
        tag = name.split(".")[0]
        text = STUB_OK % tag
        if name == broken:
            text += "this is not C++ ;\n"
        (pkg / "csrc" / name).write_text(text)
    return pkg


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
def test_clean_stub_tree_builds(tmp_path):
    pkg = _tree(tmp_path, broken=None)
    r = subprocess.run(["bash", str(pkg / "build.sh")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert (pkg / "libsslm_hip.so").exists()


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("broken", ["kernels.hip", "runtime.cpp"])
def test_compile_error_fails_the_build(tmp_path, broken):
    pkg = _tree(tmp_path, broken=None)
    assert subprocess.run(["bash", str(pkg / "build.sh")], capture_output=True).returncode == 0
    # now break one source: the stale objects and library from the good build must not survive
    (pkg / "csrc" / broken).write_text("this is not C++ ;\n")
    r = subprocess.run(["bash", str(pkg / "build.sh")], capture_output=True, text=True)
    assert r.returncode != 0
    assert "failed" in r.stderr
    assert not (pkg / "libsslm_hip.so").exists()
