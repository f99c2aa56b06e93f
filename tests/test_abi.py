"""CPU checks of the C ABI: the HIP library loads without a GPU, exports every
function include/*.h declares, and the ctypes binding declares exactly those
functions.  No compute call is made (there is no GPU here)."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(tqf_hip_\w+)\s*\(", re.M)


def declared() -> set[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(DECL.findall(text))
    return names


@pytest.fixture(scope="module")
def lib_path():
    from turboqwenfare_amd import _lib

    if not _lib.LIB_PATH.exists():
        import __graft_entry__

        __graft_entry__.build()
    return _lib.LIB_PATH


def test_headers_declare_the_boundary():
    names = declared()
    for core in ("tqf_hip_create", "tqf_hip_weights_upload", "tqf_hip_q4_gemv",
                 "tqf_hip_moe_layer", "tqf_hip_accept", "tqf_hip_verify_step_device"):
        assert core in names
    assert len(names) >= 35


def test_library_exports_every_declared_symbol(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(declared() - exported)
    assert not missing, missing
    lib = ctypes.CDLL(str(lib_path))
    for name in declared():
        assert getattr(lib, name) is not None


def test_ctypes_binding_matches_the_headers():
    from turboqwenfare_amd import _lib

    assert set(_lib.SIGNATURES) == declared()


def test_bindings_fail_loudly_without_the_library(tmp_path):
    from turboqwenfare_amd import _lib

    with pytest.raises(RuntimeError):
        _lib.load(tmp_path / "missing.so")
