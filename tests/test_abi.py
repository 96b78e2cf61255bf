"""The C-ABI libraries load and export every symbol their headers declare
(no device calls: runs without a GPU)."""
import ctypes as C
import os
import re

import pytest

import orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(orc[a-z]*_[a-z0-9_]+)\s*\(", text))
    inline = set(re.findall(r"static inline \w+ (orc[a-z]*_[a-z0-9_]+)\s*\(", text))
    return sorted(names - inline)


def test_hip_lib_exports_header():
    lib = C.CDLL(orc.HIP_LIB)
    names = declared("orc.h")
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    names = set(declared("orc.h"))
    bound = {n for n, _, _ in orc.ABI}
    assert names == bound, (names - bound, bound - names)


def test_host_lib_exports_header():
    if not os.path.exists(os.path.join(ROOT, "include", "oracle_host.h")):
        pytest.skip("host API header not present")
    lib = C.CDLL(orc.HOST_LIB)
    missing = [n for n in declared("oracle_host.h") if not hasattr(lib, n)]
    assert not missing, missing


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(orc.OrcError):
        orc.load_hip_lib(str(tmp_path / "nope.so"))
