"""The C-ABI library loads and exports every symbol include/vbhip.h declares.

CPU only: no function here touches the GPU (vb_version, vb_row_bytes and
vb_last_error are pure host code).
"""
import os
import re

import pytest

from vibeblade_amd import _lib, ggml

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))
           if f.endswith(".h")]


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(vb_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from vibeblade_amd import build
        build.build(verbose=False)
    return _lib.load()


def test_header_declares_functions():
    names = declared_functions()
    assert "vb_gemv" in names and "vb_dequant_rows" in names and "vb_last_error" in names


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in _lib.py"


def test_every_bound_symbol_is_declared():
    assert set(_lib.SIGNATURES) <= set(declared_functions())


def test_host_only_entry_points(lib):
    assert lib.vb_version() == 1
    assert lib.vb_row_bytes(ggml.GGML_TYPE_Q4_K, 4096) == 2304
    assert lib.vb_row_bytes(ggml.GGML_TYPE_Q4_K, 14336) == 8064
    assert lib.vb_row_bytes(ggml.GGML_TYPE_Q6_K, 4096) == 3360
    assert lib.vb_row_bytes(ggml.GGML_TYPE_Q8_0, 4096) == 4352
    assert lib.vb_row_bytes(ggml.GGML_TYPE_F16, 7) == 14
    assert lib.vb_row_bytes(ggml.GGML_TYPE_Q4_K, 100) == -1
    assert lib.vb_row_bytes(99, 256) == -1
    assert isinstance(lib.vb_last_error(), bytes)


def test_ggml_tables_match_library(lib):
    for t in ggml.DEVICE_TYPES:
        be, bb = ggml.BLOCK[t]
        assert lib.vb_row_bytes(t, be * 8) == ggml.row_bytes(t, be * 8) == bb * 8
    assert ggml.tensor_nbytes(ggml.GGML_TYPE_Q4_K, 300) == 288
    with pytest.raises(ValueError):
        ggml.row_bytes(ggml.GGML_TYPE_Q6_K, 100)
