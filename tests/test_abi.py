"""CPU checks of the C ABI: the library loads and exports every symbol the
header declares, and the header declares every symbol the binding expects."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "talechime_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(tc_[a-z_0-9]+)\s*\(", src))


def test_header_matches_binding():
    from talechime_amd import _lib
    assert _declared() == set(_lib.EXPORTS)


def test_library_exports_every_symbol():
    from talechime_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libtalechime_hip.so not built")
    import torch  # noqa: F401  (same HIP runtime the product binds to)
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    lib.tc_abi_version.restype = ctypes.c_int
    assert lib.tc_abi_version() == 1


def test_struct_layout_matches_header():
    from talechime_amd import _lib
    # offsets of tc_sample_params as laid out by the C compiler for this header
    assert ctypes.sizeof(_lib.SampleParams) == 72
    assert _lib.SampleParams.d_add_mask.offset == 56
    assert ctypes.sizeof(_lib.VerifyOut) == 56
