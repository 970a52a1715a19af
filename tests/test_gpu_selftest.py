"""On-device checks of the approximations whose error bounds the exact
sequential sum relies on and which use GPU-only instructions (the host-side
table generator checks the others exhaustively)."""
import ctypes
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "talechime_amd", "libtc_selftest.so")


def test_exp_approx_within_three_ulps_on_every_input():
    """exp_approx (v_exp_f32 on the exactly split argument, first-order
    corrected) against the correctly rounded exp on every float in [-87, 0]:
    at most 3 ulps, so within 4 ulps of glibc's expf, i.e. within the
    kSeqErr = 2^-21 relative bound the exact sequential sum assumes."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    assert os.path.exists(LIB), "libtc_selftest.so missing: run python -m talechime_amd.build"
    lib = ctypes.CDLL(LIB)
    out = ctypes.c_uint(0xFFFFFFFF)
    rc = lib.tc_selftest_exp_approx(ctypes.byref(out))
    assert rc == 0
    print("exp_approx max distance from the correctly rounded exp:", out.value, "ulp")
    assert out.value <= 3
