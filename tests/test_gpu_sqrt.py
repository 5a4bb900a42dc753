"""The joint and contact solves take the square roots they compare against a threshold (C > 1e-6,
sin > 1e-6, tangent speed > 1e-6, quaternion length > 1e-8) with `sqrt_gate` (dmath.h):
v_sqrt_f32 and the one-ulp correction of a correctly rounded fp32 root, without the scaling of
inputs below 2^-96. The same device code, through zeno_amd_selfcheck_sqrt, against numpy's IEEE
fp32 square root: every significand of twelve binades (even and odd exponents, both ends of the
range, the 2^-96 boundary), random bit patterns over the whole range, and the special values;
below 2^-96 the result must stay under 2^-47, below every threshold it is compared with."""
import ctypes as C

import numpy as np
import pytest

from zeno_amd import _lib

pytestmark = pytest.mark.gpu

GATE = np.float32(2.0**-96)


def device_roots(x: np.ndarray) -> np.ndarray:
    lib = _lib.load()
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    rc = lib.zeno_amd_selfcheck_sqrt(x.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p), C.c_uint32(x.size))
    assert rc == 0, _lib.last_error()
    return y


def ieee_roots(x):
    with np.errstate(invalid="ignore"):
        return np.sqrt(np.asarray(x, np.float32)).astype(np.float32)


def assert_same_bits(got, want, what):
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan, err_msg=what)
    bad = np.flatnonzero(got[~nan].view(np.uint32) != want[~nan].view(np.uint32))
    assert bad.size == 0, (what, bad.size, got[~nan][bad[:4]], want[~nan][bad[:4]])


@pytest.mark.parametrize("e", [-96, -95, -60, -21, -2, -1, 0, 1, 40, 41, 126, 127])
def test_every_significand_of_a_binade(e):
    bits = np.arange(2**23, dtype=np.uint32) | np.uint32((e + 127) << 23)
    x = bits.view(np.float32)
    assert_same_bits(device_roots(x), ieee_roots(x), f"binade 2^{e}")


def test_random_bit_patterns():
    rng = np.random.default_rng(21)
    x = rng.integers(0, 2**32, 1 << 24, dtype=np.uint64).astype(np.uint32).view(np.float32)
    keep = ~((np.abs(x) < GATE) & (x != 0))  # tiny magnitudes are checked below
    x = x[keep]
    assert_same_bits(device_roots(x), ieee_roots(x), "random")


def test_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -1.0, -1e-30, -3.4028235e38, 3.4028235e38, 1.0, 4.0,
                  2.0**-96, 1e-12, 1e-16], dtype=np.float32)
    assert_same_bits(device_roots(x), ieee_roots(x), "special")
    y = device_roots(x)
    assert np.signbit(y[1]) and y[1] == 0  # sqrt(-0) = -0


def test_below_the_gate_stays_below_every_threshold():
    rng = np.random.default_rng(22)
    bits = rng.integers(1, int(GATE.view(np.uint32)), 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), np.array([1e-45, 1e-40, 1.17549435e-38, 2.0**-97], np.float32)])
    y = device_roots(x)
    assert np.all(np.isfinite(y)) and np.all(y >= 0)
    assert np.all(y < np.float32(2.0**-47)), y.max()
