"""The step kernel divides several fp32 numbers by one divisor through one fp64 reciprocal
(v_rcp_f64 and a cubic correction, then fp32(a * y) with the subnormal tie rule; `rcp64` / `qdivs`
in dmath.h), which must give the bits of the IEEE fp32 division the reference and the oracle
evaluate. The same device code, through zeno_amd_selfcheck_divide, against numpy's fp32
division: every significand of the numerator against a set of divisors (normal, subnormal,
huge, negative), random bit patterns over the whole fp32 range, exact midpoints of the
subnormal grid and their neighbours, and the special values."""
import ctypes as C

import numpy as np
import pytest

from tests.test_shared_reciprocal import subnormal_midpoints
from zeno_amd import _lib

pytestmark = pytest.mark.gpu


def device_quotients(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    lib = _lib.load()
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    q = np.empty_like(a)
    rc = lib.zeno_amd_selfcheck_divide(a.ctypes.data_as(C.c_void_p), b.ctypes.data_as(C.c_void_p),
                                       q.ctypes.data_as(C.c_void_p), C.c_uint32(a.size))
    assert rc == 0, _lib.last_error()
    return q


def ieee_quotients(a, b):
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        return (np.asarray(a, np.float32) / np.asarray(b, np.float32)).astype(np.float32)


def assert_same_bits(got, want, what):
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan, err_msg=what)
    bad = np.flatnonzero(got[~nan].view(np.uint32) != want[~nan].view(np.uint32))
    assert bad.size == 0, (what, bad.size, got[~nan][bad[:4]], want[~nan][bad[:4]])


@pytest.mark.parametrize("d", [3.0, 7.0, 0.1, 1.1, np.pi, 1.0 - 2.0**-24, 1.5 + 2.0**-23, 1e-30, 3e37,
                               1e-40, -2.5, 1.0000001])
def test_every_significand(d):
    sig = (np.arange(2**23, dtype=np.uint32) | np.uint32(0x3F800000)).view(np.float32)  # [1, 2)
    b = np.full(sig.size, d, np.float32)
    assert_same_bits(device_quotients(sig, b), ieee_quotients(sig, b), f"divisor {d}")


def test_random_bit_patterns():
    rng = np.random.default_rng(11)
    a = rng.integers(0, 2**32, 1 << 24, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = rng.integers(0, 2**32, 1 << 24, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert_same_bits(device_quotients(a, b), ieee_quotients(a, b), "random")


def test_unit_quaternion_components():
    rng = np.random.default_rng(12)
    q = rng.standard_normal((1 << 22, 4)).astype(np.float32)
    q[::5, 0] = 0.0
    q[::9, 3] = -0.0
    l = np.sqrt((q * q).sum(axis=1, dtype=np.float32)).astype(np.float32)
    a, b = q.reshape(-1), np.repeat(l, 4)
    assert_same_bits(device_quotients(a, b), ieee_quotients(a, b), "quaternions")


def test_special_values():
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 1e-45, -1e-45, 1e-40, 1.17549435e-38,
                     3.4028235e38, -3.4028235e38, 0.5, 3.0], dtype=np.float32)
    a, b = np.meshgrid(vals, vals, indexing="ij")
    assert_same_bits(device_quotients(a.reshape(-1), b.reshape(-1)), ieee_quotients(a.reshape(-1), b.reshape(-1)),
                     "special")


def test_reciprocal_error_over_every_divisor():
    """The proof of correct rounding needs |1 - b y| below about 2^-49.1 for every divisor; the
    device reports the maximum over all 2^32 fp32 bit patterns (finite, nonzero)."""
    lib = _lib.load()
    err = C.c_double(-1.0)
    assert lib.zeno_amd_selfcheck_reciprocal_error(C.byref(err)) == 0, _lib.last_error()
    assert 0.0 < err.value <= 2.0**-52, err.value


def test_subnormal_midpoints():
    """Quotients exactly halfway between two fp32 subnormals round to the even one; their
    neighbours (numerator one step up or down) are no ties."""
    a, b = subnormal_midpoints(400_000, 31)
    assert_same_bits(device_quotients(a, b), ieee_quotients(a, b), "subnormal midpoints")
    for step in (-1, 1):
        a2 = (a.view(np.int32) + step).view(np.float32)
        assert_same_bits(device_quotients(a2, b), ieee_quotients(a2, b), f"midpoint neighbours {step}")
