"""The step kernel divides several fp32 numbers by one divisor through a single fp64
reciprocal (`rcp64` / `div_r` in zeno_amd/csrc/dmath.h: y = 1/b from v_rcp_f64 and its cubic
correction, then each quotient is fp32(fp64(a * y))). Its results must be the bits of the fp32
division a / b that the reference and the oracle evaluate. This checks that property of the
arithmetic on the CPU (numpy's float32 division and float64 product are IEEE, round to nearest
even), with y off by up to 4 fp64 ulps of 1/b (the device's y is within 2^-53 relative, about
one ulp, over every fp32 divisor; the bound allows about 8), over random operands spanning the whole fp32 range including subnormals,
every significand of a against a set of divisors, and the special values (zeros, infinities,
NaN), where the kernel keeps the raw reciprocal. tests/test_gpu_divide.py runs the device
code itself over the same operands.
"""
import numpy as np


def shared_reciprocal_quotients(a: np.ndarray, b: np.ndarray, ulps: np.ndarray) -> np.ndarray:
    """The kernel's recipe with a reciprocal that is `ulps` fp64 ulps away from 1/b."""
    b64 = b.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        raw = 1.0 / b64
        y = (raw.view(np.int64) + ulps.astype(np.int64)).view(np.float64)
        y = np.where(np.isfinite(b) & (b != 0), y, raw)
        return (a.astype(np.float64) * y).astype(np.float32)


def assert_same_bits(got: np.ndarray, want: np.ndarray):
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan)
    bad = np.flatnonzero(got[~nan].view(np.uint32) != want[~nan].view(np.uint32))
    assert bad.size == 0, (got[~nan][bad[:5]], want[~nan][bad[:5]])


def fp32_quotients(a, b):
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        return (a / b).astype(np.float32)


def test_random_operands_whole_range():
    rng = np.random.default_rng(7)
    n = 4_000_000
    bits_a = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    bits_b = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    a, b = bits_a.view(np.float32), bits_b.view(np.float32)
    keep = np.isfinite(a) & np.isfinite(b)
    a, b = a[keep], b[keep]
    ulps = rng.integers(-4, 5, a.size)
    assert_same_bits(shared_reciprocal_quotients(a, b, ulps), fp32_quotients(a, b))


def test_quaternion_like_operands():
    """The kernel's cases: components of a quaternion or 3-vector over its length."""
    rng = np.random.default_rng(8)
    q = rng.standard_normal((2_000_000, 4)).astype(np.float32) * np.float32(1.0001)
    q[::7, 1] = 0.0
    q[::11, 2] = -0.0
    l = np.sqrt((q * q).sum(axis=1, dtype=np.float32)).astype(np.float32)
    a = q.reshape(-1)
    b = np.repeat(l, 4)
    ulps = rng.integers(-4, 5, a.size)
    assert_same_bits(shared_reciprocal_quotients(a, b, ulps), fp32_quotients(a, b))


def test_every_significand_against_fixed_divisors():
    sig = (np.arange(2**23, dtype=np.uint32) | np.uint32(0x3F800000)).view(np.float32)  # [1, 2)
    divisors = np.array([3.0, 7.0, 0.1, 1.1, np.pi, 1.0 - 2.0**-24, 1.5 + 2.0**-23, 1e-30, 3e37],
                        dtype=np.float32)
    rng = np.random.default_rng(9)
    for d in divisors:
        b = np.full(sig.size, d, np.float32)
        for k in (-4, 0, 4):
            ulps = np.full(sig.size, k)
            assert_same_bits(shared_reciprocal_quotients(sig, b, ulps), fp32_quotients(sig, b))
        ulps = rng.integers(-4, 5, sig.size)
        assert_same_bits(shared_reciprocal_quotients(sig, b, ulps), fp32_quotients(sig, b))


def test_special_values():
    f = np.float32
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 1e-45, -1e-45, 1e-40,
                     1.17549435e-38, 3.4028235e38, -3.4028235e38, 2.0**-126, 0.5, 3.0], dtype=f)
    a, b = np.meshgrid(vals, vals, indexing="ij")
    a, b = a.reshape(-1), b.reshape(-1)
    for k in (-4, 0, 4):
        assert_same_bits(shared_reciprocal_quotients(a, b, np.full(a.size, k)), fp32_quotients(a, b))
