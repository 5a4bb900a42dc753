"""The step kernel divides several fp32 numbers by one divisor through a single fp64
reciprocal (`rcp64` / `qdivs` in zeno_amd/csrc/dmath.h: y = 1/b from v_rcp_f64 and its cubic
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


def shared_reciprocal_quotients(a: np.ndarray, b: np.ndarray, ulps: np.ndarray, snap: bool = True) -> np.ndarray:
    """The kernel's recipe with a reciprocal that is `ulps` fp64 ulps away from 1/b: q = a * y
    in fp64; |q| rounded to a multiple of 2^-176 by adding and subtracting 1.5 * 2^-124, the
    sign copied back; then rounded to fp32."""
    b64 = b.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        raw = 1.0 / b64
        y = (raw.view(np.int64) + ulps.astype(np.int64)).view(np.float64)
        y = np.where(np.isfinite(b) & (b != 0), y, raw)
        q = a.astype(np.float64) * y
        if snap:
            C = 1.5 * 2.0**-124
            q = np.copysign((np.abs(q) + C) - C, q)
        return q.astype(np.float32)


def subnormal_midpoints(n: int, seed: int):
    """(a, b) whose exact quotient a / b is a midpoint of two adjacent fp32 subnormals (or of 0
    and the smallest one): a = M B 2^(k-150), b = B 2^k with M, B odd, both exact in fp32."""
    rng = np.random.default_rng(seed)
    M = rng.integers(0, 2**11, n) * 2 + 1
    B = rng.integers(0, 2**11, n) * 2 + 1
    k = rng.integers(-20, 100, n)
    a = (M * B).astype(np.float64) * 2.0 ** (k - 150)
    b = B.astype(np.float64) * 2.0 ** k
    sign = np.where(rng.random(n) < 0.5, -1.0, 1.0)
    a32, b32 = (sign * a).astype(np.float32), b.astype(np.float32)
    exact = (np.abs(a32.astype(np.float64)) == a) & (b32.astype(np.float64) == b)
    return a32[exact], b32[exact]


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


def test_subnormal_midpoint_quotients():
    """Exact ties exist only for subnormal quotients (a normal quotient's midpoint needs a
    25-bit odd significand times B, more bits than a holds). Without the even-divisor rule the
    fp64 product lands on either side of the midpoint and rounds the wrong way for many. The
    device's reciprocal is within one fp64 ulp of 1/b (|1 - b y| <= 2^-53 over every divisor),
    so q is within 2^-178 of a tie and the snap to the 2^-176 grid lands on it."""
    a, b = subnormal_midpoints(400_000, 21)
    assert a.size > 100_000
    want = fp32_quotients(a, b)
    for k in (-1, 0, 1):
        ulps = np.full(a.size, k)
        assert_same_bits(shared_reciprocal_quotients(a, b, ulps), want)
    plain = shared_reciprocal_quotients(a, b, np.full(a.size, 1), snap=False)
    assert np.count_nonzero(plain.view(np.uint32) != want.view(np.uint32)) > 1000


def test_every_tie_has_an_even_integer_divisor():
    """Brute force over small cases: for every odd numerator significand M 2^-149 (M < 2^13)
    and every divisor B 2^e (B odd < 2^9, e in -12..12), the quotient is an exact fp32 rounding
    tie (an odd multiple of 2^-150: u = a / b 2^150 = 2M / (B 2^e) an odd integer, checked in
    integer arithmetic) only when the divisor is an even integer. Ties are rare operand pairs,
    not an artefact of the model."""
    M = np.arange(1, 1 << 13, 2, dtype=np.int64)[:, None]
    B = np.arange(1, 1 << 9, 2, dtype=np.int64)[None, :]
    ties = 0
    for e in range(-12, 13):
        if e <= 1:
            num, den = M << (1 - e), B          # u = num / den
        else:
            num, den = M, B << (e - 1)
        tie = (num % den == 0) & ((num // den) % 2 == 1)
        even_integer_divisor = e >= 1           # B 2^e with B odd is an even integer iff e >= 1
        assert not tie.any() or even_integer_divisor, e
        ties += int(tie.sum())
    assert ties > 1000


def test_snap_leaves_near_midpoints_alone():
    """Quotients one fp32 step of a away from an exact midpoint are no ties: at least 2^-174
    from any midpoint, so neither the reciprocal's error nor the snap moves them across."""
    a, b = subnormal_midpoints(200_000, 22)
    for step in (-1, 1):
        a2 = (a.view(np.int32) + step).view(np.float32)
        ok = np.isfinite(a2) & (np.sign(a2) == np.sign(a))
        want = fp32_quotients(a2[ok], b[ok])
        for k in (-4, 0, 4):
            assert_same_bits(shared_reciprocal_quotients(a2[ok], b[ok], np.full(ok.sum(), k)), want)
