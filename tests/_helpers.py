"""Numeric comparison helpers shared by the test modules."""
import numpy as np


def ulp_dist(x, y) -> np.ndarray:
    """ULP distance between float32 arrays.  The bit patterns are mapped to a
    monotone integer line on which -0.0 and +0.0 are adjacent keys (1 apart):
    a non-negative pattern i keeps its value, a negative one maps to
    -(i & 0x7fffffff) - 1.  NaN compares by bits."""
    def key(a):
        i = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF) - 1, i)
    return np.abs(key(x) - key(y))


def zero_sign_mismatches(got, want) -> int:
    """Number of places where `want` is a zero and `got` is not the same zero
    (a sign error at zero is one ulp apart, which a <= n ulp bar lets pass)."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    z = want == 0
    return int(np.count_nonzero(z & ((got != 0) | (np.signbit(got) != np.signbit(want)))))


def assert_within_ulp(got, want, max_ulp: int, what=None) -> None:
    """`got` within `max_ulp` of `want` everywhere, and exactly the same
    signed zero wherever `want` is zero."""
    d = ulp_dist(got, want)
    assert d.max(initial=0) <= max_ulp, (what, int(d.max()))
    assert zero_sign_mismatches(got, want) == 0, (what, "sign of a zero result")


def rel_err(got, want) -> float:
    """Lamp3's normalised error max|got - want| / max|want|
    (tests/stress/testutils.py:47-50, with |.| in the denominator)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / (np.max(np.abs(want)) + 1e-30))


# Signed zeros, infinities, NaN, subnormals (down to the smallest, 1e-45),
# the smallest normal, the extremes and the neighbours of 1.
SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 3.0, np.inf, -np.inf, np.nan,
                     1e-45, -1e-45, 1.5e-39, 1.1754944e-38, 1e-20, 3.4e38, -3.4e38,
                     1.0000001, 0.99999994], np.float32)


def special_rows(length, rng):
    """Rows of special values for max/min/sum/prod: all -inf, NaN among
    values, all NaN, +inf among values, all +0, all -0, +0 and -0 both at the
    maximum (and the minimum) among negatives (positives), random values."""
    rows = np.empty((9, length), np.float32)
    rows[0] = -np.inf
    rows[1] = rng.standard_normal(length)
    rows[1, ::5] = np.nan
    rows[2] = np.nan
    rows[3] = rng.standard_normal(length)
    rows[3, length // 2] = np.inf
    rows[4] = 0.0
    rows[5] = -0.0
    rows[6] = -1.0 - np.abs(rng.standard_normal(length))
    rows[6, 1::7] = 0.0
    rows[6, 0::11] = -0.0
    rows[7] = 1.0 + np.abs(rng.standard_normal(length))
    rows[7, 1::7] = 0.0
    rows[7, 0::11] = -0.0
    rows[8] = rng.standard_normal(length)
    return rows


def assert_sum_close(got, want, a, axis):
    """A float32 sum against the oracle's sequential sum `want` at 1e-5
    under max|diff|/max|want|.  A cancelling sum (one far smaller than the sum
    of its terms' magnitudes) has no order-independent result at that bar:
    there each output of both orders must lie within 1e-6 of the sum of
    |terms| of the float64 sum, a band that a dropped or doubled term of
    typical size still leaves.  Examples: 1995 terms up to 3.8 summing to
    -0.129 put the sequential order 2.4e-4 (relative) from float64 and the
    tree order 2.0e-5; 2506 terms up to 3.4 summing to -0.454 put them 4.1e-6
    and 1.6e-5 from it."""
    if rel_err(got, want) <= 1e-5:
        return
    a64 = a.astype(np.float64)
    truth = a64.sum(axis=axis, keepdims=True)
    band = 1e-6 * np.abs(a64).sum(axis=axis, keepdims=True)
    assert np.all(np.abs(got - truth) <= band), rel_err(got, want)
    assert np.all(np.abs(want - truth) <= band), rel_err(got, want)
