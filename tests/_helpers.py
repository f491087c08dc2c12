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
