"""Numeric comparison helpers shared by the test modules."""
import numpy as np


def ulp_dist(x, y) -> np.ndarray:
    """ULP distance between float32 arrays (monotone integer mapping of the
    bit patterns, so -0.0 and +0.0 are 1 apart and NaN compares by bits)."""
    def key(a):
        i = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, np.int64(-2**31) - i, i)
    return np.abs(key(x) - key(y))


def rel_err(got, want) -> float:
    """Lamp3's normalised error max|got - want| / max|want|
    (tests/stress/testutils.py:47-50, with |.| in the denominator)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / (np.max(np.abs(want)) + 1e-30))
