"""The lane-exchange schedule of the wave reductions (csrc/hip/wave_swap.inc).

The eager reduction kernels and the fused row kernels reduce a wave's 64 lanes
with DPP quad permutes (partner lane i^1, i^2), the DPP half-row and row
mirrors (partner 7-i within 8 lanes, 15-i within 16), a ds_swizzle xor 16
within 32 lanes and two readlanes (lanes 0 and 32).  Only the first two and
the swizzle are xor partners; the mirrors and readlanes give the xor
partner's value only when the lanes before them agree.  These checks emulate
the lane moves on the CPU and show that (1) with a symmetric combine every
lane ends with exactly the value of an xor butterfly taken in the order 1, 2,
4, 8, 16, 32, and (2) with a combine that is not symmetric lane 0 still
combines all 64 lanes.  The GPU tests compare the kernels themselves.
"""
import numpy as np

LANES = 64


def dpp_quad_perm(v, sel):
    return [v[(i & ~3) | sel[i & 3]] for i in range(LANES)]


def dpp_row_half_mirror(v):
    return [v[(i & ~7) | (7 - (i & 7))] for i in range(LANES)]


def dpp_row_mirror(v):
    return [v[(i & ~15) | (15 - (i & 15))] for i in range(LANES)]


def swizzle_xor16(v):
    # bitmask mode within groups of 32 lanes: and 0x1f, or 0, xor 0x10
    return [v[(i & ~31) | ((i & 31) ^ 16)] for i in range(LANES)]


def readlane_32(v):
    lo, hi = v[0], v[32]
    return [lo if i & 32 else hi for i in range(LANES)]


SCHEDULE = [lambda v: dpp_quad_perm(v, [1, 0, 3, 2]),
            lambda v: dpp_quad_perm(v, [2, 3, 0, 1]),
            dpp_row_half_mirror, dpp_row_mirror, swizzle_xor16, readlane_32]


def wave_reduce(v, combine):
    for move in SCHEDULE:
        o = move(v)
        v = [combine(a, b) for a, b in zip(v, o)]
    return v


def xor_butterfly(v, combine):
    for off in (1, 2, 4, 8, 16, 32):
        v = [combine(v[i], v[i ^ off]) for i in range(LANES)]
    return v


def test_symmetric_combine_equals_the_xor_butterfly_bit_for_bit():
    rng = np.random.default_rng(7)
    for _ in range(20):
        x = list(rng.standard_normal(LANES).astype(np.float32) * np.float32(1e3))
        add = lambda a, b: np.float32(a + b)
        got = wave_reduce(x, add)
        want = xor_butterfly(x, add)
        assert [g.tobytes() for g in got] == [w.tobytes() for w in want]
        # every lane holds the same value
        assert len({g.tobytes() for g in got}) == 1


def test_lane_zero_covers_every_lane_for_any_combine():
    # A combine that is not symmetric (keeps its left operand's identity on
    # ties, like max over +0 / -0) still has to see all 64 inputs in lane 0.
    lanes = [frozenset([i]) for i in range(LANES)]
    got = wave_reduce(lanes, lambda a, b: a | b)
    assert got[0] == frozenset(range(LANES))
    signed_zero_max = lambda a, b: b if a < b else a
    zeros = [np.float32(-0.0) if i % 3 else np.float32(0.0) for i in range(LANES)]
    assert wave_reduce(zeros, signed_zero_max)[0] == 0.0


def test_a_wrong_partner_is_caught():
    # Planted mistake: a plain row mirror in place of the half-row mirror
    # leaves lanes 4..7 of each row out of lane 0's result.
    bad = list(SCHEDULE)
    bad[2] = dpp_row_mirror
    v = [frozenset([i]) for i in range(LANES)]
    for move in bad:
        o = move(v)
        v = [a | b for a, b in zip(v, o)]
    assert v[0] != frozenset(range(LANES))
