"""Kernel-level parity: liblmp_hip.so through its C ABI vs the CPU oracle.

Bars (from the task statement): add/sub/mul/div/neg/relu/comparisons and the
two backward functors bit-exact; transcendentals within 2 ulp of the oracle;
reductions within 1e-5 under Lamp3's normalised metric max|d| / max|true|
(tests/stress/testutils.py:47-50); matmul within 1e-4 under the same metric.
"""
import ctypes as C
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from _helpers import (SPECIALS, assert_sum_close, assert_within_ulp, rel_err,  # noqa: E402
                      special_rows)


def up(hip, arr):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(arr))


BCAST_SHAPES = [((7, 9), (7, 9)), ((64, 33), (64, 1)), ((64, 33), (33,)),
                ((64, 32), (1, 32)), ((64, 32), (64, 1)), ((5, 6, 7), (6, 1)),
                ((4, 1, 3), (1, 5, 3)), ((13,), (1,)), ((1,), (1,)),
                ((2, 3, 4, 5), (3, 1, 5)), ((1000, 1024), (1000, 1)),
                ((1000, 1024), (1024,)), ((4099,), (4099,)), ((3, 1), (1, 8))]

EXACT_BIN = ["add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt",
             "abs_backward"]


@pytest.mark.parametrize("sa,sb", BCAST_SHAPES, ids=str)
@pytest.mark.parametrize("op", EXACT_BIN)
def test_binary_bitexact(hip, oracle, op, sa, sb):
    rng = np.random.default_rng(zlib.crc32(repr((op, sa, sb)).encode()))
    a = rng.standard_normal(sa, dtype=np.float32)
    b = rng.standard_normal(sb, dtype=np.float32)
    if op in ("eq", "ne", "ge", "le"):
        a = np.round(a).astype(np.float32)
        b = np.round(b).astype(np.float32)
    if op == "abs_backward":
        a[..., :1] = 0.0
    want = oracle.binary(op, a, b)
    for x, y, w in ((a, b, want), (b, a, oracle.binary(op, b, a))):
        got = hip.binary(op, up(hip, x), up(hip, y)).numpy()
        assert got.shape == w.shape
        assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), op


def test_binary_special_values_bitexact(hip, oracle):
    """Every pair of special values (signed zeros, infinities, NaN, subnormals
    down to 1e-45, the extremes, neighbours of 1) through the exact binary ops
    against the oracle bit for bit: subnormal inputs and results are kept (no
    flush to zero), x/0 and inf - inf as IEEE has them.  A NaN result compares
    as NaN only: x86 and the GPU give a new NaN (0/0, inf - inf) different
    sign bits."""
    col, row = SPECIALS.reshape(-1, 1), SPECIALS.reshape(1, -1)
    for op in ("add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt", "abs_backward"):
        want = oracle.binary(op, col, row)
        got = hip.binary(op, up(hip, col), up(hip, row)).numpy()
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), op
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), op


def test_clamp_backward_strict(hip, oracle):
    x = np.array([-2, -1, 0, 1, 2, 0.5, np.nan], np.float32)
    g = np.arange(7, dtype=np.float32) + 1
    got = hip.binary("clamp_backward", up(hip, x), up(hip, g), -1.0, 1.0).numpy()
    assert np.array_equal(got, oracle.binary("clamp_backward", x, g, -1.0, 1.0))


def test_pow_within_2ulp(hip, oracle):
    rng = np.random.default_rng(5)
    a = rng.uniform(0.01, 10, (256, 64)).astype(np.float32)
    b = rng.uniform(-4, 4, (256, 64)).astype(np.float32)
    got = hip.binary("pow", up(hip, a), up(hip, b)).numpy()
    assert_within_ulp(got, oracle.binary("pow", a, b), 2)


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4096, 100003])
@pytest.mark.parametrize("op", ["neg", "abs", "sqrt", "clamp"])
def test_unary_bitexact(hip, oracle, op, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * 10
    x[: min(n, 3)] = np.array([-0.0, 0.0, np.nan], np.float32)[: min(n, 3)]
    if op == "sqrt":
        x = np.abs(x)
    p0, p1 = (0.0, oracle.DBL_MAX) if op == "clamp" else (0.0, 0.0)
    got = hip.unary(op, up(hip, x), p0, p1).numpy()
    want = oracle.unary(op, x, p0, p1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_relu_special_values(hip, oracle):
    x = np.array([-1, -0.0, 0.0, np.inf, -np.inf, np.nan, 3e38, -1e-42], np.float32)
    got = hip.unary("clamp", up(hip, x), 0.0, oracle.DBL_MAX).numpy()
    assert np.array_equal(got.view(np.uint32),
                          oracle.unary("clamp", x, 0.0, oracle.DBL_MAX).view(np.uint32))
    assert np.signbit(got[1]) and np.isnan(got[5])


@pytest.mark.parametrize("op", ["exp", "log", "sin", "cos", "tan"])
def test_transcendentals_within_2ulp(hip, oracle, op):
    rng = np.random.default_rng(17)
    x = rng.uniform(-30, 30, 1 << 16).astype(np.float32)
    if op == "log":
        x = np.abs(x) + np.float32(1e-6)
    got = hip.unary(op, up(hip, x)).numpy()
    assert_within_ulp(got, oracle.unary(op, x), 2, op)


def _correctly_rounded(op, x, y=None):
    """float64 evaluation rounded once to float32: the correctly rounded value
    except where the float64 result lies within one float64 ulp of a float32
    rounding boundary (a 2^-29-relative band, covered by the 2-ulp bar)."""
    d = x.astype(np.float64)
    with np.errstate(all="ignore"):
        if op == "pow":
            return np.power(d, y.astype(np.float64)).astype(np.float32)
        return getattr(np, op)(d).astype(np.float32)


def _transcendental_inputs(op, rng):
    n = 1 << 16
    if op == "exp":
        x = rng.uniform(-103.0, 88.7, n)  # through the subnormal results to the overflow edge
        special = [0.0, -0.0, 1.0, -1.0, 88.72, 88.73, -87.3, -103.9, np.inf, -np.inf, np.nan]
    elif op == "log":
        x = 10.0 ** rng.uniform(-44.0, 38.5, n)  # subnormal inputs to near FLT_MAX
        special = [1.0, 2.0, 0.5, 0.0, -1.0, np.inf, np.nan, 1e-45, 3.4e38]
    else:
        x = np.concatenate([rng.uniform(-100.0, 100.0, n - 64),
                            rng.uniform(-1e4, 1e4, 64)])
        special = [0.0, -0.0, np.pi / 2, np.pi, 1e-30, np.inf, np.nan]
    return np.concatenate([x, special]).astype(np.float32)


@pytest.mark.parametrize("op", ["exp", "log", "sin", "cos", "tan"])
def test_transcendentals_vs_correctly_rounded(hip, op):
    """The GPU's exp/log/sin/cos/tan (ocml, reached from the functors of
    cpu/kernels.hpp:74-113) within 2 ulp of the correctly rounded float32
    result, independently of the glibc oracle; NaN where it is NaN."""
    x = _transcendental_inputs(op, np.random.default_rng(29))
    got = hip.unary(op, up(hip, x)).numpy()
    want = _correctly_rounded(op, x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), op
    assert_within_ulp(got[~nan], want[~nan], 2, op)


@pytest.mark.parametrize("op", ["sin", "tan", "sqrt", "exp", "cos", "log", "neg", "abs"])
def test_signed_zero_arguments_bitexact(hip, oracle, op):
    """Zero arguments of both signs give the oracle's value bit for bit (so
    sin/tan/sqrt of -0.0 stay -0.0, as std::sin/tan/sqrt do for the functors of
    cpu/kernels.hpp:74-113), and so does the same op inside a fused kernel."""
    import rushlite_amd as rsl
    x = np.array([-0.0, 0.0, -0.0, 0.0], np.float32)
    want = oracle.unary(op, x)
    got = hip.unary(op, up(hip, x)).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (op, got)
    v = rsl.Variable(x)
    with rsl.capture_on():
        fused = getattr(rsl, op)(v) * rsl.Variable(np.ones(4, np.float32))
    got_f = fused.numpy()
    want_f = oracle.binary("mul", want, np.ones(4, np.float32))
    assert np.array_equal(got_f.view(np.uint32), want_f.view(np.uint32)), (op, got_f)


def test_pow_vs_correctly_rounded(hip):
    rng = np.random.default_rng(31)
    a = np.concatenate([rng.uniform(0.01, 10, 1 << 15), 10.0 ** rng.uniform(-10, 10, 1 << 15)])
    b = np.concatenate([rng.uniform(-4, 4, 1 << 15), rng.uniform(-3, 3, 1 << 15)])
    a, b = a.astype(np.float32), b.astype(np.float32)
    got = hip.binary("pow", up(hip, a), up(hip, b)).numpy()
    want = _correctly_rounded("pow", a, b)
    assert_within_ulp(got, want, 2)


def test_pow_special_values(hip, oracle):
    """pow over every pair of special values plus negative bases with integer
    and fractional exponents: NaN where the oracle's powf has NaN, infinities
    and zeros with its signs (C99 Annex F: pow(-0, -1) = -inf, pow(-1, inf) = 1,
    pow(x, 0) = 1 for NaN x, ...), everything else within 2 ulp."""
    extra = np.array([-2.0, -0.5, 2.0, 0.25, -3.0, 7.0, 1e-3, 1e30, -1e30], np.float32)
    vals = np.concatenate([SPECIALS, extra])
    col, row = vals.reshape(-1, 1), vals.reshape(1, -1)
    got = hip.binary("pow", up(hip, col), up(hip, row)).numpy()
    want = oracle.binary("pow", col, row)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    exact = ~nan & (np.isinf(want) | (want == 0.0) | (want == 1.0))
    assert np.array_equal(got[exact].view(np.uint32), want[exact].view(np.uint32))
    assert_within_ulp(got[~nan], want[~nan], 2)


@pytest.mark.parametrize("shape", [(70000, 5, 4), (65536, 9, 3), (66000, 2, 7),
                                   (70000, 1, 2)], ids=str)
def test_reduce_outer_beyond_grid_z(hip, oracle, shape):
    """More outer slices than a grid's z extent (65535), which the reference
    grid-strides over (reduct.cu:166-182, 253-257): one lane per output folds
    the axis in row order, so every op equals the oracle's sequential fold
    (cpu/reduct.cpp:15-19) bit for bit."""
    rng = np.random.default_rng(zlib.crc32(repr(shape).encode()))
    a = rng.standard_normal(shape, dtype=np.float32)
    for op in ("sum", "max", "min", "prod"):
        src = (1.0 + 0.01 * a).astype(np.float32) if op == "prod" else a
        got = hip.reduce(op, up(hip, src), 1).numpy()
        want = oracle.reduce(op, src, 1)
        assert got.shape == want.shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), op


def test_binary_extent_beyond_32_bits(hip):
    """A broadcast add [2^32 + 3, 1] + [1, 2] (8.6e9 outputs, 51 GB): after
    coalescing, the outer extent is above 2^32, so the generic kernel peels
    that dim with 64-bit division.  Values planted in a around index 2^32
    must land in the right output rows."""
    L = hip.lib()
    n = (1 << 32) + 3
    a = hip.DeviceBuffer((n, 1), np.float32)
    b = up(hip, np.array([[0.25, 0.5]], np.float32))
    hip.check(L.lmp_k_fill(hip.FLOAT32, a.ptr, n, 1.0))
    marks = [0, 1, (1 << 31) + 7, (1 << 32) - 1, 1 << 32, (1 << 32) + 1, n - 1]
    for i in marks:
        v = np.array([100.0 + (i % 1000)], np.float32)
        hip.check(L.lmp_rt_memcpy_h2d(C.c_void_p(a.ptr + 4 * i), v.ctypes.data_as(C.c_void_p), 4))
    out = hip.binary("add", a, b)
    assert tuple(out.shape) == (n, 2)
    a.free()
    probe = marks + [12345, (1 << 32) - 2, n - 2]
    for i in probe:
        row = np.empty(2, np.float32)
        hip.check(L.lmp_rt_memcpy_d2h(row.ctypes.data_as(C.c_void_p), C.c_void_p(out.ptr + 8 * i), 8))
        base = np.float32(100.0 + (i % 1000)) if i in marks else np.float32(1.0)
        assert row[0] == base + np.float32(0.25) and row[1] == base + np.float32(0.5), (i, row)
    out.free()
    hip.check(L.lmp_rt_empty_cache())


def _plant(hip, buf, cols, marks):
    for (r, c), v in marks.items():
        x = np.array([v], np.float32)
        hip.check(hip.lib().lmp_rt_memcpy_h2d(C.c_void_p(buf.ptr + 4 * (r * cols + c)),
                                              x.ctypes.data_as(C.c_void_p), 4))


def test_reduce_offsets_beyond_32_bits(hip):
    """Sum and max over dim 1 of [2, 2^31 + 8] (16 GiB: row 1 starts past 2^31
    floats, each row split over 1024 workgroups) and over dim 0 of
    [2^21 + 3, 1024] (2.1e9 elements, the column kernel's chunks ending past
    2^31 floats): a background of 0 (sum) or -1 (max) with values planted at
    the ends and around 2^30 / 2^31, so every result is exact."""
    L = hip.lib()
    for (rows, cols, axis, marks) in (
            (2, (1 << 31) + 8, 1, {(0, 0): 1.0, (0, (1 << 31) + 7): 2.0, (1, 0): 4.0,
                                   (1, 1 << 30): 16.0, (1, (1 << 31) + 7): 8.0}),
            ((1 << 21) + 3, 1024, 0, {(0, 0): 1.0, ((1 << 21) + 2, 0): 2.0,
                                      ((1 << 21) + 2, 1023): 4.0, (1 << 21, 517): 8.0,
                                      (1 << 20, 3): 32.0})):
        a = hip.DeviceBuffer((rows, cols), np.float32)
        for op, background in (("sum", 0.0), ("max", -1.0)):
            hip.check(L.lmp_k_fill(hip.FLOAT32, a.ptr, rows * cols, background))
            _plant(hip, a, cols, marks)
            want = np.full(rows if axis == 1 else cols, background, np.float32)
            for (r, c), v in marks.items():
                i = r if axis == 1 else c
                want[i] = want[i] + v if op == "sum" else max(want[i], v)
            got = hip.reduce(op, a, axis).numpy().ravel()
            assert np.array_equal(got, want), (rows, cols, op)
        a.free()
        hip.check(L.lmp_rt_empty_cache())


def test_fill_cast_add_inplace(hip):
    L = hip.lib()
    buf = hip.DeviceBuffer((1001,), np.float32)
    hip.check(L.lmp_k_fill(hip.FLOAT32, buf.ptr, 1001, 2.5))
    assert np.array_equal(buf.numpy(), np.full(1001, 2.5, np.float32))
    src = np.arange(1001, dtype=np.float32) * 0.5
    s = up(hip, src)
    d64 = hip.DeviceBuffer((1001,), np.float64)
    hip.check(L.lmp_k_cast(hip.FLOAT32, hip.FLOAT64, d64.ptr, s.ptr, 1001))
    assert np.array_equal(d64.numpy(), src.astype(np.float64))
    for n in (1001, 4096):
        x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        y = np.random.default_rng(n + 1).standard_normal(n).astype(np.float32)
        dx, dy = up(hip, x), up(hip, y)
        hip.check(L.lmp_k_add_inplace(hip.FLOAT32, dx.ptr, dy.ptr, n))
        assert np.array_equal(dx.numpy(), x + y)
        assert np.array_equal(dy.numpy(), y)


REDUCE_CASES = [((300, 257), 0), ((300, 257), 1), ((4, 37, 5), 0), ((4, 37, 5), 1),
                ((4, 37, 5), 2), ((64, 16384), 1), ((16, 8192), 1), ((2, 65536), 1),
                ((2048, 1024), 0), ((512, 4096), 0), ((32, 10), 1), ((32, 10), 0),
                ((512, 1000), 1), ((3, 2), 0), ((1, 1), 0), ((7, 1, 9), 1),
                ((5, 3000, 12), 1),
                # one-pass column strips (axis of at most 4096 rows): ragged
                # strip, several outer slices, the length limit and one past it
                ((512, 1000), 0), ((6, 700, 16), 1), ((4096, 64), 0), ((4097, 64), 0),
                ((100, 4), 0),
                # more outer slices than a grid's z extent
                ((70000, 5, 4), 1),
                # cancelling one-wave sums (-0.129 from 1995 terms up to 3.8,
                # -0.454 from 2506 up to 3.4)
                ((1995,), 0), ((2506,), 0)]


@pytest.mark.parametrize("shape,axis", REDUCE_CASES, ids=str)
def test_reduce(hip, oracle, shape, axis):
    rng = np.random.default_rng(zlib.crc32(repr((shape, axis)).encode()))
    a = rng.standard_normal(shape, dtype=np.float32)
    d = up(hip, a)
    for op in ("max", "min"):
        got = hip.reduce(op, d, axis).numpy()
        assert np.array_equal(got, oracle.reduce(op, a, axis)), op
    got = hip.reduce("sum", d, axis).numpy()
    want = oracle.reduce("sum", a, axis)
    assert got.shape == want.shape
    assert_sum_close(got, want, a, axis)
    small = (1.0 + 0.01 * a).astype(np.float32)
    got = hip.reduce("prod", up(hip, small), axis).numpy()
    assert rel_err(got, oracle.reduce("prod", small, axis)) <= 1e-5


def test_reduce_ones_column_is_exact(hip):
    """Size-independent property at the config-2 shape: the backward of a
    [16384,16384] + [1,16384] broadcast add reduces a ones gradient over dim
    0, which must give exactly 16384.0 in every column."""
    n = 16384
    L = hip.lib()
    ones = hip.DeviceBuffer((n, n), np.float32)
    hip.check(L.lmp_k_fill(hip.FLOAT32, ones.ptr, n * n, 1.0))
    out = hip.reduce("sum", ones, 0).numpy()
    assert out.shape == (1, n) and np.all(out == np.float32(n))
    out1 = hip.reduce("sum", ones, 1).numpy()
    assert np.all(out1 == np.float32(n))
    ones.free()


@pytest.mark.parametrize("length", [37, 1000, 4096, 16384])
@pytest.mark.parametrize("axis", [0, 1])
def test_reduce_special_values(hip, oracle, length, axis):
    """max/min over rows holding infinities, NaN, signed zeros and all -inf
    (Lamp3's std::max(acc, x) from lowest() never lets NaN in and leaves an
    all -inf row at lowest()): bit for bit as the oracle, except the sign of a
    zero result where +0 and -0 both attain it (row 6 for max, row 7 for min):
    the CPU loop keeps the first in index order, the GPU's combine tree the
    first in its order, so only the value (0) is compared there.  sum/prod:
    NaN where the oracle has NaN (NaN inputs), equal infinities, finite
    results within 1e-5 under max|d| / max|true|."""
    rng = np.random.default_rng(length + 7 * axis)
    rows = special_rows(length, rng)
    a = np.ascontiguousarray(rows if axis == 1 else rows.T)
    d = up(hip, a)
    for op, tie_row in (("max", 6), ("min", 7)):
        got = hip.reduce(op, d, axis).numpy().reshape(-1)
        want = oracle.reduce(op, a, axis).reshape(-1)
        keep = np.arange(want.size) != tie_row
        assert np.array_equal(got[keep].view(np.uint32), want[keep].view(np.uint32)), op
        assert got[tie_row] == 0.0 and want[tie_row] == 0.0, op
    assert oracle.reduce("max", a, axis).reshape(-1)[0] == np.finfo(np.float32).min
    for op in ("sum", "prod"):
        src = a if op == "sum" else np.where(np.isfinite(a), 1.0 + 0.001 * a, a).astype(np.float32)
        got = hip.reduce(op, up(hip, src), axis).numpy().reshape(-1)
        want = oracle.reduce(op, src, axis).reshape(-1)
        assert np.array_equal(np.isnan(got), np.isnan(want)), op
        assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)]), op
        fin = np.isfinite(want)
        assert rel_err(got[fin], want[fin]) <= 1e-5, op


@pytest.mark.parametrize("shape,axis", [((3, 0, 2), 1), ((0, 4), 0), ((4, 0), 1), ((0,), 0)],
                         ids=str)
def test_reduce_empty_axis_writes_identity(hip, oracle, shape, axis):
    """A reduction over an empty axis writes the identity to every output
    (cpu/reduct.cpp:14-19 folds nothing into kIdentity), bit for bit as the
    oracle, sign of zero included; the input pointer may then be null."""
    L = hip.lib()
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    oshape = list(shape)
    oshape[axis] = 1
    for op in ("sum", "max", "min", "prod"):
        out = up(hip, np.full(oshape, np.nan, np.float32))
        hip.check(L.lmp_k_reduce(hip.RED[op], hip.FLOAT32, out.ptr, None, outer, 0, inner))
        want = oracle.reduce(op, np.zeros(shape, np.float32), axis)
        assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32)), op


def test_empty_extents_write_nothing(hip, oracle):
    """Zero-extent calls through the C ABI succeed and leave memory as it was:
    elementwise, fill, cast and add_inplace of 0 elements, reductions with no
    outer or inner position, GEMMs with m or n = 0, copies of 0 bytes.  A GEMM
    with k = 0 writes the empty product, zeros (the oracle's), or leaves C as it
    is when accumulating."""
    L = hip.lib()
    pattern = np.arange(16, dtype=np.float32) + 0.5
    g, src = up(hip, pattern), up(hip, pattern[::-1])
    d, _ = hip.make_bcast((0, 4), (1, 4))
    hip.check(L.lmp_k_binary(hip.BIN["add"], hip.FLOAT32, g.ptr, src.ptr, src.ptr, C.byref(d),
                             0.0, 0.0))
    hip.check(L.lmp_k_unary(hip.UN["exp"], hip.FLOAT32, g.ptr, src.ptr, 0, 0.0, 0.0))
    hip.check(L.lmp_k_fill(hip.FLOAT32, g.ptr, 0, 7.0))
    hip.check(L.lmp_k_cast(hip.FLOAT32, hip.FLOAT64, g.ptr, src.ptr, 0))
    hip.check(L.lmp_k_add_inplace(hip.FLOAT32, g.ptr, src.ptr, 0))
    for outer, length, inner in ((0, 5, 3), (4, 5, 0), (0, 0, 0)):
        hip.check(L.lmp_k_reduce(hip.RED["sum"], hip.FLOAT32, g.ptr, src.ptr, outer, length,
                                 inner))
    for m, n in ((0, 4), (4, 0)):
        hip.check(L.lmp_k_gemm_f32(0, 0, m, n, 3, src.ptr, 3, src.ptr, 4, g.ptr, 4, 0))
    hip.check(L.lmp_rt_memcpy_d2d(g.ptr, src.ptr, 0))
    hip.check(L.lmp_rt_memcpy_h2d(g.ptr, pattern[::-1].copy().ctypes.data, 0))
    assert np.array_equal(g.numpy(), pattern)
    hip.check(L.lmp_k_gemm_f32(0, 0, 4, 4, 0, src.ptr, 1, src.ptr, 4, g.ptr, 4, 1))
    assert np.array_equal(g.numpy(), pattern)
    hip.check(L.lmp_k_gemm_f32(0, 0, 4, 4, 0, src.ptr, 1, src.ptr, 4, g.ptr, 4, 0))
    want = oracle.matmul(np.zeros((4, 0), np.float32), np.zeros((0, 4), np.float32))
    assert np.array_equal(g.numpy().reshape(4, 4).view(np.uint32), want.view(np.uint32))


# M <= 32 with 16-byte rows takes the register-direct kernel: (32, 132, 1028)
# and (20, 132, 1028) split K with a ragged last split and a partial column
# block, (4, 260, 2048) splits K eight ways, (1, 8, 8) is a single row.
GEMM_SHAPES = [(64, 64, 64), (128, 256, 96), (33, 17, 70), (32, 512, 1024),
               (256, 1000, 128), (32, 64, 256), (32, 10, 64), (200, 3, 5),
               (1, 7, 3), (512, 512, 2048), (130, 260, 33), (32, 132, 1028),
               (20, 132, 1028), (4, 260, 2048), (1, 8, 8),
               # the tiny kernel's limits (K <= 512, at most 2^21 multiply-adds)
               # and odd K; just past them, the 32 x 256 and 64 x 64 tiles
               (64, 64, 512), (64, 65, 512), (40, 33, 1), (31, 70, 3),
               (48, 300, 1000), (130, 260, 600)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES, ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm(hip, oracle, m, n, k, ta, tb):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = (rng.standard_normal((m, k)) * 0.5).astype(np.float32)
    b = (rng.standard_normal((k, n)) * 0.5).astype(np.float32)
    want = oracle.matmul(a, b)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (m, n)
    assert rel_err(got, want) <= 1e-4
    # accumulate: C += A*B
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert rel_err(dc.numpy(), c0.astype(np.float64) + want) <= 1e-4


# Shapes that reach each LDS-DMA configuration with ragged tiles and a ragged
# last K tile: 256 x 256 tiles (their tiles cover the CUs), 256 x 128 tiles
# split over K (M >= 512, N >= 2048, K >= 2048), 128 x 128 tiles unsplit and
# split 13 ways.  Operands are small integers, so every product and partial
# sum is exact in float32 and the result must equal the float64 product bit
# for bit whatever the order: a skipped, repeated or misplaced MFMA step, tile
# or K split shows as a wrong integer.
LDS_EXACT_SHAPES = [(4000, 4100, 300), (520, 2100, 2080), (2100, 2100, 700),
                    (600, 1000, 4096)]


@pytest.mark.parametrize("m,n,k", LDS_EXACT_SHAPES, ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_lds_paths_exact_on_integer_operands(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m + 5 * n + 7 * k + 11 * ta + 13 * tb)
    a = rng.integers(-4, 5, (m, k)).astype(np.float32)
    b = rng.integers(-4, 5, (k, n)).astype(np.float32)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got, want)
    c0 = rng.integers(-100, 101, (m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert np.array_equal(dc.numpy(), c0 + want)


def test_gemm_config3_square(hip, oracle):
    """M=N=K=4096 with entries N(0, 0.02): fwd, dX and dW orientations against
    float64 (the oracle's naive fp32 GEMM at this size takes minutes; its
    order is pinned separately on small cases)."""
    n = 4096
    rng = np.random.default_rng(31)
    a = (rng.standard_normal((n, n)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((n, n)) * 0.02).astype(np.float32)
    da, db = up(hip, a), up(hip, b)
    rows = rng.choice(n, 64, replace=False)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    for ta, tb in ((0, 0), (0, 1), (1, 0)):
        got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
        A = a64.T if ta else a64
        B = b64.T if tb else b64
        want = A[rows] @ B
        assert rel_err(got[rows], want) <= 1e-4, (ta, tb)


@pytest.mark.parametrize("m,n,k", [(8, 8, 8), (64, 64, 64), (300, 260, 96), (32, 4096, 512),
                                   (512, 512, 512), (1024, 1024, 1024)], ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_gemm_subnormal_products_and_specials(hip, m, n, k, ta, tb):
    """Operands near 1e-20 make every product subnormal (about 1e-40): the
    MFMA and register paths keep them (no flush to zero), within 1e-4 of the
    float64 product under max|d| / max|true|.  An inf in A and a NaN in B put
    NaN and inf in C where the float64 product has them."""
    rng = np.random.default_rng(zlib.crc32(repr((m, n, k, ta, tb)).encode()))
    a = (rng.uniform(0.5, 1.5, (k, m) if ta else (m, k)) * 1e-20).astype(np.float32)
    b = (rng.uniform(0.5, 1.5, (n, k) if tb else (k, n)) * 1e-20).astype(np.float32)
    got = hip.gemm(up(hip, a), up(hip, b), bool(ta), bool(tb)).numpy()
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    assert np.all(got != 0.0) and rel_err(got, want) <= 1e-4
    a2 = rng.standard_normal(a.shape).astype(np.float32)
    b2 = rng.standard_normal(b.shape).astype(np.float32)
    a2[0, 0] = np.inf
    b2[(1, 0) if tb else (0, 1)] = np.nan
    got2 = hip.gemm(up(hip, a2), up(hip, b2), bool(ta), bool(tb)).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        want2 = (a2.T if ta else a2).astype(np.float64) @ (b2.T if tb else b2).astype(np.float64)
    assert np.array_equal(np.isnan(got2), np.isnan(want2))
    assert np.array_equal(got2[np.isinf(want2)], want2[np.isinf(want2)].astype(np.float32))
    fin = np.isfinite(want2)
    assert rel_err(got2[fin], want2[fin]) <= 1e-4


def test_gemm_8192_cube(hip):
    """M=N=K=8192 (the north star's 8192-scale matmul) with entries
    N(0, 0.02) in the three Linear orientations: forward X.W, dX = dY.W^T and
    dW = X^T.dY.  64 sampled rows and 64 sampled columns of each product
    against float64 at 1e-4 (matrix.cu:178-199 is the entry replaced)."""
    n = 8192
    rng = np.random.default_rng(8192)
    a = (rng.standard_normal((n, n), dtype=np.float32) * np.float32(0.02))
    b = (rng.standard_normal((n, n), dtype=np.float32) * np.float32(0.02))
    da, db = up(hip, a), up(hip, b)
    rows = np.concatenate([rng.choice(n, 62, replace=False), [0, n - 1]])
    cols = np.concatenate([rng.choice(n, 62, replace=False), [0, n - 1]])
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    for ta, tb in ((0, 0), (0, 1), (1, 0)):
        got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
        A = a64.T if ta else a64
        B = b64.T if tb else b64
        assert rel_err(got[rows], A[rows] @ B) <= 1e-4, (ta, tb, "rows")
        assert rel_err(got[:, cols], A @ B[:, cols]) <= 1e-4, (ta, tb, "cols")
        del got


def gemm_large_case(hip, rng):
    """One random large GEMM (extents log-uniform up to 9000, at least 2^30
    multiply-adds, any orientation; plain, accumulating or bias + ReLU): 26
    sampled rows and 26 sampled columns against float64 at 1e-4."""
    L = hip.lib()
    # extents log-uniform in [1, 9000], redrawn until the product has at
    # least 2^30 multiply-adds: large tile walks, ragged edges, split K
    while True:
        m, n, k = (int(np.exp(rng.uniform(0.0, np.log(9000.0)))) for _ in range(3))
        if m * n * k >= (1 << 30):
            break
    ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    kind = str(rng.choice(["gemm", "acc", "relu"]))
    ar, ac = (k, m) if ta else (m, k)
    br, bc = (n, k) if tb else (k, n)
    a = rng.standard_normal((ar, ac), dtype=np.float32) * np.float32(0.02)
    b = rng.standard_normal((br, bc), dtype=np.float32) * np.float32(0.02)
    bias = rng.standard_normal(n, dtype=np.float32) * np.float32(0.01)
    c0 = rng.standard_normal((m, n), dtype=np.float32) * np.float32(0.01)
    da, db, dbias = (hip.DeviceBuffer.from_numpy(x) for x in (a, b, bias))
    dc = hip.DeviceBuffer.from_numpy(c0)
    if kind == "relu":
        st = L.lmp_k_linear_relu_f32(ta, tb, m, n, k, da.ptr, ac, db.ptr, bc, dbias.ptr, dc.ptr, n)
    else:
        st = L.lmp_k_gemm_f32(ta, tb, m, n, k, da.ptr, ac, db.ptr, bc, dc.ptr, n, int(kind == "acc"))
    hip.check(st)
    got = dc.numpy()
    del da, db, dc
    A = (a.T if ta else a).astype(np.float64)
    B = (b.T if tb else b).astype(np.float64)
    rows = np.concatenate([rng.choice(m, min(m, 24), replace=False), [0, m - 1]])
    cols = np.concatenate([rng.choice(n, min(n, 24), replace=False), [0, n - 1]])
    for part, g, want, base, bb in (("rows", got[rows], A[rows] @ B, c0[rows], bias),
                                    ("cols", got[:, cols], A @ B[:, cols], c0[:, cols], bias[cols])):
        if kind == "acc":
            want = want + base
        elif kind == "relu":
            want = np.maximum(want + bb, 0.0)
        assert rel_err(g, want) <= 1e-4, (m, n, k, ta, tb, kind, part)


@pytest.mark.parametrize("seed", range(6))
def test_gemm_large_random_shapes(hip, seed):
    gemm_large_case(hip, np.random.default_rng(9000 + seed))


# Shapes routed to the one-workgroup-per-CU LDS tiles, with ragged edges in
# m, n and k: (4100, 4036, 100) fills the CUs with 256 x 256 tiles (partial
# last tile row and column, K not a multiple of 32); (520, 2052, 2080) takes
# 256 x 128 tiles with K split five ways.
@pytest.mark.parametrize("m,n,k", [(4100, 4036, 100), (520, 2052, 2080)], ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_wide_tiles(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m + n + k + 2 * ta + tb)
    a = (rng.standard_normal((m, k)) * 0.1).astype(np.float32)
    b = (rng.standard_normal((k, n)) * 0.1).astype(np.float32)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    rows = np.concatenate([rng.choice(m, 48, replace=False), [0, m - 1]])
    want = a[rows].astype(np.float64) @ b.astype(np.float64)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert rel_err(got[rows], want) <= 1e-4
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert rel_err(dc.numpy()[rows], c0[rows].astype(np.float64) + want) <= 1e-4


# M <= 32 with B transposed and at least one 32-column block per CU takes the
# whole-rows kernel (no split of K): config 3's dX, a short batch with a
# ragged column block and K not a multiple of the 32-value groups, and a
# very short K.
@pytest.mark.parametrize("m,n,k", [(32, 8192, 4096), (7, 8200, 1000), (32, 8256, 36)], ids=str)
def test_gemm_thin_rows(hip, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = (rng.standard_normal((m, k)) * 0.1).astype(np.float32)
    bs = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)  # stored [n, k]
    da, db = up(hip, a), up(hip, bs)
    want = a.astype(np.float64) @ bs.astype(np.float64).T
    got = hip.gemm(da, db, trans_b=True).numpy()
    assert rel_err(got, want) <= 1e-4
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_b=True, out=dc, accumulate=True)
    assert rel_err(dc.numpy(), c0.astype(np.float64) + want) <= 1e-4
    # the Linear epilogue (bias, then ReLU) on this path
    bias = rng.standard_normal(n).astype(np.float32)
    dbias = up(hip, bias)
    L = hip.lib()
    for entry, relu in ((L.lmp_k_linear_f32, False), (L.lmp_k_linear_relu_f32, True)):
        out = hip.DeviceBuffer((m, n), np.float32)
        hip.check(entry(0, 1, m, n, k, da.ptr, k, db.ptr, k, dbias.ptr, out.ptr, n))
        lin = got + bias  # the product rounded to fp32, then the bias added once
        if relu:
            lin = np.where(lin < 0, np.float32(0), lin)
        assert np.array_equal(out.numpy(), lin), relu


def test_transpose(hip):
    for shape in ((3, 2), (64, 64), (130, 70), (1, 9)):
        a = np.random.default_rng(0).standard_normal(shape).astype(np.float32)
        d = up(hip, a)
        out = hip.DeviceBuffer((shape[1], shape[0]), np.float32)
        hip.check(hip.lib().lmp_k_transpose(hip.FLOAT32, out.ptr, d.ptr, *shape))
        assert np.array_equal(out.numpy(), a.T)


def test_jit_compile_launch_cache(hip):
    L = hip.lib()
    src = b"""
extern "C" __global__ void lmp_probe(float* out, const float* a, unsigned n) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] * a[i] + 1.0f;
}
"""
    key = 0x1234ABCD5678
    h = C.c_void_p()
    assert L.lmp_jit_lookup(key, C.byref(h)) != hip.OK
    hip.check(L.lmp_jit_compile(key, src, b"lmp_probe", C.byref(h)))
    h2 = C.c_void_p()
    hip.check(L.lmp_jit_lookup(key, C.byref(h2)))
    assert h.value == h2.value
    x = np.linspace(-3, 3, 1000).astype(np.float32)
    dx = up(hip, x)
    out = hip.DeviceBuffer((1000,), np.float32)
    p_out, p_a, n = C.c_void_p(out.ptr), C.c_void_p(dx.ptr), C.c_uint32(1000)
    args = (C.c_void_p * 3)(C.addressof(p_out), C.addressof(p_a), C.addressof(n))
    hip.check(L.lmp_jit_launch(h, 4, 256, args))
    assert np.array_equal(out.numpy(), (x * x).astype(np.float32) + np.float32(1))


def test_errors_are_reported(hip):
    L = hip.lib()
    assert L.lmp_k_binary(99, hip.FLOAT32, 1, 1, 1, None, 0.0, 0.0) == hip.ERR_INVALID
    d, _ = hip.make_bcast((2, 2), (2, 2))
    x = hip.DeviceBuffer((2, 2), np.float32)
    assert L.lmp_k_binary(99, hip.FLOAT32, x.ptr, x.ptr, x.ptr, C.byref(d), 0.0, 0.0) \
        == hip.ERR_INVALID
    assert b"unknown op" in L.lmp_rt_last_error()
    assert L.lmp_rt_free(C.c_void_p(0xdead00)) == hip.ERR_INVALID


# lmp_k_gemm_colsum_f32: a Linear's weight gradient and bias gradient (the
# column sums of op(B)) together.  C must equal the plain GEMM bit for bit
# (same kernel), the column sums the float64 sums to the reductions' bar, and
# accumulation must add the same values in place.  Small products take one
# launch (the tiny kernel, 16- and 32-wide blocks); (300, 500, 600) splits K,
# so it runs the GEMM and then the dim-0 reduction; config 4's weight
# gradients (4096, 4096, 512) and (4096, 1000, 512) and the ragged
# (4100, 1000, 500) run on LDS tiles without a split, where the first tile row
# also sums B (when B is not transposed).  With A transposed and K <= 32,
# (8192, 4096, 32) (config 3's weight gradient) and the ragged (1000, 996, 17)
# run on the persistent short-K kernel, which sums B the same way.
@pytest.mark.parametrize("m,n,k", [(256, 64, 32), (64, 10, 32), (40, 33, 7), (512, 300, 12),
                                   (300, 500, 600), (4096, 4096, 512), (4096, 1000, 512),
                                   (4100, 1000, 500), (8192, 4096, 32), (1000, 996, 17)],
                         ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_colsum(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m * 5 + n + k + ta + 2 * tb)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    plain = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    L = hip.lib()
    c = hip.DeviceBuffer((m, n), np.float32)
    cs = hip.DeviceBuffer((n,), np.float32)
    hip.check(L.lmp_k_gemm_colsum_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr, db.shape[1],
                                      c.ptr, n, 0, cs.ptr, 0))
    assert np.array_equal(c.numpy(), plain)
    sums = cs.numpy()
    truth = b.astype(np.float64).sum(0)
    assert np.max(np.abs(sums - truth)) <= 1e-5 * max(1.0, np.max(np.abs(truth)))
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    s0 = rng.standard_normal(n).astype(np.float32)
    dc, dcs = up(hip, c0), up(hip, s0)
    hip.check(L.lmp_k_gemm_colsum_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr, db.shape[1],
                                      dc.ptr, n, 1, dcs.ptr, 1))
    assert np.array_equal(dc.numpy(), c0 + plain)
    assert np.array_equal(dcs.numpy(), s0 + sums)


# Short-K products with a large C (write-bound, like config 3's skinny weight
# gradient): ragged M and N, odd K, K = 1.  With A transposed, K <= 32 and
# 16-byte rows, (2048, 2048, 32), (3000, 1500, 1), (8192, 4096, 32) and
# (1000, 996, 17) run on the persistent short-K kernel (more tiles than
# resident workgroups, ragged edge tiles).
@pytest.mark.parametrize("m,n,k", [(4100, 1030, 31), (2048, 2048, 32), (3000, 1500, 1),
                                   (4100, 1030, 33), (8192, 4096, 32), (1000, 996, 17)],
                         ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_short_k_large_c(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m + n + k + 10 * ta + 20 * tb)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert rel_err(got, want) <= 1e-5
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert np.array_equal(dc.numpy(), c0 + got)
    bias = rng.standard_normal(n).astype(np.float32)
    dbias = up(hip, bias)
    out = hip.DeviceBuffer((m, n), np.float32)
    hip.check(hip.lib().lmp_k_linear_relu_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr,
                                              db.shape[1], dbias.ptr, out.ptr, n))
    t = got + bias[None, :]
    assert np.array_equal(out.numpy().view(np.uint32),
                          np.where(t < 0, np.float32(0), t).view(np.uint32))


# lmp_k_linear_f32: the bias rides in every GEMM path's epilogue (register-
# direct M <= 32, skinny M <= 64, the scalar-load kernel for odd strides, the
# split-K fold, the 128/256-wide LDS tiles), so C must equal the plain GEMM
# followed by a float32 bias add, bit for bit.
LINEAR_SHAPES = [(32, 64, 256), (20, 132, 1028), (48, 96, 64), (200, 130, 70),
                 (256, 1000, 128), (512, 2048, 2048), (4096, 4096, 256),
                 # K <= 32 past the tiny kernel's range: A transposed takes the
                 # short-K kernel, with or without a bias
                 (28, 3272, 28), (32, 4072, 20), (640, 2048, 32)]


@pytest.mark.parametrize("m,n,k", LINEAR_SHAPES, ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_linear_bias_epilogue_equals_gemm_then_add(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m + 3 * n + 7 * k + ta + 2 * tb)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    dbias = up(hip, bias)
    plain = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    out = hip.DeviceBuffer((m, n), np.float32)
    hip.check(hip.lib().lmp_k_linear_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr,
                                         db.shape[1], dbias.ptr, out.ptr, n))
    want = plain + bias[None, :]
    assert np.array_equal(out.numpy(), want)
    # ReLU in the same epilogue: clamp(t, 0, DBL_MAX) in float32, t < 0 -> +0
    hip.check(hip.lib().lmp_k_linear_relu_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr,
                                              db.shape[1], dbias.ptr, out.ptr, n))
    relu = np.where(want < 0, np.float32(0), want)
    assert np.array_equal(out.numpy().view(np.uint32), relu.view(np.uint32))
    # a bias that is not 16-byte aligned (one float into a buffer) gives the
    # same bits: the kernel choice does not depend on where the bias lies
    shifted = up(hip, np.concatenate([[np.float32(7)], bias]).astype(np.float32))
    hip.check(hip.lib().lmp_k_linear_relu_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr,
                                              db.shape[1], shifted.ptr + 4, out.ptr, n))
    assert np.array_equal(out.numpy().view(np.uint32), relu.view(np.uint32))


# Random shapes drawn on both sides of every kernel-selection threshold (M <= 32
# register-direct and whole-rows, M <= 64 skinny tiles, K <= 32 short-K, the
# tiny kernel's 2^21 multiply-adds, tiles covering the CUs, K split or not,
# 16-byte rows or not), every orientation: the product against float64 within
# 1e-5 of its largest value, accumulate as the fp32 sum of C and the product bit
# for bit, and bias + ReLU on the same product bit for bit.
def _random_gemm_shapes(count, seed):
    rng = np.random.default_rng(seed)
    shapes = []
    while len(shapes) < count:
        m = int(rng.choice([rng.integers(1, 33), rng.integers(33, 65), rng.integers(65, 700),
                            rng.integers(700, 2100)]))
        n = int(rng.choice([rng.integers(1, 130), rng.integers(130, 1100), rng.integers(1100, 4200)]))
        k = int(rng.choice([rng.integers(1, 33), rng.integers(33, 600), rng.integers(600, 4200)]))
        if rng.random() < 0.5:  # keep 16-byte rows half of the time
            m, n, k = [max(4, d - d % 4) for d in (m, n, k)]
        if m * n * k <= (1 << 31) and m * n <= (1 << 23):
            shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize("m,n,k", _random_gemm_shapes(24, 2026) + [(20, 8200, 100), (600, 2100, 2100),
                                                   (28, 3272, 28), (28, 4048, 20)],
                         ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_random_shapes_every_path(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m * 131 + n * 17 + k + 3 * ta + tb)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_err(got, want) <= 1e-5
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert np.array_equal(dc.numpy(), c0 + got)
    bias = rng.standard_normal(n).astype(np.float32)
    dbias = up(hip, bias)  # held: a freed buffer could be handed to the split-K partials
    out = hip.DeviceBuffer((m, n), np.float32)
    hip.check(hip.lib().lmp_k_linear_relu_f32(ta, tb, m, n, k, da.ptr, da.shape[1], db.ptr,
                                              db.shape[1], dbias.ptr, out.ptr, n))
    t = got + bias[None, :]
    assert np.array_equal(out.numpy().view(np.uint32),
                          np.where(t < 0, np.float32(0), t).view(np.uint32))


# ------------------------------------------------------------ host <-> device

STAGE = 16 << 20  # bytes per staging chunk of lmp_rt_memcpy_h2d/d2h
STAGED_MIN = 4 << 20


def test_kernel_launch_count(hip):
    """lmp_rt_kernel_launch_count counts the kernels the library launched: one
    for a broadcast add, a short-row reduction or a tiny GEMM, two for a
    split-K GEMM (the product and its fold), none for an empty call."""
    L = hip.lib()

    def count():
        c = C.c_uint64(0)
        hip.check(L.lmp_rt_kernel_launch_count(C.byref(c)))
        return c.value

    rng = np.random.default_rng(9)
    a = up(hip, rng.standard_normal((64, 33), dtype=np.float32))
    b = up(hip, rng.standard_normal((64, 1), dtype=np.float32))
    x = up(hip, rng.standard_normal((256, 4096), dtype=np.float32))
    w = up(hip, rng.standard_normal((4096, 256), dtype=np.float32))
    s = up(hip, rng.standard_normal((8, 8), dtype=np.float32))
    cases = [(lambda: hip.binary("add", a, b), 1), (lambda: hip.reduce("sum", a, 1), 1),
             (lambda: hip.gemm(s, s), 1), (lambda: hip.gemm(x, w), 2),
             (lambda: hip.check(L.lmp_k_fill(hip.FLOAT32, a.ptr, 0, 1.0)), 0)]
    for fn, want in cases:
        before = count()
        fn()
        assert count() - before == want
    hip.check(L.lmp_rt_synchronize())


def test_c_abi_from_several_host_threads(hip, oracle):
    """Four host threads drive the C ABI at once (ctypes releases the GIL):
    each allocates, uploads (staged and direct copies), runs a broadcast add,
    a dim-1 sum and a split-K GEMM whose partials come from the shared pool,
    downloads and frees, 6 rounds each, with shapes of its own.  Every result
    equals the oracle's (add, exact) or float64's (sum, GEMM, 1e-5 / 1e-4):
    the pool, the staging buffers and the one library stream are shared
    safely."""
    import threading
    L = hip.lib()
    errors = []

    def work(tid):
        try:
            rng = np.random.default_rng(100 + tid)
            for rnd in range(6):
                m, n = 200 + 37 * tid + rnd, 300 + 11 * tid
                a = rng.standard_normal((m, n), dtype=np.float32)
                b = rng.standard_normal((1, n), dtype=np.float32)
                da, db = up(hip, a), up(hip, b)
                s = hip.binary("add", da, db).numpy()
                assert np.array_equal(s.view(np.uint32), oracle.binary("add", a, b).view(np.uint32))
                r = hip.reduce("sum", da, 1).numpy()
                assert rel_err(r, a.astype(np.float64).sum(1, keepdims=True)) <= 1e-5
                x = rng.standard_normal((256, 4096), dtype=np.float32)
                w = rng.standard_normal((4096, 256), dtype=np.float32)
                got = hip.gemm(up(hip, x), up(hip, w)).numpy()
                assert rel_err(got, x.astype(np.float64) @ w.astype(np.float64)) <= 1e-4
                for buf in (da, db):
                    buf.free()
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            errors.append((tid, repr(e)))

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    hip.check(L.lmp_rt_synchronize())


@pytest.mark.parametrize("nbytes", [STAGED_MIN - 4, STAGED_MIN, STAGE, STAGE + 4,
                                    3 * STAGE + 12, 100 * (1 << 20) + 8])
def test_host_device_round_trip_every_byte(hip, nbytes):
    """Copies below and above the staging threshold, of whole, partial and
    several chunks, keep every bit (random words, NaN payloads included), in
    both directions; a download right after a kernel sees its result."""
    n = nbytes // 4
    words = np.random.default_rng(nbytes).integers(0, 2 ** 32, n, dtype=np.uint32)
    src = words.view(np.float32)
    buf = up(hip, src)
    back = buf.numpy()
    assert back.view(np.uint32).tobytes() == words.tobytes()
    # the download is ordered after the work queued before it
    check_fill = hip.lib().lmp_k_fill(hip.CODE_OF[np.dtype(np.float32)], buf.ptr, n, 0.75)
    hip.check(check_fill)
    assert np.all(buf.numpy() == np.float32(0.75))
    # upload into part of a larger buffer (offset destination), download the part
    big = hip.DeviceBuffer((n + 3,), np.float32)
    hip.check(hip.lib().lmp_rt_memcpy_h2d(big.ptr + 12, src.ctypes.data, n * 4))
    part = np.empty(n, np.float32)
    hip.check(hip.lib().lmp_rt_memcpy_d2h(part.ctypes.data, big.ptr + 12, n * 4))
    assert part.view(np.uint32).tobytes() == words.tobytes()


# (batch, in, out): the README MLP's two layers, odd and single-row sizes in
# the one-launch range, then a product just past it (K > 512) on two
# launches; config 4's layers and two more shapes whose dW and dX both take
# LDS tiles of one workgroup size, so they share one launch (dW on 128 x 128
# and dX on 128 x 64 tiles; 256 x 256 and 256 x 128 split four ways; 128 x 64
# both split; 256 x 128 both split).
@pytest.mark.parametrize("batch,fan_in,fan_out", [
    (32, 64, 10), (32, 256, 64), (7, 33, 5), (1, 3, 1), (40, 17, 600), (512, 4096, 1000),
    (512, 4096, 4096), (768, 1024, 1000), (4096, 2048, 2048)],
    ids=str)
@pytest.mark.parametrize("acc", [False, True], ids=["write", "accumulate"])
def test_linear_backward_equals_separate_calls(hip, batch, fan_in, fan_out, acc):
    """lmp_k_linear_backward_f32 (dX = G W^T, dW = X^T G and db = the column
    sums of G, one launch for small products) equals lmp_k_gemm_f32 for dX
    and lmp_k_gemm_colsum_f32 for dW and db bit for bit, writing and
    accumulating; and dW is X^T G against float64 on the host."""
    L = hip.lib()
    rng = np.random.default_rng(batch * 7 + fan_in * 3 + fan_out)
    x_np = rng.standard_normal((batch, fan_in)).astype(np.float32)
    w_np = rng.standard_normal((fan_in, fan_out)).astype(np.float32)
    g_np = rng.standard_normal((batch, fan_out)).astype(np.float32)
    g_np.reshape(-1)[3::41] = -0.0
    dx0 = rng.standard_normal((batch, fan_in)).astype(np.float32)
    dw0 = rng.standard_normal((fan_in, fan_out)).astype(np.float32)
    db0 = rng.standard_normal(fan_out).astype(np.float32)
    x, w, g = up(hip, x_np), up(hip, w_np), up(hip, g_np)
    dx_ref, dw_ref, db_ref = up(hip, dx0), up(hip, dw0), up(hip, db0)
    hip.check(L.lmp_k_gemm_f32(0, 1, batch, fan_in, fan_out, g.ptr, fan_out, w.ptr, fan_out,
                               dx_ref.ptr, fan_in, int(acc)))
    hip.check(L.lmp_k_gemm_colsum_f32(1, 0, fan_in, fan_out, batch, x.ptr, fan_in, g.ptr,
                                      fan_out, dw_ref.ptr, fan_out, int(acc), db_ref.ptr,
                                      int(acc)))
    dx, dw, db = up(hip, dx0), up(hip, dw0), up(hip, db0)
    hip.check(L.lmp_k_linear_backward_f32(batch, fan_in, fan_out, x.ptr, fan_in, w.ptr, fan_out,
                                          g.ptr, fan_out, dx.ptr, fan_in, int(acc), dw.ptr,
                                          fan_out, int(acc), db.ptr, int(acc)))
    for got, ref in ((dx, dx_ref), (dw, dw_ref), (db, db_ref)):
        assert np.array_equal(got.numpy().view(np.uint32), ref.numpy().view(np.uint32))
    rows = np.arange(fan_in) if fan_in <= 1024 else rng.choice(fan_in, 64, replace=False)
    want = x_np.T[rows].astype(np.float64) @ g_np.astype(np.float64) + (dw0[rows] if acc else 0.0)
    assert rel_err(dw.numpy()[rows], want) <= 1e-5
    xrows = np.arange(batch) if batch <= 1024 else rng.choice(batch, 64, replace=False)
    want = g_np[xrows].astype(np.float64) @ w_np.astype(np.float64).T + (dx0[xrows] if acc else 0.0)
    assert rel_err(dx.numpy()[xrows], want) <= 1e-4
    want = g_np.astype(np.float64).sum(0) + (db0 if acc else 0.0)
    assert rel_err(db.numpy(), want) <= 1e-5
    # null outputs are rejected, an empty batch is unsupported
    assert L.lmp_k_linear_backward_f32(batch, fan_in, fan_out, x.ptr, fan_in, w.ptr, fan_out,
                                       g.ptr, fan_out, None, fan_in, 0, dw.ptr, fan_out, 0,
                                       db.ptr, 0) == hip.ERR_INVALID
    assert L.lmp_k_linear_backward_f32(0, fan_in, fan_out, x.ptr, fan_in, w.ptr, fan_out,
                                       g.ptr, fan_out, dx.ptr, fan_in, 0, dw.ptr, fan_out, 0,
                                       db.ptr, 0) == hip.ERR_UNSUPPORTED


# Seeded random Linear shapes past the tiny range with 16-byte rows, so that
# dW and dX both take LDS tiles (of one workgroup size or not): the paired
# launch, or the two calls, must give the bits of the separate calls.
_PAIR_RNG = np.random.default_rng(20260)
PAIR_SHAPES = [(int(_PAIR_RNG.integers(130, 2700)), 4 * int(_PAIR_RNG.integers(129, 1026)),
                4 * int(_PAIR_RNG.integers(129, 1026))) for _ in range(8)]


@pytest.mark.parametrize("batch,fan_in,fan_out", PAIR_SHAPES, ids=str)
def test_linear_backward_random_shapes_equal_separate_calls(hip, batch, fan_in, fan_out):
    L = hip.lib()
    rng = np.random.default_rng(batch + 3 * fan_in + 7 * fan_out)
    x_np = (rng.standard_normal((batch, fan_in)) * 0.1).astype(np.float32)
    w_np = (rng.standard_normal((fan_in, fan_out)) * 0.1).astype(np.float32)
    g_np = (rng.standard_normal((batch, fan_out)) * 0.1).astype(np.float32)
    x, w, g = up(hip, x_np), up(hip, w_np), up(hip, g_np)
    for acc in (0, 1):
        dx0 = rng.standard_normal((batch, fan_in)).astype(np.float32)
        dw0 = rng.standard_normal((fan_in, fan_out)).astype(np.float32)
        db0 = rng.standard_normal(fan_out).astype(np.float32)
        dx_ref, dw_ref, db_ref = up(hip, dx0), up(hip, dw0), up(hip, db0)
        hip.check(L.lmp_k_gemm_f32(0, 1, batch, fan_in, fan_out, g.ptr, fan_out, w.ptr, fan_out,
                                   dx_ref.ptr, fan_in, acc))
        hip.check(L.lmp_k_gemm_colsum_f32(1, 0, fan_in, fan_out, batch, x.ptr, fan_in, g.ptr,
                                          fan_out, dw_ref.ptr, fan_out, acc, db_ref.ptr, acc))
        dx, dw, db = up(hip, dx0), up(hip, dw0), up(hip, db0)
        hip.check(L.lmp_k_linear_backward_f32(batch, fan_in, fan_out, x.ptr, fan_in, w.ptr,
                                              fan_out, g.ptr, fan_out, dx.ptr, fan_in, acc, dw.ptr,
                                              fan_out, acc, db.ptr, acc))
        for got, ref in ((dx, dx_ref), (dw, dw_ref), (db, db_ref)):
            assert np.array_equal(got.numpy().view(np.uint32), ref.numpy().view(np.uint32)), acc
    # the last (accumulating) call against float64 on sampled rows
    rows = rng.choice(fan_in, 48, replace=False)
    want = x_np.T[rows].astype(np.float64) @ g_np.astype(np.float64) + dw0[rows]
    assert rel_err(dw.numpy()[rows], want) <= 1e-5
    xrows = rng.choice(batch, 48, replace=False)
    want = g_np[xrows].astype(np.float64) @ w_np.astype(np.float64).T + dx0[xrows]
    assert rel_err(dx.numpy()[xrows], want) <= 1e-5
    assert rel_err(db.numpy(), g_np.astype(np.float64).sum(0) + db0) <= 1e-5


# Strided B past the one-launch range: the column sums cannot ride in the
# GEMM (B transposed, or K split for few tiles), so they take the strided
# column-sum kernel after it.  (600, 96, 80) is a Linear's weight gradient at
# batch 600 with its output gradient a view of a wider buffer.
@pytest.mark.parametrize("m,n,k,ta,tb,pad", [
    (96, 80, 600, 1, 0, 5), (96, 80, 600, 1, 1, 3), (300, 2100, 4100, 0, 0, 4),
    (64, 1000, 2048, 0, 1, 7), (40, 300, 1000, 1, 1, 1)], ids=str)
def test_gemm_colsum_strided_b(hip, m, n, k, ta, tb, pad):
    L = hip.lib()
    rng = np.random.default_rng(m + 3 * n + 7 * k + pad)
    a_np = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    bst = rng.standard_normal((n, k + pad) if tb else (k, n + pad)).astype(np.float32)
    b = bst[:, :k].T if tb else bst[:, :n]  # op(B) [k, n]
    ldb = bst.shape[1]
    a, db = up(hip, a_np), up(hip, bst)
    lda = m if ta else k
    plain = hip.DeviceBuffer((m, n), np.float32)
    hip.check(L.lmp_k_gemm_f32(ta, tb, m, n, k, a.ptr, lda, db.ptr, ldb, plain.ptr, n, 0))
    c = hip.DeviceBuffer((m, n), np.float32)
    cs = hip.DeviceBuffer((n,), np.float32)
    hip.check(L.lmp_k_gemm_colsum_f32(ta, tb, m, n, k, a.ptr, lda, db.ptr, ldb, c.ptr, n, 0,
                                      cs.ptr, 0))
    assert np.array_equal(c.numpy(), plain.numpy())
    truth = b.astype(np.float64).sum(0)
    sums = cs.numpy()
    assert np.max(np.abs(sums - truth)) <= 1e-5 * max(1.0, np.max(np.abs(truth)))
    aa = a_np.T if ta else a_np
    assert rel_err(c.numpy(), aa.astype(np.float64) @ b.astype(np.float64)) <= 1e-4
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    s0 = rng.standard_normal(n).astype(np.float32)
    dc, dcs = up(hip, c0), up(hip, s0)
    hip.check(L.lmp_k_gemm_colsum_f32(ta, tb, m, n, k, a.ptr, lda, db.ptr, ldb, dc.ptr, n, 1,
                                      dcs.ptr, 1))
    assert np.array_equal(dc.numpy(), c0 + plain.numpy())
    assert np.array_equal(dcs.numpy(), s0 + sums)


@pytest.mark.parametrize("acc", [False, True], ids=["write", "accumulate"])
def test_linear_backward_strided_g_two_launch(hip, acc):
    """Batch 600 (past the one-launch range) with the output gradient a view
    of a wider buffer (ldg > out): lmp_k_linear_backward_f32 gives dX, dW and
    db equal to float64 on the host, and the same bits as the separate calls."""
    L = hip.lib()
    batch, fan_in, fan_out, pad = 600, 96, 80, 5
    rng = np.random.default_rng(600)
    x_np = rng.standard_normal((batch, fan_in)).astype(np.float32)
    w_np = rng.standard_normal((fan_in, fan_out)).astype(np.float32)
    gst = rng.standard_normal((batch, fan_out + pad)).astype(np.float32)
    g_np = gst[:, :fan_out]
    ldg = fan_out + pad
    dx0 = rng.standard_normal((batch, fan_in)).astype(np.float32)
    dw0 = rng.standard_normal((fan_in, fan_out)).astype(np.float32)
    db0 = rng.standard_normal(fan_out).astype(np.float32)
    x, w, g = up(hip, x_np), up(hip, w_np), up(hip, gst)
    dx_ref, dw_ref, db_ref = up(hip, dx0), up(hip, dw0), up(hip, db0)
    hip.check(L.lmp_k_gemm_f32(0, 1, batch, fan_in, fan_out, g.ptr, ldg, w.ptr, fan_out,
                               dx_ref.ptr, fan_in, int(acc)))
    hip.check(L.lmp_k_gemm_colsum_f32(1, 0, fan_in, fan_out, batch, x.ptr, fan_in, g.ptr, ldg,
                                      dw_ref.ptr, fan_out, int(acc), db_ref.ptr, int(acc)))
    dx, dw, db = up(hip, dx0), up(hip, dw0), up(hip, db0)
    hip.check(L.lmp_k_linear_backward_f32(batch, fan_in, fan_out, x.ptr, fan_in, w.ptr, fan_out,
                                          g.ptr, ldg, dx.ptr, fan_in, int(acc), dw.ptr, fan_out,
                                          int(acc), db.ptr, int(acc)))
    for got, ref in ((dx, dx_ref), (dw, dw_ref), (db, db_ref)):
        assert np.array_equal(got.numpy().view(np.uint32), ref.numpy().view(np.uint32))
    g64 = g_np.astype(np.float64)
    base = (lambda t: t) if acc else (lambda t: 0.0)
    assert rel_err(dx.numpy(), g64 @ w_np.astype(np.float64).T + base(dx0)) <= 1e-4
    assert rel_err(dw.numpy(), x_np.astype(np.float64).T @ g64 + base(dw0)) <= 1e-4
    assert rel_err(db.numpy(), g64.sum(0) + base(db0)) <= 1e-5


@pytest.mark.parametrize("m,n,k,ta,ldb_pad", [
    (256, 64, 32, 1, 0), (64, 10, 32, 1, 0), (5, 7, 3, 1, 0), (96, 40, 17, 0, 0),
    (64, 33, 20, 1, 3), (4096, 1000, 512, 1, 0), (300, 260, 600, 1, 4)], ids=str)
@pytest.mark.parametrize("acc", [False, True], ids=["write", "accumulate"])
def test_gemm_colsum_masked_equals_mask_then_colsum(hip, m, n, k, ta, ldb_pad, acc):
    """lmp_k_gemm_colsum_masked_f32 (ReLU's backward applied to B inside the
    column-sum GEMM, or through a scratch buffer for large products) equals
    the clamp-backward kernel followed by lmp_k_gemm_colsum_f32 bit for bit,
    for masks holding NaN, +-0, +-inf, negative and positive values, strided
    B and both A orientations."""
    L = hip.lib()
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    ldb = n + ldb_pad
    a_np = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    g_np = rng.standard_normal((k, ldb)).astype(np.float32)
    h_np = rng.standard_normal((k, ldb)).astype(np.float32)
    specials = np.array([np.nan, 0.0, -0.0, np.inf, -np.inf, 1e-38, -1e-38, 3.0], np.float32)
    h_np.reshape(-1)[: min(h_np.size, 64)] = np.resize(specials, min(h_np.size, 64))
    g_np.reshape(-1)[5::97] = -0.0
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    s0 = rng.standard_normal(n).astype(np.float32)
    a, g, h = up(hip, a_np), up(hip, g_np), up(hip, h_np)
    lda = m if ta else k
    # reference: mask into a contiguous buffer, then the column-sum GEMM
    gm = hip.DeviceBuffer((k, n), np.float32)
    d, _ = hip.make_bcast((k, n), (k, n))
    d.stride_a[0] = d.stride_b[0] = ldb
    hip.check(L.lmp_k_binary(hip.BIN["clamp_backward"], hip.CODE_OF[np.dtype(np.float32)],
                             gm.ptr, h.ptr, g.ptr, C.byref(d), 0.0, 1.7976931348623157e308))
    c_ref, s_ref = up(hip, c0), up(hip, s0)
    hip.check(L.lmp_k_gemm_colsum_f32(ta, 0, m, n, k, a.ptr, lda, gm.ptr, n, c_ref.ptr, n,
                                      int(acc), s_ref.ptr, int(acc)))
    c_got, s_got = up(hip, c0), up(hip, s0)
    hip.check(L.lmp_k_gemm_colsum_masked_f32(ta, m, n, k, a.ptr, lda, g.ptr, h.ptr, ldb,
                                             c_got.ptr, n, int(acc), s_got.ptr, int(acc)))
    assert np.array_equal(c_got.numpy().view(np.uint32), c_ref.numpy().view(np.uint32))
    assert np.array_equal(s_got.numpy().view(np.uint32), s_ref.numpy().view(np.uint32))
    # and the product is the masked one (against float64 on the host)
    gmask = np.where((h_np[:, :n] > 0) & (h_np[:, :n] < np.inf), g_np[:, :n], 0.0)
    aa = a_np.T if ta else a_np
    want = aa.astype(np.float64) @ gmask.astype(np.float64) + (c0 if acc else 0.0)
    assert rel_err(c_got.numpy(), want) <= 1e-5
