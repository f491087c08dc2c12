"""Non-fp32 dtypes on the device: bool, int16, int32, int64 and float64.

Lamp3 instantiates every kernel for all six dtypes and runs its tensor tests
over int16/int32/int64/float32/float64 on each device
(tests/tensor_tests.cpp:760-770), and its stress suites in float64 on the GPU
(tests/stress/pytorch_stress_test.py:57-66).  The checker is the typed
restatement of the CPU kernels (oracle/lamp_typed.py).  Bars: integer and bool
results, float64 add/sub/mul/div/comparisons/neg/abs/sqrt/clamp and float64
max/min bit-exact; float64 transcendentals and pow within 2 ulp; float64
sums/products within 1e-12 under Lamp3's normalised metric; float64 matmul
within 1e-12 (bit-exact on integer-valued inputs, whose partial sums are
exact in any order).
"""
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from _helpers import rel_err  # noqa: E402
from oracle import lamp_typed as T  # noqa: E402

INTS = [np.int16, np.int32, np.int64]
TYPED = [np.bool_, np.int16, np.int32, np.int64, np.float64]
SHAPES = [((7, 9), (7, 9)), ((64, 33), (64, 1)), ((64, 33), (33,)), ((5, 6, 7), (6, 1)),
          ((4, 1, 3), (1, 5, 3)), ((13,), (1,)), ((1000, 257), (1000, 1))]


def up(hip, arr):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(arr))


def ulp64(x, y):
    def key(a):
        i = np.ascontiguousarray(a, np.float64).view(np.int64).astype(object)
        return np.array([(-(2 ** 63) - v) if v < 0 else v for v in i.ravel()], object)
    return np.abs(key(x) - key(y)).astype(np.float64)


def sample(dt, shape, rng, small=False):
    dt = np.dtype(dt)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if dt.kind == "i":
        info = np.iinfo(dt)
        lo, hi = (-50, 50) if small else (info.min, info.max)
        return rng.integers(lo, hi, shape, dtype=dt, endpoint=True)
    return rng.standard_normal(shape) * (3.0 if small else 1e3)


def same(got, want):
    assert got.dtype == want.dtype and got.shape == want.shape
    if got.dtype.kind == "f":
        assert np.array_equal(got.view(np.int64), want.view(np.int64))
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("sa,sb", SHAPES, ids=str)
@pytest.mark.parametrize("dt", TYPED, ids=lambda d: np.dtype(d).name)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt"])
def test_typed_binary_exact(hip, op, dt, sa, sb):
    rng = np.random.default_rng(zlib.crc32(repr((op, np.dtype(dt).name, sa, sb)).encode()))
    a, b = sample(dt, sa, rng), sample(dt, sb, rng)
    if op in ("eq", "ne", "ge", "le") and np.dtype(dt).kind == "f":
        a, b = np.round(a / 300), np.round(b / 300)  # make ties occur
    if op == "div" and np.dtype(dt).kind in "ib":
        # division by zero and INT_MIN / -1 are undefined in the reference
        b = np.where(b == 0, 1, b).astype(dt)
        if np.dtype(dt).kind == "i":
            b = np.where(b == -1, 3, b).astype(dt)
    got = hip.binary(op, up(hip, a), up(hip, b)).numpy()
    same(got, T.binary(op, a, b))


SPECIALS64 = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 3.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324,
                       1e-310, 2.2250738585072014e-308, 1e-160, 1.7e308, -1.7e308,
                       1.0000000000000002, 0.9999999999999999])


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt"])
def test_float64_special_values_exact(hip, op):
    """Every pair of float64 special values (signed zeros, infinities, NaN,
    subnormals down to 5e-324, the extremes, the neighbours of 1) bit for bit
    as the typed oracle; NaN results compare as NaN (x86 and the GPU create
    NaN with different sign bits)."""
    col, row = SPECIALS64.reshape(-1, 1), SPECIALS64.reshape(1, -1)
    got = hip.binary(op, up(hip, col), up(hip, row)).numpy()
    with np.errstate(all="ignore"):
        want = T.binary(op, col, row)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.int64), want[~nan].view(np.int64))


@pytest.mark.parametrize("dt", INTS + [np.bool_], ids=lambda d: np.dtype(d).name)
def test_typed_pow_integers(hip, dt):
    """Integer pow is double pow truncated back: exact on exactly
    representable results."""
    rng = np.random.default_rng(5)
    if dt is np.bool_:
        a, b = sample(dt, (200,), rng), sample(dt, (200,), rng)
    else:
        a = rng.integers(-6, 7, 300).astype(dt)
        # keep |a|^b inside the type (the conversion is undefined past it)
        b = rng.integers(0, 6 if dt is np.int16 else 9, 300).astype(dt)
    same(hip.binary("pow", up(hip, a), up(hip, b)).numpy(), T.binary("pow", a, b))


def test_typed_pow_float64(hip):
    rng = np.random.default_rng(6)
    a = np.abs(rng.standard_normal(4096)) * 10
    b = rng.standard_normal(4096) * 4
    got = hip.binary("pow", up(hip, a), up(hip, b)).numpy()
    assert ulp64(got, T.binary("pow", a, b)).max() <= 2


@pytest.mark.parametrize("dt", TYPED, ids=lambda d: np.dtype(d).name)
def test_typed_unary(hip, dt):
    rng = np.random.default_rng(zlib.crc32(np.dtype(dt).name.encode()))
    x = sample(dt, (4099,), rng, small=True)
    for op in ("neg", "abs"):
        same(hip.unary(op, up(hip, x)).numpy(), T.unary(op, x))
    same(hip.unary("clamp", up(hip, x), -7.0, 20.0).numpy(), T.unary("clamp", x, -7.0, 20.0))
    pos = np.abs(x).astype(dt) if np.dtype(dt) != np.bool_ else x
    same(hip.unary("sqrt", up(hip, pos)).numpy(), T.unary("sqrt", pos))
    ops = ("exp", "log", "sin", "cos", "tan")
    for op in ops:
        src = pos if op == "log" else x
        if op == "log" and np.dtype(dt).kind in "ib":
            src = np.where(src == 0, 1, src).astype(dt)  # log(0) -> -inf is out of int range
        if op == "exp" and np.dtype(dt).kind == "i":
            # keep exp(x) inside the integer range (conversion is undefined past it)
            src = np.clip(src, -20, 10 if dt is np.int16 else 20).astype(dt)
        got = hip.unary(op, up(hip, src)).numpy()
        want = T.unary(op, src)
        if np.dtype(dt).kind == "f":
            assert ulp64(got, want).max() <= 2, op
        else:
            same(got, want)


@pytest.mark.parametrize("shape,axis", [((300, 257), 0), ((300, 257), 1), ((4, 37, 5), 1),
                                        ((64, 16384), 1), ((2048, 1024), 0), ((1, 1), 0),
                                        ((5, 3000, 12), 1), ((3, 0, 4), 1)], ids=str)
@pytest.mark.parametrize("dt", TYPED, ids=lambda d: np.dtype(d).name)
def test_typed_reduce(hip, dt, shape, axis):
    rng = np.random.default_rng(zlib.crc32(repr((np.dtype(dt).name, shape, axis)).encode()))
    x = sample(dt, shape, rng)
    d = up(hip, x)
    for op in ("sum", "max", "min", "prod"):
        src, dsrc = x, d
        if op == "prod" and np.dtype(dt) == np.float64:
            src = 1.0 + 1e-4 * rng.standard_normal(shape)  # keep products finite
            dsrc = up(hip, src)
        got = hip.reduce(op, dsrc, axis).numpy()
        want = T.reduce(op, src, axis)
        if np.dtype(dt) == np.float64 and op in ("sum", "prod"):
            assert got.shape == want.shape
            assert rel_err(got, want) <= 1e-12, op
        else:
            same(got, want)


GEMM_SHAPES = [(64, 64, 64), (33, 17, 70), (128, 256, 96), (1, 7, 3), (130, 260, 33),
               (200, 3, 5), (256, 1000, 128)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES, ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("dt", TYPED, ids=lambda d: np.dtype(d).name)
def test_typed_gemm(hip, dt, m, n, k, ta, tb):
    rng = np.random.default_rng(m * 7 + n * 3 + k + ta * 2 + tb)
    a, b = sample(dt, (m, k), rng), sample(dt, (k, n), rng)
    if np.dtype(dt) == np.float64:
        a, b = np.round(a / 100), np.round(b / 100)  # integer-valued: exact in any order
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    want = T.matmul(a, b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    same(got, want)
    c0 = sample(dt, (m, n), rng)
    if np.dtype(dt) == np.float64:
        c0 = np.round(c0)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    same(dc.numpy(), T.binary("add", c0, want))


def test_gemm_float64_random_and_large(hip):
    """Random float64 operands at 1024^3 in all orientations, within 1e-12
    of numpy's float64 product."""
    rng = np.random.default_rng(11)
    a = rng.standard_normal((1024, 1024))
    b = rng.standard_normal((1024, 1024))
    for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
        got = hip.gemm(up(hip, a), up(hip, b), trans_a=bool(ta), trans_b=bool(tb)).numpy()
        want = (a.T if ta else a) @ (b.T if tb else b)
        assert rel_err(got, want) <= 1e-12, (ta, tb)


# float64 products whose 128 x 128 tiles cover the CUs run on the large-tile
# kernel: ragged edges, short and odd K, every orientation, accumulate;
# integer-valued operands exact, random ones within 1e-12 of numpy.
@pytest.mark.parametrize("m,n,k", [(2048, 2048, 256), (2100, 2060, 37), (4100, 1030, 130)],
                         ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_float64_large_tiles(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(m + 3 * n + 7 * k + 11 * ta + 13 * tb)
    a = np.round(rng.standard_normal((m, k)) * 100)
    b = np.round(rng.standard_normal((k, n)) * 100)
    da = up(hip, a.T.copy() if ta else a)
    db = up(hip, b.T.copy() if tb else b)
    got = hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got, a @ b)  # integer products and sums below 2^53: exact
    c0 = np.round(rng.standard_normal((m, n)) * 100)
    dc = up(hip, c0)
    hip.gemm(da, db, trans_a=bool(ta), trans_b=bool(tb), out=dc, accumulate=True)
    assert np.array_equal(dc.numpy(), c0 + a @ b)
    ar, br = rng.standard_normal((m, k)), rng.standard_normal((k, n))
    got = hip.gemm(up(hip, ar.T.copy() if ta else ar), up(hip, br.T.copy() if tb else br),
                   trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert rel_err(got, ar @ br) <= 1e-12


def _up_offset(hip, arr):
    """arr stored one double past a 16-byte boundary, rows padded by one
    element: returns (buffer, address of element [0, 0], leading dimension)."""
    rows, cols = arr.shape
    flat = np.zeros(1 + rows * (cols + 1), np.float64)
    flat[1:].reshape(rows, cols + 1)[:, :cols] = arr
    buf = up(hip, flat)
    return buf, buf.ptr + 8, cols + 1


# Both float64 kernels (128 x 128 tiles once those cover the CUs, 64 x 64
# below) load 16-byte pairs without bounds checks for tiles inside C when both
# operands are 16-byte aligned with even leading dimensions, and checked pairs
# otherwise.  Both fill the same LDS tile, so the same random product through
# operands one double off alignment with odd leading dimensions gives the same
# bits.
@pytest.mark.parametrize("m,n,k", [(2048, 2048, 200), (2180, 1990, 96), (1000, 1030, 96),
                                   (200, 130, 50)], ids=str)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_float64_large_tiles_unaligned_same_bits(hip, m, n, k, ta, tb):
    rng = np.random.default_rng(5 * m + n + 3 * k + 17 * ta + 19 * tb)
    a, b = rng.standard_normal((m, k)), rng.standard_normal((k, n))
    sa, sb = (a.T.copy() if ta else a), (b.T.copy() if tb else b)
    got = hip.gemm(up(hip, sa), up(hip, sb), trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert rel_err(got, a @ b) <= 1e-12
    (ba, pa, lda), (bb, pb, ldb) = _up_offset(hip, sa), _up_offset(hip, sb)
    out = hip.DeviceBuffer((m, n), np.float64)
    hip.check(hip.lib().lmp_k_gemm(out.code, ta, tb, m, n, k, pa, lda, pb, ldb, out.ptr, n, 0))
    assert np.array_equal(out.numpy().view(np.int64), got.view(np.int64))


# ------------------------------------------------- framework level

@pytest.fixture(scope="module")
def rsl(hip):
    import rushlite_amd
    return rushlite_amd


def test_mixed_dtype_promotion(rsl):
    """Operands are cast to the promoted dtype, then the op runs in it."""
    i = rsl.Variable(np.array([[16777217, -3]], np.int32), dtype=rsl.dtype.int32)
    f = rsl.Variable(np.array([[0.0, 0.5]], np.float32))
    d = rsl.Variable(np.array([[0.25, 0.5]], np.float64), dtype=rsl.dtype.float64)
    r = i + f
    assert r.dtype == rsl.dtype.float32
    assert r.numpy().tolist() == [[16777216.0, -2.5]]
    r2 = f * d
    assert r2.dtype == rsl.dtype.float64 and r2.numpy().tolist() == [[0.0, 0.25]]
    m = rsl.matmul(i, rsl.Variable(np.array([[2], [1]], np.int16), dtype=rsl.dtype.int16))
    assert m.dtype == rsl.dtype.int32 and m.numpy().tolist() == [[33554431]]


def test_float64_autograd_matches_torch(rsl):
    """A float64 graph through every autograd formula, with a Linear-style
    matmul, against torch float64 autograd (the reference's own stress
    oracle, pytorch_stress_test.py:92-110)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(12)
    x0 = rng.standard_normal((16, 24))
    w0 = rng.standard_normal((24, 8)) * 0.3
    b0 = rng.standard_normal((8,)) * 0.1
    f64 = rsl.dtype.float64
    x = rsl.Variable(x0, requires_grad=True, dtype=f64)
    w = rsl.Variable(w0, requires_grad=True, dtype=f64)
    b = rsl.Variable(b0, requires_grad=True, dtype=f64)
    h = rsl.clamp(rsl.matmul(x, w) + b, 0.0, 1e300)
    s = rsl.exp(rsl.sin(h)) / (rsl.sqrt(h * h + 1.0)) - rsl.log(h + 2.0) * h
    loss = rsl.sum(rsl.sum(s * s, 1), 0)
    loss.backward()
    tx = torch.tensor(x0, dtype=torch.float64, requires_grad=True)
    tw = torch.tensor(w0, dtype=torch.float64, requires_grad=True)
    tb = torch.tensor(b0, dtype=torch.float64, requires_grad=True)
    th = torch.clamp(tx @ tw + tb, 0.0, 1e300)
    ts = torch.exp(torch.sin(th)) / torch.sqrt(th * th + 1.0) - torch.log(th + 2.0) * th
    tl = (ts * ts).sum()
    tl.backward()
    assert loss.dtype == f64
    assert abs(loss.numpy().item() - tl.item()) <= 1e-12 * abs(tl.item())
    for mine, ref in ((x, tx), (w, tw), (b, tb)):
        assert rel_err(mine.grad.numpy(), ref.grad.numpy()) <= 1e-12


@pytest.mark.parametrize("dt", ["int16", "int32", "int64", "float32", "float64"])
def test_known_answer_ops_per_reference_dtype(rsl, dt):
    """tensor_tests.cpp's broadcast, pow and comparison known answers for
    every dtype its TensorOpTest runs (tensor_tests.cpp:760-770); inputs are
    made from floats with the dtype's conversion, as Tensor(vector<float>,
    ..., dtype) does."""
    kind = getattr(rsl.dtype, dt)
    A = [[1, 2], [3, 4], [5, 6]]
    V = lambda v: rsl.Variable(np.array(v, np.float64), dtype=kind)  # noqa: E731
    check = lambda out, want: np.testing.assert_allclose(  # noqa: E731
        out.numpy().reshape(-1).astype(np.float64), want, atol=1e-5, rtol=0)
    check(V(A) + V([100.0]), [101, 102, 103, 104, 105, 106])      # :100-113
    check(V(A) + V([[10, 20]]), [11, 22, 13, 24, 15, 26])          # :115-127
    check(V(A) + V([[10], [20], [30]]), [11, 12, 23, 24, 35, 36])  # :129-141
    check(rsl.pow(V(A), V([2.0])), [1, 4, 9, 16, 25, 36])          # :554-579
    check(rsl.pow(V(A), V([[0, 0], [0, 0], [0, 0]])), [1] * 6)     # :596-613
    B = [[0.5, 1.5], [2.5, 3.5], [4.5, 5.5]]
    check(V(A) != V(B), [1] * 6)                                   # :629-638
    check(V(A) < V(B), [0] * 6)                                    # :640-649
    check(V(A) > V(B), [1] * 6)                                    # :651-660
    check(V(A) >= V(A), [1] * 6)                                   # :676-687
    check(V(A) < V([[10], [20], [30]]), [1] * 6)                   # :743-752
    if dt.startswith("int"):
        check(rsl.pow(V(A), V([[2.0, 3.0]])), [1, 8, 9, 64, 25, 216])       # :704-716
        check(rsl.pow(V(A), V([[1, 2], [1, 2], [1, 2]])), [1, 4, 3, 16, 5, 36])  # :519-532
    else:
        check(rsl.pow(V(A), V([[10, 20]]) / 10), [1, 4, 3, 16, 5, 36])    # :717-727
    check(rsl.sum(V(A), 0), [9, 12])                               # :196-212
    check(rsl.sum(V(A), 1), [3, 7, 11])                            # :213-224


def test_float64_capture_fuses_one_kernel_equal_to_eager(rsl):
    """A captured float64 chain with [M,1] broadcasts becomes one hipRTC
    kernel, bit-identical to the eager float64 kernels, and within 1e-14 of the
    typed oracle under the normalised metric (exp is the only step that may
    differ, by an ulp, and the subtraction can cancel, so ulps of the result
    are not the measure)."""
    rng = np.random.default_rng(21)
    a_np, b_np = rng.standard_normal((257, 64)), rng.standard_normal((257, 1))
    f64 = rsl.dtype.float64
    a, b = rsl.Variable(a_np, dtype=f64), rsl.Variable(b_np, dtype=f64)
    big = 1.7976931348623157e308

    def chain():
        return rsl.exp(a) * b - rsl.clamp(a, 0.0, big) / (b + 1.0)

    s0 = rsl._stats()
    with rsl.capture_on():
        c = chain()
        assert rsl._is_deferred(c)
        src = rsl._fused_source(c)
    got = c.numpy()
    s1 = rsl._stats()
    assert s1["fused_launches"] - s0["fused_launches"] == 1
    assert "double" in src and "expf" not in src
    eager = chain().numpy()
    assert got.dtype == np.float64
    assert np.array_equal(got.view(np.int64), eager.view(np.int64))
    want = T.binary("sub", T.binary("mul", T.unary("exp", a_np), b_np),
                    T.binary("div", T.unary("clamp", a_np, 0.0, big),
                             T.binary("add", b_np, np.array([1.0]))))
    assert rel_err(got, want) <= 1e-14


def test_mixed_dtype_chain_under_capture_stays_correct(rsl):
    """Nodes whose operands have different dtypes are not fused; capture must
    still give the eager result (cast-then-operate)."""
    i = rsl.Variable(np.arange(12, dtype=np.int32).reshape(3, 4), dtype=rsl.dtype.int32)
    f = rsl.Variable(np.full((3, 1), 0.5, np.float32))
    with rsl.capture_on():
        c = (i * 3) + f
    eager = ((i * 3) + f).numpy()
    got = c.numpy()
    assert got.dtype == np.float32 and np.array_equal(got, eager)
    assert got.tolist() == (np.arange(12).reshape(3, 4) * 3 + 0.5).tolist()
