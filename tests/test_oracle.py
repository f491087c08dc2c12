"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something that does not share its
code: the reference gtests' known answers (tests/golden), numpy's IEEE float32
ops (one rounding per op, bit-exact), correctly rounded values (float64
evaluation rounded to float32) for transcendentals, brute-force sequential
folds in pure Python for the reduction / matmul order, float64 numpy for sums
and products, and torch float64 autograd for the gradient formulas.
"""
import json
import math
import subprocess
import sys
import zlib
from pathlib import Path

import numpy as np
import pytest

from _helpers import assert_within_ulp, ulp_dist, zero_sign_mismatches

GOLDEN = json.loads((Path(__file__).parent / "golden" / "lamp3_known_answers.json").read_text())
ATOL = GOLDEN["tolerance"]["atol"]


def _num(v):
    return float(v) if not isinstance(v, str) else float(v.replace("inf", "inf"))


def correctly_rounded(fn, *args):
    return fn(*[np.asarray(a, np.float64) for a in args]).astype(np.float32)


# ------------------------------------------------------- timing (fast) builds


def _fast_builds(oracle):
    """Paths of the fast builds this host can run: x86-64-v3 always, the
    AVX-512 one where the CPU has its flags."""
    names = ["liblamp_cpu_fast.so"]
    if oracle.host_isa() == "x86-64-v4":
        names.append("liblamp_cpu_fast_v4.so")
    return [oracle.HERE / n for n in names]


def test_fast_builds_leave_the_process_denormal_mode_alone(oracle):
    """Loading a -ffast-math build must not switch the process to
    flush-to-zero (gcc's fast-math startup code would: numpy's 1e-40 * 2
    would become 0 for the rest of the process)."""
    import ctypes
    for path in _fast_builds(oracle):
        ctypes.CDLL(str(path))
        assert np.float32(1e-40) * np.float32(2) != 0, path.name


def test_denormal_flush_is_scoped(oracle):
    x = np.array([1e-40, 3.0], np.float32)
    two = np.array([2.0], np.float32)
    with oracle.denormal_flush():
        assert oracle.binary("mul", x, two, fast=True)[0] == 0  # flushed
    assert oracle.binary("mul", x, two, fast=True)[0] == np.float32(1e-40) * np.float32(2)
    assert np.float32(1e-40) * np.float32(2) != 0


def test_fast_builds_agree_with_the_strict_build():
    """Both ISA levels of the timed build compute what the parity build does:
    single IEEE operations bit for bit, sums to the reductions' 1e-5."""
    import ctypes
    from oracle import lamp_oracle as O
    rng = np.random.default_rng(7)
    a = rng.standard_normal(100003).astype(np.float32)
    b = rng.standard_normal(100003).astype(np.float32)
    want_mul = O.binary("mul", a, b, fast=False)
    want_sum = O.reduce("sum", a.reshape(1, -1), 1, fast=False)
    for path in _fast_builds(O):
        lib = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        lib.lcpu_binary_f32.argtypes = [ctypes.c_int, P, P, P, ctypes.c_int, P, P, P,
                                        ctypes.c_int, ctypes.c_double, ctypes.c_double]
        lib.lcpu_reduce_f32.argtypes = [ctypes.c_int, P, P, ctypes.c_int, P, ctypes.c_int]
        out = np.empty_like(a)
        shape = np.array([a.size], np.int64)
        strides = np.array([1], np.int64)
        lib.lcpu_binary_f32(O.BIN["mul"], out.ctypes.data, a.ctypes.data, b.ctypes.data, 1,
                            shape.ctypes.data, strides.ctypes.data, strides.ctypes.data, 0,
                            0.0, 0.0)
        assert np.array_equal(out, want_mul), path.name
        red = np.empty((1, 1), np.float32)
        shp2 = np.array([1, a.size], np.int64)
        lib.lcpu_reduce_f32(O.RED["sum"], red.ctypes.data, a.ctypes.data, 2, shp2.ctypes.data, 1)
        assert abs(float(red[0, 0]) - float(want_sum[0, 0])) <= 1e-5 * np.abs(a).sum(), path.name


# ------------------------------------------------------------ golden vectors


def test_known_answer_fixture_matches_its_transcription():
    """tests/golden/lamp3_known_answers.json is exactly what the committed
    transcription script writes."""
    script = Path(__file__).parent / "golden" / "make_known_answers.py"
    assert subprocess.run([sys.executable, str(script), "--check"]).returncode == 0


@pytest.mark.parametrize("case", GOLDEN["tensor"], ids=lambda c: c["name"])
def test_known_answers_binary(oracle, case):
    out = oracle.binary(case["op"], np.array(case["a"], np.float32),
                        np.array(case["b"], np.float32))
    assert list(out.shape) == case["shape"]
    np.testing.assert_allclose(out.reshape(-1), np.array(case["expect"], np.float64),
                               atol=case.get("atol", ATOL), rtol=0)


@pytest.mark.parametrize("case", GOLDEN["reduce"], ids=lambda c: c["name"])
def test_known_answers_reduce(oracle, case):
    out = oracle.reduce(case["op"], np.array(case["a"], np.float32), case["axis"])
    assert list(out.shape) == case["shape"]
    np.testing.assert_allclose(out.reshape(-1), case["expect"], atol=ATOL, rtol=0)


def _close(got, want):
    want = np.array([_num(v) for v in want], np.float64)
    got = np.asarray(got, np.float64).reshape(-1)
    fin = np.isfinite(want)
    assert np.array_equal(np.isinf(got), np.isinf(want))
    assert np.array_equal(np.sign(got[~fin]), np.sign(want[~fin]))
    np.testing.assert_allclose(got[fin], want[fin], atol=ATOL, rtol=0)


@pytest.mark.parametrize("case", GOLDEN["autograd"], ids=lambda c: c["name"])
def test_known_answers_autograd(oracle, case):
    O = oracle
    a = O.OVar(np.array(GOLDEN["inputs"]["a"], np.float32), True)
    b = O.OVar(np.array(GOLDEN["inputs"]["b"], np.float32), True)
    extra = {}
    e = case["expr"]
    if e == "a + b": out = a + b
    elif e == "a - b": out = a - b
    elif e == "a * b": out = a * b
    elif e == "a / b":
        with np.errstate(divide="ignore", invalid="ignore"):
            out = a / b
    elif e == "exp(b)": out = O.exp(b)
    elif e == "log(a)": out = O.log(a)
    elif e == "a @ m":
        extra["m"] = O.OVar(np.array(case["m"], np.float32), True)
        out = a @ extra["m"]
    elif e == "transpose(a)": out = O.transpose_v(a)
    elif e == "sum(a, 1)": out = O.sum_(a, 1)
    elif e == "max(a, 1)": out = O.max_(a, 1)
    elif e == "min(a, 1)": out = O.min_(a, 1)
    elif e == "a + r":
        extra["r"] = O.OVar(np.array(case["r"], np.float32), True)
        out = a + extra["r"]
    else:
        raise AssertionError(e)
    _close(out.data, case["out"])
    out.backward()
    if "grad_a" in case: _close(a.grad, case["grad_a"])
    if "grad_b" in case: _close(b.grad, case["grad_b"])
    if "grad_m" in case: _close(extra["m"].grad, case["grad_m"])
    if "grad_r" in case:
        _close(extra["r"].grad, case["grad_r"])
        assert extra["r"].grad.shape == (1, 2)


@pytest.mark.parametrize("case", GOLDEN["autograd_unary"], ids=lambda c: c["name"])
def test_known_answers_unary_grads(oracle, case):
    O = oracle
    x = O.OVar(np.array(case["x"], np.float32), True)
    fn = case["fn"]
    out = {"sqrt": O.sqrt, "cos": O.cos, "tan": O.tan, "abs": O.abs_}.get(fn)
    out = out(x) if out else O.clamp(x, case["lo"], case["hi"])
    out.backward()
    _close(x.grad, case["grad"])


def test_repeated_backward_accumulates(oracle):
    a = oracle.OVar(np.array(GOLDEN["inputs"]["a"], np.float32), True)
    r = a * 2.0
    r.backward()
    r.backward()
    _close(a.grad, GOLDEN["repeated_backward"]["grad_a"])


def test_functional_sgd(oracle):
    g = GOLDEN["functional_sgd"]
    w = oracle.OVar(np.array(g["w"], np.float32), True)
    x, y = oracle.OVar(np.array(g["x"], np.float32)), oracle.OVar(np.array(g["y"], np.float32))
    err = x * w - y
    (oracle.sum_(err * err, 0)).backward()
    new = w.data - np.float32(g["lr"]) * w.grad
    np.testing.assert_allclose(new, g["expect"], rtol=1e-6)


# ------------------------------------------------- independent closed forms

SHAPES = [((7, 9), (7, 9)), ((64, 33), (64, 1)), ((64, 33), (33,)),
          ((64, 33), (1, 33)), ((5, 6, 7), (6, 1)), ((4, 1, 3), (1, 5, 3)),
          ((13,), (1,)), ((2, 3, 4, 5), (3, 1, 5))]


@pytest.mark.parametrize("op,npf", [("add", np.add), ("sub", np.subtract),
                                    ("mul", np.multiply), ("div", np.divide)])
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_bitexact_vs_numpy(oracle, op, npf, sa, sb):
    rng = np.random.default_rng(zlib.crc32(repr((op, sa, sb)).encode()))
    a = rng.standard_normal(sa, dtype=np.float32)
    b = rng.standard_normal(sb, dtype=np.float32) + np.float32(3.0)
    got = oracle.binary(op, a, b)
    want = npf(a, b)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got_r = oracle.binary(op, b, a)  # reversed operand order
    assert np.array_equal(got_r.view(np.uint32), npf(b, a).view(np.uint32))


@pytest.mark.parametrize("op,npf", [("eq", np.equal), ("ne", np.not_equal),
                                    ("ge", np.greater_equal), ("le", np.less_equal),
                                    ("gt", np.greater), ("lt", np.less)])
def test_compare_vs_numpy(oracle, op, npf):
    rng = np.random.default_rng(3)
    a = rng.integers(-3, 4, (40, 17)).astype(np.float32)
    b = rng.integers(-3, 4, (1, 17)).astype(np.float32)
    got = oracle.binary(op, a, b)
    assert np.array_equal(got, npf(a, b).astype(np.float32))


def test_unary_exact_ops(oracle):
    x = np.array([-2.5, -0.0, 0.0, 1.5, np.inf, -np.inf, np.nan, 1e-40, -3e38],
                 np.float32)
    assert np.array_equal(oracle.unary("neg", x).view(np.uint32), (-x).view(np.uint32))
    assert np.array_equal(oracle.unary("abs", x).view(np.uint32),
                          np.abs(x).view(np.uint32))
    pos = np.abs(x[np.isfinite(x)])
    assert np.array_equal(oracle.unary("sqrt", pos), np.sqrt(pos))
    # ReLU = clamp(x, 0, DBL_MAX): -0.0 stays -0.0, NaN stays NaN, +inf stays.
    r = oracle.unary("clamp", x, 0.0, oracle.DBL_MAX)
    want = np.where(x < 0, np.float32(0), x)
    assert np.array_equal(r.view(np.uint32), want.view(np.uint32))
    assert np.signbit(r[1]) and np.isnan(r[6])


@pytest.mark.parametrize("op,fn", [("exp", np.exp), ("log", np.log), ("sin", np.sin),
                                   ("cos", np.cos), ("tan", np.tan)])
def test_transcendentals_within_1ulp_of_correctly_rounded(oracle, op, fn):
    rng = np.random.default_rng(11)
    x = rng.uniform(-20, 20, 20000).astype(np.float32)
    if op == "log":
        x = np.abs(x) + np.float32(1e-3)
    got = oracle.unary(op, x)
    assert_within_ulp(got, correctly_rounded(fn, x), 1, op)


def test_pow_within_1ulp(oracle):
    rng = np.random.default_rng(5)
    a = rng.uniform(0.01, 10, 5000).astype(np.float32)
    b = rng.uniform(-4, 4, 5000).astype(np.float32)
    got = oracle.binary("pow", a, b)
    assert_within_ulp(got, correctly_rounded(np.power, a, b), 1)


def test_ulp_helpers_see_the_sign_of_zero():
    """-0.0 and +0.0 are adjacent but distinct on the ulp line, distances are
    monotone across zero, and a zero of the wrong sign is reported even though
    it is only one ulp away."""
    d = np.float32(1e-45)  # the smallest subnormal
    assert ulp_dist(np.float32(-0.0), np.float32(0.0)) == 1
    assert ulp_dist(-d, d) == 3
    assert ulp_dist(np.float32(-1.0), np.float32(1.0)) == 2 * 0x3F800000 + 1
    xs = np.sort(np.random.default_rng(3).standard_normal(4001).astype(np.float32))
    xs = np.concatenate([xs[xs < 0], [np.float32(-0.0), np.float32(0.0)], xs[xs > 0]])
    keys = ulp_dist(xs, np.full_like(xs, -np.inf))
    assert np.all(np.diff(keys) > 0)  # strictly increasing distance from -inf
    want = np.array([0.0, -0.0, 1.0, -0.0], np.float32)
    assert zero_sign_mismatches(want, want) == 0
    assert zero_sign_mismatches(np.array([0.0, 0.0, 1.0, -0.0], np.float32), want) == 1
    assert zero_sign_mismatches(np.array([0.0, -1e-45, 1.0, -0.0], np.float32), want) == 1
    with pytest.raises(AssertionError):
        assert_within_ulp(np.array([0.0, 0.0], np.float32),
                          np.array([0.0, -0.0], np.float32), 2)


def _tree_sum_f32(v):
    """A 64-lane strided then butterfly float32 sum (another valid order)."""
    lanes = np.zeros(64, np.float32)
    for j in range(0, len(v), 64):
        chunk = np.zeros(64, np.float32)
        chunk[:len(v) - j] = v[j:j + 64]
        lanes = (lanes + chunk).astype(np.float32)
    for s in (1, 2, 4, 8, 16, 32):
        lanes = (lanes + lanes[np.arange(64) ^ s]).astype(np.float32)
    return lanes[:1]


def _seq_sum_f32(v):
    acc = np.float32(0.0)
    for x in v:
        acc = np.float32(acc + x)
    return np.array([acc], np.float32)


@pytest.mark.parametrize("n", [1995, 2506, 4096])
def test_sum_bound_accepts_other_orders_and_catches_term_errors(n):
    """assert_sum_close (the GPU sum tests' bound) accepts a tree-order float32
    sum against the sequential one, cancelling or not (the 1995- and 2506-term
    vectors are the cancelling sums of test_reduce), and rejects a sum that
    dropped or doubled one typical term."""
    from _helpers import assert_sum_close
    a = np.random.default_rng(zlib.crc32(repr(((n,), 0)).encode())).standard_normal(
        n, dtype=np.float32)
    want, got = _seq_sum_f32(a), _tree_sum_f32(a)
    assert_sum_close(got, want, a, 0)
    j = int(np.argsort(np.abs(a))[n // 2])  # a term of median size
    for bad in (got - a[j], got + a[j]):
        with pytest.raises(AssertionError):
            assert_sum_close(bad.astype(np.float32), want, a, 0)


@pytest.mark.parametrize("op,fn,x,want", [
    ("sin", math.sin, -0.0, -0.0), ("sin", math.sin, 0.0, 0.0),
    ("tan", math.tan, -0.0, -0.0), ("tan", math.tan, 0.0, 0.0),
    ("sqrt", math.sqrt, -0.0, -0.0), ("exp", math.exp, -0.0, 1.0),
    ("cos", math.cos, -0.0, 1.0), ("neg", lambda v: -v, 0.0, -0.0),
    ("abs", abs, -0.0, 0.0)])
def test_oracle_signed_zero_results(oracle, op, fn, x, want):
    """std::sin/tan/sqrt keep the sign of a zero argument (C99 Annex F), the
    functors of cpu/kernels.hpp:74-113 return them unchanged; Python's math
    module states the same values."""
    got = oracle.unary(op, np.array([x], np.float32))
    assert np.array_equal(got.view(np.uint32), np.array([want], np.float32).view(np.uint32))
    assert math.copysign(1.0, fn(x)) == math.copysign(1.0, want)


def test_gemm_orders_are_valid_and_distinct(oracle):
    """Every GEMM order used to size the README-MLP loss envelope is within the
    1e-4 GEMM bar of the float64 product, and the orders really differ (each
    pair disagrees in some bit on a product with K = 256)."""
    rng = np.random.default_rng(12)
    a = rng.standard_normal((64, 256)).astype(np.float32)
    b = rng.standard_normal((256, 48)).astype(np.float32)
    truth = a.astype(np.float64) @ b.astype(np.float64)
    outs = {}
    for name, mm in oracle.GEMM_ORDERS.items():
        got = mm(a, b)
        assert got.dtype == np.float32 and got.shape == (64, 48)
        assert np.max(np.abs(got - truth)) / np.max(np.abs(truth)) <= 1e-4, name
        outs[name] = got
    assert np.array_equal(outs["seq"], oracle.matmul(a, b))
    names = list(outs)
    for i, p in enumerate(names):
        for q in names[i + 1:]:
            assert not np.array_equal(outs[p], outs[q]), (p, q)


def test_reduction_order_is_sequential(oracle):
    """The oracle folds each output in index order from the identity: compare
    with a pure-Python float32 fold (small case, bit-exact)."""
    rng = np.random.default_rng(1)
    a = rng.standard_normal((4, 37, 5), dtype=np.float32)
    for axis in range(3):
        got = oracle.reduce("sum", a, axis)
        moved = np.moveaxis(a, axis, -1)
        want = np.zeros(moved.shape[:-1], np.float32)
        for idx in np.ndindex(*moved.shape[:-1]):
            acc = np.float32(0)
            for v in moved[idx]:
                acc = np.float32(acc + v)
            want[idx] = acc
        assert np.array_equal(got.reshape(-1), np.expand_dims(want, axis).reshape(-1))


@pytest.mark.parametrize("axis", [0, 1])
def test_reduce_vs_numpy(oracle, axis):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((300, 257), dtype=np.float32)
    for op, fn in (("max", np.max), ("min", np.min)):
        assert np.array_equal(oracle.reduce(op, a, axis), fn(a, axis=axis, keepdims=True))
    s = oracle.reduce("sum", a, axis).astype(np.float64)
    t = a.astype(np.float64).sum(axis=axis, keepdims=True)
    assert np.max(np.abs(s - t)) / np.max(np.abs(t)) < 1e-5
    p = oracle.reduce("prod", (a[:8] * 0.5 + 1).astype(np.float32), axis)
    tp = np.prod((a[:8] * 0.5 + 1).astype(np.float64), axis=axis, keepdims=True)
    np.testing.assert_allclose(p, tp, rtol=1e-5)


EMPTY_AXIS_CASES = [((3, 0, 2), 1), ((0, 4), 0), ((4, 0), 1), ((0,), 0), ((2, 0, 0), 1)]


@pytest.mark.parametrize("shape,axis", EMPTY_AXIS_CASES, ids=str)
def test_reduce_empty_axis_gives_identity(oracle, shape, axis):
    """cpu/reduct.cpp:14-19 folds nothing into OpFn::kIdentity and writes it to
    each of out().numel() outputs (reduct.cpp:45-46): 0, lowest(), max(), 1.
    Every output is checked, so an unwritten (garbage) output fails."""
    f32 = np.finfo(np.float32)
    oshape = list(shape)
    oshape[axis] = 1
    for op, ident in (("sum", 0.0), ("max", -f32.max), ("min", f32.max), ("prod", 1.0)):
        got = oracle.reduce(op, np.zeros(shape, np.float32), axis)
        assert got.shape == tuple(oshape)
        assert np.array_equal(got, np.full(oshape, ident, np.float32)), op
        assert not np.signbit(got).any() or op == "max", op


def test_matmul_order_and_value(oracle):
    rng = np.random.default_rng(4)
    a = rng.standard_normal((5, 11), dtype=np.float32)
    b = rng.standard_normal((11, 3), dtype=np.float32)
    got = oracle.matmul(a, b)
    want = np.zeros((5, 3), np.float32)
    for i in range(5):
        for j in range(3):
            s = np.float32(0)
            for t in range(11):
                s = np.float32(s + np.float32(a[i, t] * b[t, j]))
            want[i, j] = s
    assert np.array_equal(got, want)
    a = rng.standard_normal((64, 300), dtype=np.float32)
    b = rng.standard_normal((300, 40), dtype=np.float32)
    t = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(oracle.matmul(a, b) - t)) / np.max(np.abs(t)) < 1e-5


def test_transpose_fill_add_inplace(oracle):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(oracle.transpose(a), a.T)
    f = oracle.fill((3, 5), 2.5)
    assert np.array_equal(f, np.full((3, 5), 2.5, np.float32))
    d = a.copy()
    oracle.add_inplace(d, a)
    assert np.array_equal(d, a + a)


def test_planted_stride_mistake_is_caught(oracle):
    """Sensitivity check: transposing the broadcast operand's padded strides
    (a plausible indexing bug) must break agreement with numpy."""
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.arange(4, dtype=np.float32).reshape(1, 4)
    good = oracle.binary("add", a, b)
    assert np.array_equal(good, a + b)
    orig = oracle.padded_strides
    try:
        oracle.padded_strides = lambda s, nd: list(reversed(orig(s, nd)))
        bad = oracle.binary("add", a, b)
    finally:
        oracle.padded_strides = orig
    assert not np.array_equal(bad, a + b)


# ----------------------------------------------- autograd vs torch float64

torch = pytest.importorskip("torch")


def _torch_softmax_lamp(x, dim):
    # Lamp3's softmax graph: max with an eq-mask gradient (reduct_ops.cpp:14),
    # so torch must rebuild it from primitives rather than use torch.softmax.
    m = x.max(dim=dim, keepdim=True).values
    mask_src = x.detach()
    class LampMax(torch.autograd.Function):
        @staticmethod
        def forward(ctx, inp):
            out = inp.max(dim=dim, keepdim=True).values
            ctx.save_for_backward(inp, out)
            return out
        @staticmethod
        def backward(ctx, g):
            inp, out = ctx.saved_tensors
            return g * (inp == out).to(g.dtype)
    m = LampMax.apply(x)
    e = torch.exp(x - m)
    return e / e.sum(dim=dim, keepdim=True)


def test_autograd_graph_vs_torch(oracle):
    rng = np.random.default_rng(7)
    x0 = rng.uniform(0.5, 2.0, (6, 5)).astype(np.float32)
    w0 = rng.standard_normal((5, 4), dtype=np.float32)
    b0 = rng.standard_normal((4,), dtype=np.float32)
    O = oracle
    x, w, b = O.OVar(x0, True), O.OVar(w0, True), O.OVar(b0, True)
    h = O.relu(x @ w + b)
    s = O.softmax(O.sqrt(O.exp(O.sin(h)) * 2.0) / (O.log(x @ w * 0.1 + 3.0) + 1.0), -1)
    loss = O.sum_(O.sum_(s * O.tan(O.cos(h) * 0.5), 1), 0)
    loss.backward()

    tx = torch.tensor(x0, dtype=torch.float64, requires_grad=True)
    tw = torch.tensor(w0, dtype=torch.float64, requires_grad=True)
    tb = torch.tensor(b0, dtype=torch.float64, requires_grad=True)
    th = torch.clamp(tx @ tw + tb, min=0.0)
    ts = _torch_softmax_lamp(torch.sqrt(torch.exp(torch.sin(th)) * 2.0)
                             / (torch.log(tx @ tw * 0.1 + 3.0) + 1.0), -1)
    tl = (ts * torch.tan(torch.cos(th) * 0.5)).sum(1, keepdim=True).sum(0, keepdim=True)
    tl.backward()
    for mine, ref in ((loss.data, tl.detach()), (x.grad, tx.grad), (w.grad, tw.grad),
                      (b.grad, tb.grad)):
        ref = ref.numpy()
        assert np.max(np.abs(mine - ref)) / (np.max(np.abs(ref)) + 1e-10) < 1e-4


def test_mlp_trajectory_vs_torch(oracle):
    """README MLP (config 0) shapes, 5 steps: oracle vs a torch float64
    restatement of the same graph."""
    rng = np.random.default_rng(0)
    x = rng.random((32, 256), dtype=np.float32)
    y = rng.random((32, 10), dtype=np.float32)
    ws = [rng.standard_normal((256, 64), dtype=np.float32),
          rng.standard_normal((64, 10), dtype=np.float32)]
    bs = [rng.standard_normal((64,), dtype=np.float32),
          rng.standard_normal((10,), dtype=np.float32)]
    losses, fw, fb = oracle.mlp_train(ws, bs, x, y, steps=5)

    tw = [torch.tensor(w, dtype=torch.float64) for w in ws]
    tb = [torch.tensor(b, dtype=torch.float64) for b in bs]
    tx, ty = torch.tensor(x, dtype=torch.float64), torch.tensor(y, dtype=torch.float64)
    tl = []
    for _ in range(5):
        for t in tw + tb:
            t.requires_grad_(True)
        h = torch.clamp(tx @ tw[0] + tb[0], min=0.0)
        p = _torch_softmax_lamp(h @ tw[1] + tb[1], -1)
        loss = (-ty * torch.log(p + 1e-3)).sum(1, keepdim=True).sum(0, keepdim=True)
        loss.backward()
        tl.append(float(loss.detach()))
        tw = [(w - 1e-3 * w.grad).detach() for w in tw]
        tb = [(b - 1e-3 * b.grad).detach() for b in tb]
    np.testing.assert_allclose(losses, tl, rtol=1e-4)
    for mine, ref in zip(fw + fb, tw + tb):
        ref = ref.numpy()
        assert np.max(np.abs(mine - ref)) / np.max(np.abs(ref)) < 1e-4


def test_mlp_step_gemm_orders_vs_torch(oracle):
    """Both GEMM orders of the oracle's MLP step (sequential fp32, float64
    accumulation) match a torch float64 step of the same graph within 1e-5
    (the remaining error is the fp32 elementwise rounding both share); a
    wrong product (a transposed operand, a dropped term) would miss both."""
    rng = np.random.default_rng(5)
    x = rng.random((32, 256), dtype=np.float32)
    y = rng.random((32, 10), dtype=np.float32)
    ws = [(rng.standard_normal((256, 64)) * 0.1).astype(np.float32),
          (rng.standard_normal((64, 10)) * 0.1).astype(np.float32)]
    bs = [(rng.standard_normal(64) * 0.1).astype(np.float32),
          (rng.standard_normal(10) * 0.1).astype(np.float32)]
    tw = [torch.tensor(w, dtype=torch.float64, requires_grad=True) for w in ws]
    tb = [torch.tensor(b, dtype=torch.float64, requires_grad=True) for b in bs]
    tx, ty = torch.tensor(x, dtype=torch.float64), torch.tensor(y, dtype=torch.float64)
    h = torch.clamp(tx @ tw[0] + tb[0], min=0.0)
    p = _torch_softmax_lamp(h @ tw[1] + tb[1], -1)
    tl = (-ty * torch.log(p + 1e-3)).sum(1, keepdim=True).sum(0, keepdim=True)
    tl.backward()
    want = [t.grad.numpy() for t in (tw[0], tb[0], tw[1], tb[1])]
    tlv = float(tl.detach())
    for f64 in (False, True):
        loss, gw, gb = oracle.mlp_step(ws, bs, x, y, f64_gemm=f64)
        assert abs(loss - tlv) <= 1e-5 * abs(tlv)
        got = [gw[0], gb[0], gw[1], gb[1]]
        for g, w in zip(got, want):
            assert np.max(np.abs(g - w)) / np.max(np.abs(w)) < 1e-5


def test_mlp_step_with_relu_masks_vs_torch(oracle):
    """relu_masks replaces the ReLU's backward mask and nothing else: with
    the natural mask (0 < t) the step equals the plain step exactly, and with
    two units flipped (one passing unit blocked, one blocked unit passed) it
    matches a torch float64 step whose ReLU has that gradient mask and
    clamp's values."""
    rng = np.random.default_rng(6)
    x = rng.random((32, 256), dtype=np.float32)
    y = rng.random((32, 10), dtype=np.float32)
    ws = [(rng.standard_normal((256, 64)) * 0.1).astype(np.float32),
          (rng.standard_normal((64, 10)) * 0.1).astype(np.float32)]
    bs = [(rng.standard_normal(64) * 0.1).astype(np.float32),
          (rng.standard_normal(10) * 0.1).astype(np.float32)]
    t = oracle.binary("add", oracle.matmul(x, ws[0]), bs[0])
    natural = t > 0
    plain = oracle.mlp_step(ws, bs, x, y)
    same = oracle.mlp_step(ws, bs, x, y, relu_masks=[natural])
    assert same[0] == plain[0]
    for g, w in zip(same[1] + same[2], plain[1] + plain[2]):
        assert np.array_equal(g, w)
    mask = natural.copy()
    pos, neg = np.argwhere(natural)[3], np.argwhere(~natural)[5]
    mask[tuple(pos)], mask[tuple(neg)] = False, True
    tw = [torch.tensor(w, dtype=torch.float64, requires_grad=True) for w in ws]
    tb = [torch.tensor(b, dtype=torch.float64, requires_grad=True) for b in bs]
    tx, ty = torch.tensor(x, dtype=torch.float64), torch.tensor(y, dtype=torch.float64)
    th = tx @ tw[0] + tb[0]
    tm = torch.tensor(mask, dtype=torch.float64)
    h = torch.clamp(th, min=0.0).detach() + (th - th.detach()) * tm
    p = _torch_softmax_lamp(h @ tw[1] + tb[1], -1)
    tl = (-ty * torch.log(p + 1e-3)).sum(1, keepdim=True).sum(0, keepdim=True)
    tl.backward()
    want = [t_.grad.numpy() for t_ in (tw[0], tb[0], tw[1], tb[1])]
    loss, gw, gb = oracle.mlp_step(ws, bs, x, y, f64_gemm=True, relu_masks=[mask])
    assert abs(loss - float(tl.detach())) <= 1e-5 * abs(float(tl.detach()))
    for g, w in zip([gw[0], gb[0], gw[1], gb[1]], want):
        assert np.max(np.abs(g - w)) / np.max(np.abs(w)) < 1e-5
    # the flips are visible: the first layer's gradients move
    assert np.max(np.abs(gw[0] - plain[1][0])) > 1e-3 * np.max(np.abs(plain[1][0]))


# ------------------------------------------------ typed (non-fp32) oracle

from oracle import lamp_typed as T  # noqa: E402

_INT_BITS = {np.int16: 16, np.int32: 32, np.int64: 64}


def _signed(v: int, bits: int) -> int:
    v &= (1 << bits) - 1
    return v - (1 << bits) if v >> (bits - 1) else v


def _cdiv(x: int, y: int) -> int:
    q = abs(x) // abs(y)
    return q if (x < 0) == (y < 0) else -q


@pytest.mark.parametrize("dt", [np.int16, np.int32, np.int64])
def test_typed_int_arithmetic_vs_python_ints(dt):
    """Wrap-around add/sub/mul and truncating division against Python's exact
    integers reduced modulo 2^bits (the two's-complement results the
    reference's C++ kernels produce), extremes included."""
    bits = _INT_BITS[dt]
    info = np.iinfo(dt)
    rng = np.random.default_rng(bits)
    a = np.concatenate([rng.integers(info.min, info.max, 400, dtype=dt, endpoint=True),
                        np.array([info.min, info.max, -1, 0, 1, 7, -7], dt)])
    b = np.concatenate([rng.integers(info.min, info.max, 400, dtype=dt, endpoint=True),
                        np.array([1, -1, 2, 3, -2, 2, -2], dt)])
    for op, f in (("add", lambda x, y: x + y), ("sub", lambda x, y: x - y),
                  ("mul", lambda x, y: x * y)):
        got = T.binary(op, a, b)
        assert got.dtype == dt
        want = [_signed(f(int(x), int(y)), bits) for x, y in zip(a, b)]
        assert got.tolist() == want, op
    ok = (b != 0) & ~((a == info.min) & (b == -1))
    got = T.binary("div", a[ok], b[ok])
    assert got.tolist() == [_cdiv(int(x), int(y)) for x, y in zip(a[ok], b[ok])]
    assert T.binary("div", np.array([-7, 7, -7], dt), np.array([2, -2, -2], dt)).tolist() == [-3, -3, 3]


def test_typed_bool_arithmetic_is_cpp_bool():
    """bool + bool etc. promote to int and convert back (nonzero -> true)."""
    t = np.array([False, False, True, True])
    u = np.array([False, True, False, True])
    assert T.binary("add", t, u).tolist() == [bool(int(x) + int(y)) for x, y in zip(t, u)]
    assert T.binary("sub", t, u).tolist() == [bool(int(x) - int(y)) for x, y in zip(t, u)]
    assert T.binary("mul", t, u).tolist() == [bool(int(x) * int(y)) for x, y in zip(t, u)]
    assert T.binary("eq", t, u).tolist() == [x == y for x, y in zip(t, u)]
    assert T.unary("neg", t).tolist() == t.tolist()
    assert T.reduce("sum", np.array([[0, 1], [0, 0]], bool), 0).tolist() == [[False, True]]
    assert T.reduce("prod", np.array([[1, 1], [0, 1]], bool), 0).tolist() == [[False, True]]


def test_typed_promotion_and_casts():
    """Promotion is the larger DataType code; float -> int truncates."""
    names = [np.bool_, np.int16, np.int32, np.int64, np.float32, np.float64]
    for i, x in enumerate(names):
        for j, y in enumerate(names):
            got = T.binary("add", np.zeros(2, x), np.zeros(2, y)).dtype
            assert got == np.dtype(names[max(i, j)])
    assert T.cast(np.array([2.7, -2.7, 0.5]), np.int32).tolist() == [2, -2, 0]
    # int32 + float32: the int is rounded to float32 before the add
    got = T.binary("add", np.array([16777217], np.int32), np.array([0.0], np.float32))
    assert got.dtype == np.float32 and got.tolist() == [16777216.0]


def test_typed_int_transcendentals_truncate():
    x = np.array([0, 1, 2, 3, 10], np.int32)
    assert T.unary("exp", x).tolist() == [1, 2, 7, 20, 22026]
    assert T.unary("sqrt", np.array([10, 16, 99], np.int64)).tolist() == [3, 4, 9]
    assert T.unary("log", np.array([1, 2, 100], np.int16)).tolist() == [0, 0, 4]
    assert T.unary("neg", np.array([-32768, 5], np.int16)).tolist() == [-32768, -5]
    assert T.unary("clamp", np.array([-5, 3, 9], np.int32), 0.0, 4.7).tolist() == [0, 3, 4]
    assert T.binary("pow", np.array([2, 3, -2], np.int32), np.array([10, 3, 3], np.int32)).tolist() == [1024, 27, -8]


def test_typed_reductions():
    x = np.array([[30000, 1], [30000, 2]], np.int16)
    assert T.reduce("sum", x, 0).tolist() == [[_signed(60000, 16), 3]]
    assert T.reduce("prod", np.array([[65536], [65536]], np.int64), 0).tolist() == [[2 ** 32]]
    assert T.reduce("max", np.array([[np.nan], [1.0]]), 0).tolist() == [[1.0]]
    assert T.reduce("max", np.array([[1.0], [np.nan]]), 0).tolist() == [[1.0]]
    assert T.reduce("min", np.zeros((0, 2), np.int32), 0).tolist() == [[2 ** 31 - 1] * 2]
    assert T.reduce("max", np.zeros((0, 1)), 0).tolist() == [[-np.finfo(np.float64).max]]
    v = np.random.default_rng(3).standard_normal((50, 3))
    np.testing.assert_allclose(T.reduce("sum", v, 0)[0], [sum(c) for c in v.T], rtol=1e-14)


@pytest.mark.parametrize("dt", [np.int16, np.int32, np.int64, np.bool_])
def test_typed_matmul_vs_brute_force(dt):
    rng = np.random.default_rng(7)
    if dt is np.bool_:
        a, b = rng.random((5, 7)) < 0.3, rng.random((7, 4)) < 0.3
        want = [[any(a[i, k] and b[k, j] for k in range(7)) for j in range(4)] for i in range(5)]
    else:
        info, bits = np.iinfo(dt), _INT_BITS[dt]
        a = rng.integers(info.min, info.max, (5, 7), dtype=dt, endpoint=True)
        b = rng.integers(info.min, info.max, (7, 4), dtype=dt, endpoint=True)
        want = [[_signed(sum(int(a[i, k]) * int(b[k, j]) for k in range(7)), bits)
                 for j in range(4)] for i in range(5)]
    got = T.matmul(a, b)
    assert got.dtype == np.dtype(dt) and got.tolist() == want


def test_typed_float64_ops_are_ieee():
    """numpy float64 arithmetic is the IEEE double arithmetic of the C++
    kernels: pin against Python floats (also binary64)."""
    xs = [0.1, -3.5, 1e300, 2.0 ** -1074, 7.0]
    ys = [0.2, 1e-300, 3.0, -0.0, 7.0]
    a, b = np.array(xs), np.array(ys)
    assert T.binary("add", a, b).tolist() == [x + y for x, y in zip(xs, ys)]
    assert T.binary("mul", a, b).tolist() == [x * y for x, y in zip(xs, ys)]
    assert T.binary("div", a[:4], b[:4] + 1).tolist() == [x / (y + 1) for x, y in zip(xs[:4], ys[:4])]
