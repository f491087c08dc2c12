"""Random float64 graphs on the device against torch float64 autograd.

The reference checks its device backend with float64 differential suites:
random chains of ops evaluated by rushlite and by torch, forward value and
every input gradient compared, with and without capture
(tests/graphs/test_graphs.py:38-45, tests/graphs/runner.py:44-74,
tests/stress/pytorch_stress_test.py:57-110).  This suite does the same for the
MI355X backend with its own generator, in float64 and float32: each seed draws
a program of 10-14 ops
over broadcastable leaves -- binary ops, bounded unary ops, keep-dims
reductions over either axis, matmul and transpose -- builds it in both
libraries, and compares under Lamp3's normalised metric
(tests/stress/testutils.py:47-50) at 1e-9.  Where Lamp3's gradient rules differ
from torch's, the torch side uses Lamp3's: max/min send the gradient to every
tied position (functions/reduct_ops.cpp:14; torch picks one), and clamp's
backward uses strict bounds (cpu/kernels.hpp:143-152; torch's is inclusive).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from _helpers import rel_err  # noqa: E402

torch = pytest.importorskip("torch")

SHAPES = [(16, 16), (16, 1), (1, 16), (16,)]
TOL = 1e-9


class _LampMax(torch.autograd.Function):
    """max/min over `dim` (keep-dims) with Lamp3's tie rule: every position
    equal to the result receives the gradient."""

    @staticmethod
    def forward(ctx, x, dim, is_max):
        out = x.amax(dim, keepdim=True) if is_max else x.amin(dim, keepdim=True)
        ctx.save_for_backward(x, out)
        return out

    @staticmethod
    def backward(ctx, g):
        x, out = ctx.saved_tensors
        return g * (x == out).to(g.dtype), None, None


class _LampClamp(torch.autograd.Function):
    """clamp with Lamp3's strict-bounds backward (ClampBackwardFunctor,
    cpu/kernels.hpp:143-152): a value sitting exactly on a bound gets no
    gradient (torch passes it through)."""

    @staticmethod
    def forward(ctx, x, lo, hi):
        ctx.save_for_backward(x)
        ctx.lo, ctx.hi = lo, hi
        return torch.clamp(x, lo, hi)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return g * ((x > ctx.lo) & (x < ctx.hi)).to(g.dtype), None, None


class TorchOps:
    add = staticmethod(lambda a, b: a + b)
    sub = staticmethod(lambda a, b: a - b)
    mul = staticmethod(lambda a, b: a * b)
    div = staticmethod(lambda a, b: a / b)
    pow = staticmethod(lambda a, b: a ** b)
    neg = staticmethod(lambda a: -a)
    exp = staticmethod(torch.exp)
    log = staticmethod(torch.log)
    sqrt = staticmethod(torch.sqrt)
    sin = staticmethod(torch.sin)
    cos = staticmethod(torch.cos)
    tan = staticmethod(torch.tan)
    abs = staticmethod(torch.abs)
    clamp = staticmethod(lambda a, lo, hi: _LampClamp.apply(a, lo, hi))
    sum = staticmethod(lambda a, d: a.sum(d, keepdim=True))
    max = staticmethod(lambda a, d: _LampMax.apply(a, d, True))
    min = staticmethod(lambda a, d: _LampMax.apply(a, d, False))
    matmul = staticmethod(lambda a, b: a @ b)
    transpose = staticmethod(lambda a: a.t())

    @staticmethod
    def const(like, v):
        return torch.tensor([v], dtype=torch.float64)


def lamp_ops(rsl, kind):
    class LampOps:
        add = staticmethod(lambda a, b: a + b)
        sub = staticmethod(lambda a, b: a - b)
        mul = staticmethod(lambda a, b: a * b)
        div = staticmethod(lambda a, b: a / b)
        pow = staticmethod(lambda a, b: rsl.pow(a, b))
        neg = staticmethod(lambda a: -a)
        exp = staticmethod(rsl.exp)
        log = staticmethod(rsl.log)
        sqrt = staticmethod(rsl.sqrt)
        sin = staticmethod(rsl.sin)
        cos = staticmethod(rsl.cos)
        tan = staticmethod(rsl.tan)
        abs = staticmethod(rsl.abs)
        clamp = staticmethod(lambda a, lo, hi: rsl.clamp(a, lo, hi))
        sum = staticmethod(lambda a, d: rsl.sum(a, d))
        max = staticmethod(lambda a, d: rsl.max(a, d))
        min = staticmethod(lambda a, d: rsl.min(a, d))
        matmul = staticmethod(rsl.matmul)
        transpose = staticmethod(rsl.transpose)

        @staticmethod
        def const(like, v):
            return rsl.Variable(np.array([v]), dtype=kind)
    return LampOps


def broadcast(a, b):
    a, b = list(a), list(b)
    n = max(len(a), len(b))
    a, b = [1] * (n - len(a)) + a, [1] * (n - len(b)) + b
    out = []
    for x, y in zip(a, b):
        if x != 1 and y != 1 and x != y:
            return None
        out.append(max(x, y))
    return tuple(out)


def make_program(seed):
    """A list of steps over a value pool; each step names an op and the pool
    indices it reads, with every operation kept in a numerically tame range
    (denominators >= 1, positive log/sqrt/pow arguments, bounded tan)."""
    rng = np.random.default_rng(seed)
    leaves = [SHAPES[i] for i in rng.integers(0, len(SHAPES), 4)]
    leaves[0] = (16, 16)
    shapes = list(leaves)
    steps = []
    for _ in range(int(rng.integers(10, 15))):
        kind = rng.choice(["bin", "bin", "bin", "unary", "unary", "reduce", "matmul", "transpose"])
        recent = list(range(max(0, len(shapes) - 5), len(shapes)))
        if kind == "bin":
            i = int(rng.choice(recent))
            js = [j for j in range(len(shapes)) if broadcast(shapes[i], shapes[j])]
            j = int(rng.choice(js))
            op = str(rng.choice(["add", "sub", "mul", "div", "pow"]))
            steps.append(("bin", op, i, j))
            shapes.append(broadcast(shapes[i], shapes[j]))
        elif kind == "unary":
            i = int(rng.choice(recent))
            op = str(rng.choice(["neg", "exp", "log", "sqrt", "sin", "cos", "tan", "abs", "clamp"]))
            steps.append(("unary", op, i))
            shapes.append(shapes[i])
        elif kind == "reduce":
            cand = [i for i in recent if len(shapes[i]) == 2]
            if not cand:
                continue
            i = int(rng.choice(cand))
            axis = int(rng.integers(0, 2))
            op = str(rng.choice(["sum", "max", "min"]))
            steps.append(("reduce", op, i, axis))
            s = list(shapes[i])
            s[axis] = 1
            shapes.append(tuple(s))
        elif kind == "matmul":
            cand = [i for i in range(len(shapes)) if shapes[i] == (16, 16)]
            rhs = [j for j in range(len(shapes)) if len(shapes[j]) == 2 and shapes[j][0] == 16]
            i, j = int(rng.choice(cand)), int(rng.choice(rhs))
            steps.append(("matmul", "matmul", i, j))
            shapes.append((16, shapes[j][1]))
        else:
            cand = [i for i in recent if len(shapes[i]) == 2]
            if not cand:
                continue
            i = int(rng.choice(cand))
            steps.append(("transpose", "transpose", i))
            shapes.append((shapes[i][1], shapes[i][0]))
    return leaves, steps, shapes


def run(ops, leaves, steps, shapes):
    out = _run_steps(ops, leaves, steps)
    if len(shapes[-1]) == 1:
        return ops.sum(out, 0)
    return ops.sum(ops.sum(out, 0), 1)


@pytest.fixture(scope="module")
def rsl(hip):
    import rushlite_amd
    return rushlite_amd


def _torch_eval(evaluate, arrs):
    tv = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in arrs]
    out = evaluate(tv)
    out.backward()
    return (out.detach().numpy().reshape(-1),
            [np.zeros(a.shape) if t.grad is None else t.grad.numpy() for t, a in zip(tv, arrs)])


def skip_if_ill_conditioned(evaluate, arrs, dtype, tol):
    """Skips a program whose torch float64 value or input gradients move by
    more than `tol` when its inputs move by one ulp of `dtype` (two random
    perturbations): a max/min tie that one rounding breaks, or a cancelling
    sum, where two correct evaluation orders may differ by more than the bar."""
    base_out, base_grads = _torch_eval(evaluate, arrs)
    eps = float(np.finfo(dtype).eps)
    for trial in range(2):
        rng = np.random.default_rng(77 + trial)
        moved = [(a * (1 + eps * rng.uniform(-1, 1, a.shape))).astype(dtype) for a in arrs]
        out, grads = _torch_eval(evaluate, moved)
        errs = [rel_err(out, base_out)]
        errs += [rel_err(g.reshape(b.shape), b) for g, b in zip(grads, base_grads)]
        if max(errs) > tol:
            pytest.skip(f"ill-conditioned: a one-ulp input change moves torch float64 by {max(errs):.2g}")


def check_graph(rsl, seed, capture, dtype, tol):
    leaves, steps, shapes = make_program(seed)
    rng = np.random.default_rng(1000 + seed)
    arrs = [rng.uniform(-1.0, 1.0, s).astype(dtype) for s in leaves]
    skip_if_ill_conditioned(lambda tv: run(TorchOps, tv, steps, shapes), arrs, dtype, tol)
    tv = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in arrs]
    t_out = run(TorchOps, tv, steps, shapes)
    t_out.backward()
    kind = rsl.dtype.float64 if dtype == np.float64 else rsl.dtype.float32
    lv = [rsl.Variable(a, requires_grad=True, dtype=kind) for a in arrs]
    ops = lamp_ops(rsl, kind)
    with rsl.capture_on(capture):
        l_out = run(ops, lv, steps, shapes)
    l_out.backward()
    want = t_out.detach().numpy().reshape(-1)
    got = l_out.numpy().reshape(-1)
    assert rel_err(got, want) <= tol, (seed, steps)
    for i, (t, l) in enumerate(zip(tv, lv)):
        g_want = t.grad.numpy() if t.grad is not None else np.zeros(leaves[i])
        assert rel_err(l.grad.numpy().reshape(g_want.shape), g_want) <= tol, (seed, i, steps)


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
@pytest.mark.parametrize("seed", range(24))
def test_random_graph_float64_matches_torch(rsl, seed, capture):
    check_graph(rsl, seed, capture, np.float64, TOL)


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
@pytest.mark.parametrize("seed", range(24))
def test_random_graph_float32_matches_torch(rsl, seed, capture):
    """The float32 path (fused regions, row kernels, MFMA GEMMs) on the same
    programs, against torch float64 at the reference stress suites' 1e-4
    (tests/stress/pytorch_stress_test.py:92-110)."""
    check_graph(rsl, seed, capture, np.float32, 1e-4)


# ---------------------------------------------------------------- other shapes
#
# The same kind of program over [R, C] leaves (with [R, 1], [1, C] and [C]
# broadcasts), at shapes that take the other code paths: float4 bodies and
# multi-wave rows (64 x 128, 130 x 64), the indexed path and short rows (33 x 7),
# and long rows, large reductions and a K = 1000 GEMM (256 x 1000).  Float32
# only, where the fused kernels differ most from the eager ones.  The checker is
# the float32 oracle (Lamp3's CPU arithmetic and tie rule); a program whose
# float32 oracle is itself more than 1e-4 from torch float64 is ill-conditioned
# in float32 (a max/min tie that one rounding breaks, a cancelling sum), where
# any two valid summation orders may differ by more than the bar, and is skipped.

RC_SHAPES = [(64, 128), (33, 7), (130, 64), (256, 1000)]


def make_program_rc(seed, R, C):
    """make_program over [R, C]-based leaves; a matmul takes any 2-D value
    and a right operand whose rows match its columns."""
    rng = np.random.default_rng(seed)
    pool_shapes = [(R, C), (R, 1), (1, C), (C,)]
    leaves = [pool_shapes[i] for i in rng.integers(0, len(pool_shapes), 4)]
    leaves[0] = (R, C)
    shapes = list(leaves)
    steps = []
    for _ in range(int(rng.integers(10, 18))):
        kind = rng.choice(["bin", "bin", "bin", "unary", "unary", "reduce", "matmul", "transpose"])
        recent = list(range(max(0, len(shapes) - 5), len(shapes)))
        if kind == "bin":
            i = int(rng.choice(recent))
            j = int(rng.choice([j for j in range(len(shapes)) if broadcast(shapes[i], shapes[j])]))
            op = str(rng.choice(["add", "sub", "mul", "div", "pow"]))
            steps.append(("bin", op, i, j))
            shapes.append(broadcast(shapes[i], shapes[j]))
        elif kind == "unary":
            i = int(rng.choice(recent))
            op = str(rng.choice(["neg", "exp", "log", "sqrt", "sin", "cos", "tan", "abs", "clamp"]))
            steps.append(("unary", op, i))
            shapes.append(shapes[i])
        elif kind == "reduce":
            cand = [i for i in recent if len(shapes[i]) == 2]
            if not cand:
                continue
            i = int(rng.choice(cand))
            axis = int(rng.integers(0, 2))
            steps.append(("reduce", str(rng.choice(["sum", "max", "min"])), i, axis))
            s = list(shapes[i])
            s[axis] = 1
            shapes.append(tuple(s))
        elif kind == "matmul":
            i = int(rng.choice([i for i in range(len(shapes)) if len(shapes[i]) == 2]))
            rhs = [j for j in range(len(shapes))
                   if len(shapes[j]) == 2 and shapes[j][0] == shapes[i][1]]
            if not rhs:
                continue
            j = int(rng.choice(rhs))
            steps.append(("matmul", "matmul", i, j))
            shapes.append((shapes[i][0], shapes[j][1]))
        else:
            cand = [i for i in recent if len(shapes[i]) == 2]
            if not cand:
                continue
            i = int(rng.choice(cand))
            steps.append(("transpose", "transpose", i))
            shapes.append((shapes[i][1], shapes[i][0]))
    return leaves, steps, shapes


def oracle_ops(O):
    class OracleOps:
        add = staticmethod(O.add)
        sub = staticmethod(O.sub)
        mul = staticmethod(O.mul)
        div = staticmethod(O.div)
        pow = staticmethod(O.pow_)
        neg = staticmethod(O.neg)
        exp = staticmethod(O.exp)
        log = staticmethod(O.log)
        sqrt = staticmethod(O.sqrt)
        sin = staticmethod(O.sin)
        cos = staticmethod(O.cos)
        tan = staticmethod(O.tan)
        abs = staticmethod(O.abs_)
        clamp = staticmethod(O.clamp)
        sum = staticmethod(O.sum_)
        max = staticmethod(O.max_)
        min = staticmethod(O.min_)
        matmul = staticmethod(O.matmul_v)
        transpose = staticmethod(O.transpose_v)

        @staticmethod
        def const(like, v):
            return O.OVar(np.array([v], np.float32))
    return OracleOps


def _errors(out, grads, want_out, want_grads, leaves):
    errs = [rel_err(np.asarray(out).reshape(-1), np.asarray(want_out).reshape(-1))]
    for i, (g, w) in enumerate(zip(grads, want_grads)):
        w = np.zeros(leaves[i]) if w is None else np.asarray(w)
        errs.append(rel_err(np.asarray(g).reshape(w.shape), w))
    return max(errs)


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
@pytest.mark.parametrize("shape", RC_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("seed", range(6))
def test_random_graph_float32_shapes_vs_oracle(rsl, oracle, seed, shape, capture):
    R, C = shape
    leaves, steps, shapes = make_program_rc(seed, R, C)
    rng = np.random.default_rng(1000 + seed)
    arrs = [rng.uniform(-1.0, 1.0, s).astype(np.float32) for s in leaves]
    ov = [oracle.OVar(a.copy(), requires_grad=True) for a in arrs]
    o_out = run(oracle_ops(oracle), ov, steps, shapes)
    o_out.backward()
    tv = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in arrs]
    t_out = run(TorchOps, tv, steps, shapes)
    t_out.backward()
    conditioning = _errors(o_out.data, [o.grad for o in ov], t_out.detach().numpy(),
                           [None if t.grad is None else t.grad.numpy() for t in tv], leaves)
    if conditioning > 1e-4:
        pytest.skip(f"ill-conditioned in float32: oracle vs torch float64 {conditioning:.2g}")
    lv = [rsl.Variable(a, requires_grad=True) for a in arrs]
    with rsl.capture_on(capture):
        l_out = run(lamp_ops(rsl, rsl.dtype.float32), lv, steps, shapes)
    l_out.backward()
    err = _errors(l_out.numpy(), [v.grad.numpy() for v in lv], o_out.data,
                  [o.grad for o in ov], leaves)
    assert err <= 1e-4, (seed, shape, err, steps)


# ---------------------------------------------------------------- 3-d programs
#
# Elementwise and keep-dims reduction programs over 3-d leaves with every kind
# of broadcast ([A,B,C] against [A,1,C], [1,B,1], [B,C], [C], [A,B,1],
# [1,1,C]) and reductions over any axis: the n-d indexed kernels, 3-d fused
# regions and rows.  Float64 against torch float64 at 1e-9; float32 against the
# float32 oracle at 1e-4, skipping a program ill-conditioned in float32 as above.

D3_SHAPES = [(4, 33, 64), (3, 5, 7), (2, 130, 256)]


def make_program_3d(seed, A, B, C):
    rng = np.random.default_rng(seed)
    pool_shapes = [(A, B, C), (A, 1, C), (1, B, 1), (B, C), (C,), (A, B, 1), (1, 1, C)]
    leaves = [pool_shapes[i] for i in rng.integers(0, len(pool_shapes), 4)]
    leaves[0] = (A, B, C)
    shapes = list(leaves)
    steps = []
    for _ in range(int(rng.integers(8, 16))):
        kind = rng.choice(["bin", "bin", "bin", "unary", "unary", "reduce"])
        recent = list(range(max(0, len(shapes) - 5), len(shapes)))
        i = int(rng.choice(recent))
        if kind == "bin":
            j = int(rng.choice([j for j in range(len(shapes)) if broadcast(shapes[i], shapes[j])]))
            steps.append(("bin", str(rng.choice(["add", "sub", "mul", "div", "pow"])), i, j))
            shapes.append(broadcast(shapes[i], shapes[j]))
        elif kind == "unary":
            op = str(rng.choice(["neg", "exp", "log", "sqrt", "sin", "cos", "tan", "abs", "clamp"]))
            steps.append(("unary", op, i))
            shapes.append(shapes[i])
        else:
            axis = int(rng.integers(0, len(shapes[i])))
            steps.append(("reduce", str(rng.choice(["sum", "max", "min"])), i, axis))
            s = list(shapes[i])
            s[axis] = 1
            shapes.append(tuple(s))
    return leaves, steps, shapes


@pytest.mark.parametrize("capture", [False, True], ids=["eager", "captured"])
@pytest.mark.parametrize("shape", D3_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("seed", range(4))
def test_random_graph_3d(rsl, oracle, seed, shape, capture):
    leaves, steps, shapes = make_program_3d(seed, *shape)
    rng = np.random.default_rng(1000 + seed)
    arrs = [rng.uniform(-1.0, 1.0, s) for s in leaves]
    for dtype in (np.float64, np.float32):
        a = [x.astype(dtype) for x in arrs]
        tv = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in a]
        t_out = _sum_all(TorchOps, _run_steps(TorchOps, tv, steps), shapes)
        t_out.backward()
        t_grads = [None if t.grad is None else t.grad.numpy() for t in tv]
        if dtype == np.float64:
            want, want_grads, tol = t_out.detach().numpy(), t_grads, 1e-9
            kind = rsl.dtype.float64
            try:
                skip_if_ill_conditioned(
                    lambda v: _sum_all(TorchOps, _run_steps(TorchOps, v, steps), shapes), a,
                    dtype, tol)
            except pytest.skip.Exception:
                continue  # ill-conditioned in float64: the float32 check below still runs
        else:
            ov = [oracle.OVar(x.copy(), requires_grad=True) for x in a]
            o_ops = oracle_ops(oracle)
            o_out = _sum_all(o_ops, _run_steps(o_ops, ov, steps), shapes)
            o_out.backward()
            want, want_grads, tol = o_out.data, [o.grad for o in ov], 1e-4
            if _errors(want, want_grads, t_out.detach().numpy(), t_grads, leaves) > 1e-4:
                continue  # ill-conditioned in float32
            kind = rsl.dtype.float32
        lv = [rsl.Variable(x, requires_grad=True, dtype=kind) for x in a]
        l_ops = lamp_ops(rsl, kind)
        with rsl.capture_on(capture):
            l_out = _sum_all(l_ops, _run_steps(l_ops, lv, steps), shapes)
        l_out.backward()
        err = _errors(l_out.numpy(), [v.grad.numpy() for v in lv], want, want_grads, leaves)
        assert err <= tol, (seed, shape, np.dtype(dtype).name, err, steps)


def _run_steps(ops, leaves, steps):
    """Evaluates the steps over the value pool, every operation kept in a tame
    range (denominators >= 1, positive log/sqrt/pow arguments, bounded tan);
    returns the last value."""
    pool = list(leaves)
    one = ops.const(pool[0], 1.0)
    half = ops.const(pool[0], 0.5)
    for st in steps:
        kind, op = st[0], st[1]
        if kind == "bin":
            a, b = pool[st[2]], pool[st[3]]
            if op == "div":
                r = ops.div(a, ops.add(ops.mul(b, b), one))
            elif op == "pow":
                r = ops.pow(ops.add(ops.mul(a, a), half), ops.clamp(b, -1.5, 1.5))
            else:
                r = getattr(ops, op)(a, b)
        elif kind == "unary":
            a = pool[st[2]]
            if op in ("log", "sqrt"):
                r = getattr(ops, op)(ops.add(ops.mul(a, a), one))
            elif op == "exp":
                r = ops.exp(ops.clamp(a, -3.0, 3.0))
            elif op == "tan":
                r = ops.tan(ops.mul(ops.sin(a), half))
            elif op == "clamp":
                r = ops.clamp(a, -0.75, 0.75)
            else:
                r = getattr(ops, op)(a)
        elif kind == "reduce":
            r = getattr(ops, op)(pool[st[2]], st[3])
        elif kind == "matmul":
            r = ops.matmul(pool[st[2]], pool[st[3]])
        else:
            r = ops.transpose(pool[st[2]])
        pool.append(r)
    return pool[-1]


def _sum_all(ops, out, shapes):
    for ax in range(len(shapes[-1]) - 1, -1, -1):
        out = ops.sum(out, ax)
    return out
