"""Framework-level parity on the HIP device, through rushlite_amd's Python API.

Covers the reference's known answers (tensor_tests.cpp, autograd_tests.cpp,
tests/unit/*) run on the GPU, capture/fusion semantics (one fused launch per
chain, fused == eager == oracle bit for bit where the ops are exact), the
README MLP trajectory against the oracle, and config-size properties.
"""
import json
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

from _helpers import SPECIALS, assert_within_ulp, rel_err, special_rows

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "lamp3_known_answers.json").read_text())
ATOL = GOLDEN["tolerance"]["atol"]
DBL_MAX = sys.float_info.max


@pytest.fixture(scope="module")
def rsl(hip):
    import rushlite_amd
    return rushlite_amd


def V(rsl, x, rg=False):
    return rsl.Variable(np.asarray(x, np.float32), requires_grad=rg)


def close(got, want):
    want = np.array([float(v) for v in want], np.float64)
    got = np.asarray(got, np.float64).reshape(-1)
    fin = np.isfinite(want)
    assert np.array_equal(np.isinf(got), np.isinf(want))
    np.testing.assert_allclose(got[fin], want[fin], atol=ATOL, rtol=0)


# --------------------------------------------------------- known answers

@pytest.mark.parametrize("case", GOLDEN["tensor"], ids=lambda c: c["name"])
@pytest.mark.parametrize("capture", [False, True])
def test_known_answers_binary(rsl, case, capture):
    a, b = V(rsl, case["a"]), V(rsl, case["b"])
    fn = getattr(rsl, case["op"])
    with rsl.capture_on(capture):
        out = fn(a, b)
    assert list(out.shape) == case["shape"]
    np.testing.assert_allclose(out.numpy().reshape(-1), case["expect"],
                               atol=case.get("atol", ATOL), rtol=0)


@pytest.mark.parametrize("case", GOLDEN["reduce"], ids=lambda c: c["name"])
def test_known_answers_reduce(rsl, case):
    out = getattr(rsl, case["op"])(V(rsl, case["a"]), case["axis"])
    assert list(out.shape) == case["shape"]
    close(out.tolist(), case["expect"])


@pytest.mark.parametrize("case", GOLDEN["autograd"], ids=lambda c: c["name"])
def test_known_answers_autograd(rsl, case):
    a = V(rsl, GOLDEN["inputs"]["a"], True)
    b = V(rsl, GOLDEN["inputs"]["b"], True)
    e, extra = case["expr"], {}
    if e == "a + b": out = a + b
    elif e == "a - b": out = a - b
    elif e == "a * b": out = a * b
    elif e == "a / b": out = a / b
    elif e == "exp(b)": out = rsl.exp(b)
    elif e == "log(a)": out = rsl.log(a)
    elif e == "a @ m":
        extra["m"] = V(rsl, case["m"], True)
        out = rsl.matmul(a, extra["m"])
    elif e == "transpose(a)": out = rsl.transpose(a)
    elif e == "sum(a, 1)": out = rsl.sum(a, 1)
    elif e == "max(a, 1)": out = rsl.max(a, 1)
    elif e == "min(a, 1)": out = rsl.min(a, 1)
    elif e == "a + r":
        extra["r"] = V(rsl, case["r"], True)
        out = a + extra["r"]
    else:
        raise AssertionError(e)
    close(out.tolist(), case["out"])
    out.backward()
    for key, var in (("grad_a", a), ("grad_b", b), ("grad_m", extra.get("m")),
                     ("grad_r", extra.get("r"))):
        if key in case:
            close(var.grad.tolist(), case[key])
    if "grad_r" in case:
        assert list(extra["r"].grad.shape) == [1, 2]


@pytest.mark.parametrize("case", GOLDEN["autograd_unary"], ids=lambda c: c["name"])
def test_known_answers_unary_grads(rsl, case):
    x = V(rsl, case["x"], True)
    fn = case["fn"]
    out = rsl.clamp(x, case["lo"], case["hi"]) if fn == "clamp" else getattr(rsl, fn)(x)
    out.backward()
    close(x.grad.tolist(), case["grad"])


def test_repeated_backward_accumulates_in_place(rsl):
    a = V(rsl, GOLDEN["inputs"]["a"], True)
    ptr = rsl._storage_ptr(a.grad)
    r = a * 2.0
    r.backward()
    assert rsl._storage_ptr(a.grad) == ptr
    r.backward()
    assert rsl._storage_ptr(a.grad) == ptr
    close(a.grad.tolist(), GOLDEN["repeated_backward"]["grad_a"])


def test_constant_gradient_then_a_term_accumulates_in_place(rsl):
    """a + b backward leaves a.grad the seed passed through (a constant, kept
    pending); a tensor handle taken from .grad then (a Variable made from it
    shares the tensor), and the gradient after a second pass adds a
    non-constant term (a * a: 2a), are the same tensor in the same buffer
    holding 1 + 2a, as the reference's in-place accumulation gives
    (variable.cpp:30-35, autograd_tests.cpp:487-514)."""
    a = V(rsl, [[1.0, 2.0], [3.0, 4.0]], True)
    b = V(rsl, [[5.0, 6.0], [7.0, 8.0]], True)
    (a + b).backward()
    held = rsl.Variable(a.grad)  # not read yet: still the pending constant
    (a * a).backward()
    want = [3.0, 5.0, 7.0, 9.0]
    assert a.grad.tolist() == want
    assert held.tolist() == want
    assert rsl._storage_ptr(held.data) == rsl._storage_ptr(a.grad)
    # a third pass keeps that buffer
    (a * 2.0).backward()
    assert held.tolist() == [5.0, 7.0, 9.0, 11.0]
    assert rsl._storage_ptr(held.data) == rsl._storage_ptr(a.grad)


def test_tensor_api(rsl):
    t = rsl._C._Tensor([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [3, 2], rsl.device.hip, rsl.dtype.float32)
    assert t.index([2, 1]) == 6.0 and t.index([1, 0]) == 3.0
    u = (t + 100.0) * 2.0
    assert u.tolist() == [202.0, 204.0, 206.0, 208.0, 210.0, 212.0]
    c = t.to(rsl.device.cpu)
    assert c.device == rsl.device.cpu and c.tolist() == t.tolist()
    back = c.to(rsl.device.hip)
    assert back.tolist() == t.tolist()
    t.fill(42.0)
    assert t.tolist() == [42.0] * 6
    i32 = rsl._C._Tensor([1, 2, 3, 4, 5, 6], [3, 2], rsl.device.hip, rsl.dtype.int32)
    s = rsl._C._Tensor([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [3, 2], rsl.device.hip, rsl.dtype.float32) + i32
    assert s.dtype == rsl.dtype.float32 and s.tolist() == [2.0, 4.0, 6.0, 8.0, 10.0, 12.0]
    r = t.reshape([6]).expand_dims(0)
    assert r.shape == [1, 6]
    with pytest.raises(RuntimeError):
        t.reshape([4])


def test_errors_surface_as_runtime_error(rsl):
    a = V(rsl, np.ones((3, 2)))
    b = V(rsl, np.ones((4, 5)))
    with pytest.raises(RuntimeError, match="Broadcast rule violation"):
        a + b
    with pytest.raises(RuntimeError, match="Incompatible"):
        rsl.matmul(a, a)
    with pytest.raises(RuntimeError):
        a.grad


# ------------------------------------------------------------- fusion

def test_capture_fuses_broadcast_chain_into_one_kernel(rsl, oracle):
    rng = np.random.default_rng(0)
    a_np = rng.random((257, 64), dtype=np.float32)
    b_np = rng.random((257, 1), dtype=np.float32)
    a, b = V(rsl, a_np), V(rsl, b_np)
    s0 = rsl._stats()
    with rsl.capture_on():
        c = a * a + b
        assert rsl._is_deferred(c)
    got = c.numpy()
    s1 = rsl._stats()
    assert s1["fused_launches"] - s0["fused_launches"] == 1
    assert s1["eager_launches"] == s0["eager_launches"]
    want = oracle.binary("add", oracle.binary("mul", a_np, a_np), b_np)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    eager = (a * a + b).numpy()
    assert np.array_equal(eager.view(np.uint32), got.view(np.uint32))


def chain6(rsl, a, b):
    return rsl.exp(a) * b - rsl.clamp(a, 0, DBL_MAX) / (b + 1)


def test_six_op_chain_fused_matches_eager_and_oracle(rsl, oracle):
    rng = np.random.default_rng(1)
    a_np = (rng.random((300, 128), dtype=np.float32) * 4 - 2).astype(np.float32)
    b_np = rng.random((300, 1), dtype=np.float32)
    a, b = V(rsl, a_np), V(rsl, b_np)
    s0 = rsl._stats()["fused_launches"]
    with rsl.capture_on():
        c = chain6(rsl, a, b)
    fused = c.numpy()
    assert rsl._stats()["fused_launches"] - s0 == 1
    eager = chain6(rsl, a, b).numpy()
    assert np.array_equal(fused.view(np.uint32), eager.view(np.uint32))
    O = oracle
    want = O.binary("sub", O.binary("mul", O.unary("exp", a_np), b_np),
                    O.binary("div", O.unary("clamp", a_np, 0.0, DBL_MAX),
                             O.binary("add", b_np, np.array([1.0], np.float32))))
    assert rel_err(fused, want) <= 1e-6


def test_fusion_cache_reuses_kernels(rsl):
    a, b = V(rsl, np.ones((64, 64))), V(rsl, np.ones((64, 1)))
    with rsl.capture_on():
        (a * a + b).realize()
    s0 = rsl._stats()
    for _ in range(3):
        with rsl.capture_on():
            (a * a + b).realize()
    s1 = rsl._stats()
    assert s1["jit_compiles"] == s0["jit_compiles"]
    assert s1["jit_cache_hits"] - s0["jit_cache_hits"] == 3


@pytest.mark.parametrize("sa,sb", [((5, 6, 7), (6, 1)), ((4, 1, 3), (1, 5, 3)),
                                   ((13,), (1,)), ((7, 9), (7, 9)), ((33, 10), (10,))])
def test_fusion_generic_layouts(rsl, oracle, sa, sb):
    rng = np.random.default_rng(7)
    a_np = rng.standard_normal(sa).astype(np.float32)
    b_np = (rng.random(sb) + 0.5).astype(np.float32)
    a, b = V(rsl, a_np), V(rsl, b_np)
    with rsl.capture_on():
        c = (-(a * b) + a) / b - rsl.abs(a)
    got = c.numpy()
    O = oracle
    want = O.binary("sub", O.binary("div", O.binary("add", O.unary("neg", O.binary("mul", a_np, b_np)), a_np), b_np),
                    O.unary("abs", a_np))
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_capture_realizes_outside_block_and_under_grad(rsl, oracle):
    a_np = np.arange(12, dtype=np.float32).reshape(3, 4) / 7
    a = V(rsl, a_np, True)
    with rsl.capture_on():
        y = rsl.sum(a * a + 1.0, 1)  # sum realises the fused a*a+1
    y.backward()
    assert np.array_equal(a.grad.numpy(), (a_np + a_np).astype(np.float32))


# ------------------------------------------------------------ module API

def test_module_params_and_functional_sgd(rsl):
    class S(rsl.Module):
        def __init__(self):
            super().__init__()
            self.w = rsl.Variable([1.0, 2.0], requires_grad=True)

        def forward(self, x):
            return x * self.w

    m = S()
    assert "w" not in vars(m) and m.w is m._params_dict["w"]
    x, y = rsl.Variable([1.0, 1.0]), rsl.Variable([3.0, 5.0])
    err = m(x) - y
    (err * err).sum(0).backward()
    p = m.params["w"]
    m.params["w"] = rsl.Variable(p.data - 0.1 * p.grad, requires_grad=True)
    np.testing.assert_allclose(m.params["w"].tolist(), [1.4, 2.6], rtol=1e-6)
    with rsl.no_grad():
        z = m.w * 2.0
    assert not z.requires_grad and z.grad_fn is None
    m.w = 3
    assert list(m.parameters()) == []


def test_sequential_named_parameters(rsl):
    from rushlite_amd.nets import layers
    model = layers.Sequential([layers.Linear(2, 2), layers.ReLU()])
    assert [n for n, _ in model.named_parameters()] == ["0.weights", "0.bias"]
    nb = rsl.Variable([1.0, 2.0], requires_grad=True)
    model.params["0.bias"] = nb
    assert model.layers[0].bias is nb
    lin = layers.Linear(2, 2, bias=False)
    lin.params["weights"] = rsl.Variable([[1.0, 0.0], [0.0, 1.0]], requires_grad=True)
    assert lin(rsl.Variable([[3.0, 4.0]])).tolist() == [3.0, 4.0]


# --------------------------------------------------------------- MLP

def _mlp(rsl, ws, bs):
    from rushlite_amd.nets import layers
    mods = []
    for i in range(len(ws)):
        mods.append(layers.Linear(*ws[i].shape))
        if i < len(ws) - 1:
            mods.append(layers.ReLU())
    mods.append(layers.Softmax(dim=-1))
    model = layers.Sequential(mods)
    li = 0
    for i, m in enumerate(mods):
        if isinstance(m, layers.Linear):
            model.params[f"{i}.weights"] = rsl.Variable(ws[li], requires_grad=True)
            model.params[f"{i}.bias"] = rsl.Variable(bs[li], requires_grad=True)
            li += 1
    return model


def run_mlp(rsl, model, x, y, steps, lr=1e-3):
    @rsl.capture()
    def forward(inp):
        return model(inp)

    losses = []
    for _ in range(steps):
        probs = forward(x)
        loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        losses.append(loss.tolist()[0])
        for name, p in list(model.named_parameters()):
            model.params[name] = rsl.Variable(p.data - lr * p.grad, requires_grad=True)
    return losses


def _mlp_problem(dims, batch, scale, seed=2):
    rng = np.random.default_rng(seed)
    x_np = rng.random((batch, dims[0]), dtype=np.float32)
    y_np = rng.random((batch, dims[-1]), dtype=np.float32)
    ws = [(rng.standard_normal((dims[i], dims[i + 1])) * scale).astype(np.float32)
          for i in range(len(dims) - 1)]
    bs = [(rng.standard_normal(dims[i + 1]) * scale).astype(np.float32)
          for i in range(len(dims) - 1)]
    return x_np, y_np, ws, bs


# Config 0 with the reference's randn(0, 1) Linear init, and a deeper net
# with a 0.1-scaled init.
MLP_CASES = [((256, 64, 10), 32, 1.0), ((128, 96, 40, 7), 20, 0.1)]


@pytest.mark.parametrize("dims,batch,scale", MLP_CASES)
def test_mlp_free_running_matches_oracle(rsl, oracle, dims, batch, scale):
    """README MLP (config 0) and a deeper variant, free-running for the first
    3 steps: per-step loss and final parameters within 1e-4 of the oracle.
    (Longer horizons amplify 1-ulp GEMM rounding differences chaotically,
    so they are checked step by step below instead.)"""
    x_np, y_np, ws, bs = _mlp_problem(dims, batch, scale)
    model = _mlp(rsl, ws, bs)
    steps = 3
    losses = run_mlp(rsl, model, V(rsl, x_np), V(rsl, y_np), steps)
    ref_losses, ref_w, ref_b = oracle.mlp_train(ws, bs, x_np, y_np, steps)
    assert rel_err(losses, ref_losses) <= 1e-4
    got = [p.numpy() for _, p in model.named_parameters()]
    ref = [t for pair in zip(ref_w, ref_b) for t in pair]
    for g, r in zip(got, ref):
        assert rel_err(g, r) <= 1e-4


@pytest.mark.parametrize("dims,batch,scale", MLP_CASES)
def test_mlp_each_step_matches_oracle(rsl, oracle, dims, batch, scale):
    """30 training steps on the GPU; before every step the oracle runs the
    same step from the GPU's current parameters, and the step's loss and
    every parameter gradient must agree within 1e-4 (teacher forcing).

    GEMM summation order is free within the GEMM tolerance, and at the
    reference's randn(0, 1) init the softmax of large logits amplifies it: two
    valid orders computed by the oracle itself (sequential fp32, and float64
    accumulation rounded once) already differ by up to ~5e-5 in a step's
    gradients.  Each gradient must therefore be within 1e-4 of at least one
    of those two oracle steps."""
    x_np, y_np, ws, bs = _mlp_problem(dims, batch, scale)
    model = _mlp(rsl, ws, bs)
    x, y = V(rsl, x_np), V(rsl, y_np)

    @rsl.capture()
    def forward(inp):
        return model(inp)

    for step in range(30):
        names = [n for n, _ in model.named_parameters()]
        params = [p.numpy() for _, p in model.named_parameters()]
        cur_w, cur_b = params[0::2], params[1::2]
        ref_loss, ref_gw, ref_gb = oracle.mlp_step(cur_w, cur_b, x_np, y_np)
        _, ref64_gw, ref64_gb = oracle.mlp_step(cur_w, cur_b, x_np, y_np, f64_gemm=True)
        probs = forward(x)
        loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        assert abs(loss.tolist()[0] - ref_loss) <= 1e-4 * abs(ref_loss), step
        grads = [p.grad.numpy() for _, p in model.named_parameters()]
        refs = [t for pair in zip(ref_gw, ref_gb) for t in pair]
        refs64 = [t for pair in zip(ref64_gw, ref64_gb) for t in pair]
        for g, r, r64 in zip(grads, refs, refs64):
            assert min(rel_err(g, r), rel_err(g, r64)) <= 1e-4, step
        for name, p in zip(names, list(model.parameters())):
            model.params[name] = rsl.Variable(p.data - 1e-3 * p.grad, requires_grad=True)


def _c4_problem(scale):
    """Config 4 as bench.py draws it: one generator (seed 2) gives x
    normal(0, 1) [512, 4096], the one-hot labels (integers in [0, 1000)),
    then each Linear's weights [in, out] and bias [out], normal(0, 1) times
    `scale` (1 is the reference's randn(0, 1) init, linear.py:25-29)."""
    dims, batch = (4096, 4096, 4096, 1000), 512
    rng = np.random.default_rng(2)
    x = rng.standard_normal((batch, dims[0]), dtype=np.float32)
    y = np.zeros((batch, dims[-1]), np.float32)
    y[np.arange(batch), rng.integers(0, dims[-1], batch)] = 1.0
    ws, bs = [], []
    for i in range(len(dims) - 1):
        ws.append(rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32) * np.float32(scale))
        bs.append(rng.standard_normal(dims[i + 1], dtype=np.float32) * np.float32(scale))
    return x, y, ws, bs


def _gpu_relu_masks(rsl, x, params, params_np):
    """Where each hidden ReLU of the GPU's forward passes gradient: the signs
    of its pre-activations x @ W + b from rsl.linear, the GEMM the Sequential's
    Linear -> ReLU node runs with ReLU added to its epilogue.  Each mask
    differs from the float64 pre-activation's sign (on the same GPU inputs)
    only where that value lies within 1e-4 of max|t| of zero."""
    masks, h = [], x
    with rsl.no_grad():
        for i in range(len(params) // 2 - 1):
            t = rsl.linear(h, params[2 * i], params[2 * i + 1])
            t_np = t.numpy()
            t64 = h.numpy().astype(np.float64) @ params_np[2 * i].astype(np.float64) \
                + params_np[2 * i + 1].astype(np.float64)
            m = t_np > 0
            flipped = m != (t64 > 0)
            assert np.all(np.abs(t64[flipped]) <= 1e-4 * np.abs(t64).max()), i
            assert flipped.sum() <= 1e-4 * m.size, (i, int(flipped.sum()))
            masks.append(m)
            h = rsl.clamp(t, 0, DBL_MAX)
    return masks


@pytest.mark.parametrize("scale", [1.0, 1.0 / 64], ids=["randn_init", "fan_in_init"])
def test_config4_wide_mlp_matches_oracle(rsl, oracle, scale):
    """Config 4 (Linear(4096,4096)-ReLU-Linear(4096,4096)-ReLU-Linear(4096,1000)
    -Softmax, batch 512, one-hot y) trained as the bench trains it: forward
    captured, loss and SGD update captured, three steps.  Before each step
    the oracle runs the same step from the GPU's parameters (README.md:116-126,
    linear.cpp:21-26, matrix_ops.cpp:8-24) with float64-accumulated GEMMs, a
    summation order within the GEMM tolerance; loss and every gradient must
    agree within 1e-4 under max|d| / max|true|, and each update must equal the
    oracle's p - lr*g on the GPU's p and g bit for bit.

    At the reference's randn(0, 1) init the logits reach ~1e5, the softmax is
    exactly one-hot in fp32 and every gradient is exactly zero (the gradient
    through the max cancels the one at the argmax), so that case pins the
    loss and exact zeros; the 1/64 (fan-in) init gives dense gradients (two
    oracle GEMM orders agree to ~6e-7 there).

    ReLU masks: a hidden pre-activation within rounding of zero can fall on
    either side of it in another valid summation order (K = 4096: ~1e-6),
    and one such unit moves a whole weight-gradient column by a batch row's
    share (~1e-2 of its largest entry).  The oracle step therefore takes the
    GPU's masks (signs of its own Linear GEMMs' pre-activations), and every
    place they differ from the float64 pre-activation's sign must lie within
    the GEMM bar (1e-4 of max|t|) of zero."""
    x_np, y_np, ws, bs = _c4_problem(scale)
    model = _mlp(rsl, ws, bs)
    x, y = V(rsl, x_np), V(rsl, y_np)
    lr = np.float32(1e-3)

    @rsl.capture()
    def forward(inp):
        return model(inp)

    for step in range(3):
        names = [n for n, _ in model.named_parameters()]
        params = [p.numpy() for _, p in model.named_parameters()]
        masks = _gpu_relu_masks(rsl, x, [p for _, p in model.named_parameters()], params)
        ref_loss, ref_gw, ref_gb = oracle.mlp_step(params[0::2], params[1::2], x_np, y_np,
                                                   f64_gemm=True, relu_masks=masks)
        probs = forward(x)
        with rsl.capture_on():
            loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        got_loss = loss.tolist()[0]
        assert abs(got_loss - ref_loss) <= 1e-4 * abs(ref_loss), (step, got_loss, ref_loss)
        grads = [p.grad.numpy() for _, p in model.named_parameters()]
        refs = [t for pair in zip(ref_gw, ref_gb) for t in pair]
        for name, g, r in zip(names, grads, refs):
            assert g.shape == r.shape, name
            if not np.any(r):
                assert not np.any(g), (step, name, float(np.abs(g).max()))
            else:
                assert rel_err(g, r) <= 1e-4, (step, name, rel_err(g, r))
        with rsl.capture_on():
            for name, p in list(model.named_parameters()):
                model.params[name] = rsl.Variable(p.data - 1e-3 * p.grad, requires_grad=True)
        rsl.realize_all(p for _, p in model.named_parameters())
        for name, p0, g, (_, p1) in zip(names, params, grads, model.named_parameters()):
            want = oracle.binary("sub", p0, oracle.binary("mul", np.array([lr]), g))
            assert np.array_equal(p1.numpy().view(np.uint32), want.view(np.uint32)), (step, name)
        del grads, refs, params


# ------------------------------------------------- config-size properties

def _oracle_chain6(oracle, e, a, b):
    """exp(a)*b - relu(a)/(b+1) from exp(a) = e, with the oracle's exact ops."""
    lhs = oracle.binary("mul", e, b)
    rhs = oracle.binary("div", oracle.unary("clamp", a, 0.0, DBL_MAX),
                        oracle.binary("add", b, np.array([1.0], np.float32)))
    return oracle.binary("sub", lhs, rhs)


def test_config1_full_size_bitexact(rsl, oracle):
    """c = a*a + b at a [8192,8192], b [8192,1] (uniform, seeded): one fused
    kernel, bit-identical to the oracle.  The 6-op chain: bit-identical to
    the GPU's own eager path; its exp within 2 ulp of the oracle's; the
    oracle's exact ops applied to the GPU's exp give the fused result bit for
    bit (so exp is the only source of difference); and the whole chain within
    1e-6 of the oracle's chain under max|d| / max|true|."""
    n = 8192
    a_np = np.random.default_rng(0).random((n, n), dtype=np.float32)
    b_np = np.random.default_rng(1).random((n, 1), dtype=np.float32)
    a, b = V(rsl, a_np), V(rsl, b_np)
    with rsl.capture_on():
        c = a * a + b
    got = c.numpy()
    want = oracle.binary("add", oracle.binary("mul", a_np, a_np), b_np)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    del got, want, c
    with rsl.capture_on():
        c6 = chain6(rsl, a, b)
    fused = c6.numpy()
    eager = chain6(rsl, a, b).numpy()
    assert np.array_equal(fused.view(np.uint32), eager.view(np.uint32))
    del eager
    e = oracle.unary("exp", a_np)
    e_gpu = rsl.exp(a).numpy()
    assert_within_ulp(e_gpu, e, 2)
    same_exp = _oracle_chain6(oracle, e_gpu, a_np, b_np)
    assert np.array_equal(fused.view(np.uint32), same_exp.view(np.uint32))
    del same_exp, e_gpu
    assert rel_err(fused, _oracle_chain6(oracle, e, a_np, b_np)) <= 1e-6


def test_config2_backward_and_reductions(rsl, oracle):
    """A[16384,16384] + B[1,16384]: A.grad is all ones and B.grad is exactly
    16384 (the dim-0 reduction of the ones gradient); dim reductions of
    normal data within 1e-5 of the oracle."""
    n = 16384
    x_np = np.random.default_rng(3).standard_normal((n, n), dtype=np.float32)
    A = V(rsl, x_np, True)
    B = V(rsl, np.zeros((1, n), np.float32), True)
    (A + B).backward()
    bg = B.grad.numpy()
    assert np.all(bg == np.float32(n))
    ag = A.grad.numpy()
    assert np.all(ag == 1.0)
    del ag
    for op, axis in (("sum", 0), ("sum", 1), ("max", 1)):
        got = getattr(rsl, op)(A, axis).numpy()
        want = oracle.reduce(op, x_np, axis)
        if op == "max":
            assert np.array_equal(got, want)
        else:
            assert rel_err(got, want) <= 1e-5


def test_config3_linear_forward_backward(rsl):
    """Linear fwd + both backward GEMMs at 4096^3 and the skinny
    32x4096x8192 shape through autograd, with a random upstream gradient:
    loss = sum(sum(Y * G, 1), 0) with G normal(0, 0.02) makes dY = G exactly
    (matrix_ops.cpp:8-24 then forms dX = G.W^T and dW = X^T.G).  Sampled rows
    and columns of Y, dX and dW against float64."""
    rng = np.random.default_rng(4)
    for m, k, n in ((4096, 4096, 4096), (32, 8192, 4096)):
        x_np = (rng.standard_normal((m, k)) * 0.02).astype(np.float32)
        w_np = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
        g_np = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
        x, w = V(rsl, x_np, True), V(rsl, w_np, True)
        y = rsl.matmul(x, w)
        loss = rsl.sum(rsl.sum(y * V(rsl, g_np), 1), 0)
        loss.backward()
        rows = rng.choice(m, min(m, 32), replace=False)
        cols = rng.choice(n, 32, replace=False)
        x64, w64, g64 = (t.astype(np.float64) for t in (x_np, w_np, g_np))
        yv = y.numpy()
        assert rel_err(yv[rows], x64[rows] @ w64) <= 1e-4
        assert rel_err(yv[:, cols], x64 @ w64[:, cols]) <= 1e-4
        gx = x.grad.numpy()
        kcols = rng.choice(k, 32, replace=False)
        assert rel_err(gx[rows], g64[rows] @ w64.T) <= 1e-4
        assert rel_err(gx[:, kcols], g64 @ w64[kcols].T) <= 1e-4
        gw = w.grad.numpy()
        wrows = rng.choice(k, 32, replace=False)
        assert rel_err(gw[wrows], x64.T[wrows] @ g64) <= 1e-4
        assert rel_err(gw[:, cols], x64.T @ g64[:, cols]) <= 1e-4


@pytest.mark.parametrize("m,k,n", [(96, 80, 72), (4096, 64, 128), (2048, 256, 256)])
def test_matmul_grad_accumulates_in_gemm_epilogue(rsl, m, k, n):
    """A weight reached twice accumulates its second product in the GEMM
    epilogue; that must equal the fp32 sum of the two separate gradients
    bit for bit (covers the split-K fold with accumulation too)."""
    rng = np.random.default_rng(m + k + n)
    xs = [rng.standard_normal((m, k)).astype(np.float32) for _ in range(2)]
    w_np = (rng.standard_normal((k, n)) * 0.1).astype(np.float32)

    def grad_of(inputs):
        w = V(rsl, w_np, True)
        for x_np in inputs:
            rsl.matmul(V(rsl, x_np, False), w).backward()
        return w.grad.numpy()

    g1, g2, g12 = grad_of(xs[:1]), grad_of(xs[1:]), grad_of(xs)
    assert np.array_equal(g12, g1 + g2)
    want = xs[0].astype(np.float64).T.sum(1, keepdims=True) + xs[1].astype(np.float64).T.sum(
        1, keepdims=True)
    assert rel_err(g12, np.broadcast_to(want, (k, n))) <= 1e-4


_JIT_CHILD = textwrap.dedent("""
    import ctypes as C, json, sys
    import numpy as np
    sys.path.insert(0, sys.argv[1])
    import rushlite_amd as rsl
    from rushlite_amd import abi
    a = rsl.Variable(np.arange(24, dtype=np.float32).reshape(4, 6))
    b = rsl.Variable(np.full((4, 1), 0.25, np.float32))
    with rsl.capture_on():
        c = rsl.exp(a * 0.125) * b - a
    vals = c.numpy()
    n, d = C.c_uint64(), C.c_uint64()
    abi.check(abi.lib().lmp_jit_compiled_count(C.byref(n)))
    abi.check(abi.lib().lmp_jit_disk_loaded_count(C.byref(d)))
    print(json.dumps({"compiled": n.value, "disk": d.value,
                      "bits": vals.view(np.uint32).ravel().tolist()}))
""")


def _jit_child(cache_dir):
    root = str(Path(__file__).resolve().parents[1])
    env = dict(os.environ, LMP_HIP_JIT_CACHE=str(cache_dir))
    print(f"jit disk cache child, cache={cache_dir}", flush=True)
    out = subprocess.run([sys.executable, "-c", _JIT_CHILD, root], env=env,
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    return json.loads(out.stdout.strip().splitlines()[-1])


def test_jit_disk_cache_reused_by_a_new_process(tmp_path):
    """A second process loads the fused kernel the first one compiled; a
    truncated cache file is a miss that recompiles, never a wrong kernel."""
    first = _jit_child(tmp_path)
    assert first["compiled"] >= 1 and first["disk"] == 0
    files = sorted(tmp_path.glob("*.hsaco"))
    assert len(files) == first["compiled"]
    second = _jit_child(tmp_path)
    assert second["compiled"] == 0 and second["disk"] == first["compiled"]
    assert second["bits"] == first["bits"]
    for f in files:
        f.write_bytes(f.read_bytes()[: f.stat().st_size // 2])
    third = _jit_child(tmp_path)
    assert third["compiled"] == first["compiled"] and third["disk"] == 0
    assert third["bits"] == first["bits"]


# ------------------------------------------------- row (reduction) fusion

def _softmax(rsl, x):
    m = rsl.max(x, 1)
    e = rsl.exp(x - m)
    return e / rsl.sum(e, 1)


@pytest.mark.parametrize("shape,dt", [((512, 1000), "float32"), ((32, 10), "float32"),
                                      ((7, 333), "float32"), ((64, 100), "float64"),
                                      ((3, 2048), "float32")], ids=str)
def test_softmax_row_fusion_matches_eager(rsl, shape, dt):
    """Under capture a softmax row (max, sub, exp, sum, div) is one kernel
    whose reductions replay the eager kernels' order: bit-identical to the
    eager softmax.  Rows of 2048 or more are reduced by the eager kernels."""
    rng = np.random.default_rng(shape[1])
    x_np = (rng.standard_normal(shape) * 4).astype(dt)
    x = rsl.Variable(x_np, dtype=getattr(rsl.dtype, dt))
    eager = _softmax(rsl, x).numpy()
    s0 = rsl._stats()
    with rsl.no_grad(), rsl.capture_on():
        p = _softmax(rsl, x)
    got = p.numpy()
    s1 = rsl._stats()
    if shape[1] < 2048:
        assert s1["fused_launches"] - s0["fused_launches"] == 1
        assert s1["eager_launches"] == s0["eager_launches"]
    assert got.dtype == eager.dtype
    assert np.array_equal(got.view(np.uint8), eager.view(np.uint8))
    x64 = x_np.astype(np.float64)
    e64 = np.exp(x64 - x64.max(1, keepdims=True))
    assert rel_err(got, e64 / e64.sum(1, keepdims=True)) <= (1e-6 if dt == "float32" else 1e-14)


@pytest.mark.parametrize("op", ["sum", "max", "min", "prod"])
@pytest.mark.parametrize("shape", [(300, 257), (512, 1000), (5, 3, 12), (9, 4)], ids=str)
def test_captured_reductions_equal_eager(rsl, op, shape):
    """A reduction over the last axis of a captured elementwise chain (with a
    row-broadcast [N] operand) fuses into one row kernel equal to eager."""
    rng = np.random.default_rng(len(shape) * 100 + shape[-1])
    a_np = rng.standard_normal(shape, dtype=np.float32)
    w_np = (1.0 + 0.01 * rng.standard_normal(shape[-1:])).astype(np.float32)
    a, w = V(rsl, a_np), V(rsl, w_np)
    fn = getattr(rsl, op)
    eager = fn(a * w + 0.5, len(shape) - 1).numpy()
    s0 = rsl._stats()
    with rsl.no_grad(), rsl.capture_on():
        r = fn(a * w + 0.5, len(shape) - 1)
    got = r.numpy()
    assert rsl._stats()["fused_launches"] - s0["fused_launches"] == 1
    assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))


@pytest.mark.parametrize("capture", [False, True])
def test_binary_special_values_through_variables(rsl, oracle, capture):
    """Every pair of special values (signed zeros, infinities, NaN, subnormals,
    extremes, neighbours of 1) through Variable binary ops, eager and inside a
    fused kernel (a * 1 and b * 1 feed them, exact for every value), bit for
    bit as the oracle; NaN results compare as NaN only (the sign of a NaN made
    by 0/0 or inf - inf differs between x86 and the GPU)."""
    col, row = SPECIALS.reshape(-1, 1), SPECIALS.reshape(1, -1)
    a, b = V(rsl, col), V(rsl, row)
    for op in ("add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt"):
        fn = getattr(rsl, op)
        with rsl.no_grad(), rsl.capture_on(capture):
            r = fn(a * 1.0, b * 1.0)
        got = r.numpy()
        want = oracle.binary(op, col, row)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), op
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), op


def test_unary_special_values_fused_and_eager(rsl, oracle):
    """Each unary op over the special values (signed zeros, infinities, NaN,
    subnormals, extremes, neighbours of 1): the fused kernel gives the eager
    kernel's bits, NaN results compared as NaN (inside a fused kernel the
    compiler may fold neg(x * 1) into x * -1, which keeps a NaN's sign where a
    separate neg flips it; a NaN's sign carries no value); against the oracle
    NaN at the same positions, neg / abs / sqrt / ReLU bit for bit, the
    transcendentals within 2 ulp with the same signed zeros."""
    x = V(rsl, SPECIALS.reshape(1, -1))
    exact = {"neg": rsl.neg, "abs": rsl.abs, "sqrt": rsl.sqrt}
    approx = {"exp": rsl.exp, "log": rsl.log, "sin": rsl.sin, "cos": rsl.cos, "tan": rsl.tan}
    for name, fn in list(exact.items()) + list(approx.items()) + [("clamp", None)]:
        call = (lambda t: rsl.clamp(t, 0, DBL_MAX)) if name == "clamp" else fn
        eager = call(x * 1.0).numpy()
        with rsl.no_grad(), rsl.capture_on():
            r = call(x * 1.0)
        fused = r.numpy()
        fnan = np.isnan(eager)
        assert np.array_equal(np.isnan(fused), fnan), name
        assert np.array_equal(fused[~fnan].view(np.uint32), eager[~fnan].view(np.uint32)), name
        p0, p1 = (0.0, DBL_MAX) if name == "clamp" else (0.0, 0.0)
        want = oracle.unary(name, SPECIALS.reshape(1, -1), p0, p1)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(eager), nan), name
        if name in approx:
            assert_within_ulp(eager[~nan], want[~nan], 2, name)
        else:
            assert np.array_equal(eager[~nan].view(np.uint32), want[~nan].view(np.uint32)), name


@pytest.mark.parametrize("length", [37, 1000])
def test_captured_max_min_special_values_equal_eager(rsl, length):
    """max/min over the last axis of rows holding infinities, NaN, signed zeros
    (both signs tying at the extreme included) and all -inf: the fused row
    kernel gives the eager kernel's bits, as both combine in one order."""
    a_np = special_rows(length, np.random.default_rng(length))
    a = V(rsl, a_np)
    for op in ("max", "min"):
        fn = getattr(rsl, op)
        eager = fn(a * 1.0, 1).numpy()
        s0 = rsl._stats()
        with rsl.no_grad(), rsl.capture_on():
            r = fn(a * 1.0, 1)
        got = r.numpy()
        assert rsl._stats()["fused_launches"] - s0["fused_launches"] == 1
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), op


@pytest.mark.parametrize("dtype", ["float32", "float64"])
def test_captured_reduction_used_elementwise_after_signed_zero_tie(rsl, dtype):
    """A max/min whose +0 and -0 tie at the extreme, used by elementwise ops in
    the same fused row kernel: every lane must go on with the value the eager
    kernel stores (lane 0's after the butterfly; other lanes can hold the
    other zero), so min(x) / (1 + x*x) keeps one zero sign along the row, as
    eager.  Found by a wider random run (a float64 row of 103 -0 and 7 +0)."""
    dt = np.float64 if dtype == "float64" else np.float32
    kind = getattr(rsl.dtype, dtype)
    rows = np.ones((6, 128), dt)
    rows[0, 0:64:2] = -0.0
    rows[0, 1:64:2] = 0.0                       # -0 in even lanes, +0 in odd
    rows[1, :64] = 0.0
    rows[1, 5] = -0.0                           # one -0 among +0
    rows[2, :] = -0.0
    rows[2, 77] = 0.0                           # one +0 in the second half
    rows[3, 64:] = 0.0
    rows[3, 100:128:3] = -0.0                   # the tie in the second half
    rows[4, ::5] = -0.0
    rows[4, 1::5] = 0.0
    rows[5, :] = -1.0                           # no zero at the minimum
    for op in ("max", "min"):
        src = -rows if op == "max" else rows
        a = rsl.Variable(src, dtype=kind)
        fn = getattr(rsl, op)
        eager = (fn(a, 1) / (a * a + 1.0)).numpy()
        with rsl.no_grad(), rsl.capture_on():
            r = fn(a, 1) / (a * a + 1.0)
        got = r.numpy()
        assert np.array_equal(got.view(np.uint8), eager.view(np.uint8)), op
        for i in range(5):  # one zero sign along each tying row
            assert len(set(np.signbit(got[i]).tolist())) == 1, (op, i)


@pytest.mark.parametrize("capture", [False, True])
def test_empty_tensors(rsl, oracle, capture):
    """Variables with a zero extent, eager and under capture_on: elementwise
    results are empty, a reduction over the empty axis gives the identity per
    output as the oracle (cpu/reduct.cpp:14-19), over another axis an empty
    result, and a product with K = 0 gives zeros."""
    e_np = np.zeros((3, 0), np.float32)
    e = V(rsl, e_np)
    with rsl.capture_on(capture):
        elem = e * 2.0 + 1.0
        reds = {op: getattr(rsl, op)(e * 2.0 + 1.0, 1) for op in ("sum", "max", "min", "prod")}
        across = rsl.sum(e + 1.0, 0)
        mm = rsl.matmul(e, V(rsl, np.zeros((0, 4), np.float32)))
    assert list(elem.shape) == [3, 0] and elem.numpy().size == 0
    for op, r in reds.items():
        want = oracle.reduce(op, e_np, 1)
        got = r.numpy()
        assert got.shape == want.shape and np.array_equal(got.view(np.uint32),
                                                          want.view(np.uint32)), op
    assert list(across.shape) == [1, 0]
    assert np.array_equal(mm.numpy(), np.zeros((3, 4), np.float32))


def test_loss_row_chain_fuses(rsl):
    """The README loss's row part, sum(-y * log(p + 1e-3), 1), is one kernel."""
    rng = np.random.default_rng(8)
    p, y = V(rsl, rng.random((32, 10), dtype=np.float32)), V(rsl, rng.random((32, 10), dtype=np.float32))
    eager = rsl.sum(-y * rsl.log(p + 1e-3), 1).numpy()
    s0 = rsl._stats()
    with rsl.no_grad(), rsl.capture_on():
        r = rsl.sum(-y * rsl.log(p + 1e-3), 1)
    got = r.numpy()
    assert rsl._stats()["fused_launches"] - s0["fused_launches"] == 1
    assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))


def _softmax_loss(rsl, z, y):
    m = rsl.max(z, 1)
    sh = z - m
    e = rsl.exp(sh)
    s = rsl.sum(e, 1)
    p = e / s
    q = p + 1e-3
    lg = rsl.log(q)
    ny = -y
    t = ny * lg
    r = rsl.sum(t, 1)
    return r, [m, sh, e, s, p, q, lg, ny, t]


@pytest.mark.parametrize("shape", [(512, 1000), (32, 10), (7, 333)], ids=str)
def test_softmax_loss_with_autograd_is_one_kernel(rsl, shape):
    """With autograd on, every forward value is held by its Variable for the
    backward pass.  Under capture the whole softmax + loss row chain is still
    one kernel: the values autograd holds are stored by that kernel as extra
    outputs.  Every stored value, the loss and the gradient equal the eager
    ones bit for bit."""
    rng = np.random.default_rng(shape[1] + 3)
    z_np = (rng.standard_normal(shape) * 3).astype(np.float32)
    y_np = rng.random(shape, dtype=np.float32)

    def run(captured):
        z = rsl.Variable(z_np, requires_grad=True)
        y = rsl.Variable(y_np)
        s0 = rsl._stats()
        with rsl.capture_on(captured):
            r, vals = _softmax_loss(rsl, z, y)
        r.realize()
        s1 = rsl._stats()
        assert all(not rsl._is_deferred(v) for v in vals)
        out = [r.numpy()] + [v.numpy() for v in vals]
        rsl.sum(r, 0).backward()
        return out, z.grad.numpy(), (s1["fused_launches"] - s0["fused_launches"],
                                     s1["eager_launches"] - s0["eager_launches"])

    eager, g_eager, _ = run(False)
    fused, g_fused, (nf, ne) = run(True)
    assert (nf, ne) == (1, 0)
    # The backward of the row chain, from the [1, 1] seed through both row
    # sums and the max, is one row kernel too (after the loss's column sum).
    z = rsl.Variable(z_np, requires_grad=True)
    y = rsl.Variable(y_np)
    with rsl.capture_on():
        r, _ = _softmax_loss(rsl, z, y)
    loss = rsl.sum(r, 0)
    s0 = rsl._stats()
    loss.backward()
    s1 = rsl._stats()
    assert (s1["fused_launches"] - s0["fused_launches"], s1["eager_launches"] - s0["eager_launches"]) == (1, 0)
    assert np.array_equal(z.grad.numpy().view(np.uint32), g_eager.view(np.uint32))
    assert np.all(loss.grad.numpy() == 1.0)
    for i, (a, b) in enumerate(zip(fused, eager)):
        assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    assert np.array_equal(g_fused.view(np.uint32), g_eager.view(np.uint32))


@pytest.mark.parametrize("dt", ["float32", "float64"])
def test_fused_abs_and_clamp_backward(rsl, dt):
    """The backward functors of abs and clamp are fusible nodes (the backward
    pass runs captured): the gradient equals the functors' definition --
    g strictly inside (lo, hi), sign(x) * g with 0 at x == 0 and at NaN -- bit
    for bit, at 0, -0, the bounds, infinities and NaN."""
    rng = np.random.default_rng(21)
    x_np = rng.standard_normal((96, 130)).astype(dt)
    flat = x_np.reshape(-1)
    flat[:8] = [0.0, -0.0, 0.5, -0.5, np.inf, -np.inf, np.nan, 1e-30]
    g_np = rng.standard_normal((96, 130)).astype(dt)
    x = rsl.Variable(x_np, dtype=getattr(rsl.dtype, dt), requires_grad=True)
    g = rsl.Variable(g_np, dtype=getattr(rsl.dtype, dt))
    y = rsl.clamp(x, -0.5, 0.5) * g + rsl.clamp(x, 0.0, DBL_MAX) * (g * 2.0) + rsl.abs(x) * g
    rsl.sum(rsl.sum(y, 1), 0).backward()
    got = x.grad.numpy()
    zero = np.zeros((), dt)
    with np.errstate(invalid="ignore"):
        t1 = np.where((x_np > -0.5) & (x_np < 0.5), g_np, zero)
        hi = np.array(DBL_MAX if dt == "float64" else np.inf, dt)
        t2 = np.where((x_np > 0) & (x_np < hi), g_np * np.array(2.0, dt), zero)
        t3 = np.where(x_np > 0, g_np, np.where(x_np < 0, -g_np, zero))
    terms = {"c1": t1, "c2": t2, "a": t3}
    view = np.uint32 if dt == "float32" else np.uint64
    # Accumulation order of the three terms follows the graph; each term is
    # exact, so any order of two IEEE adds from +0 is checked by trying all.
    import itertools
    ok = False
    for order in itertools.permutations(terms):
        acc = zero + terms[order[0]]
        for k in order[1:]:
            acc = acc + terms[k]
        ok |= np.array_equal(acc.view(view), got.view(view))
    assert ok


def test_held_interior_value_is_stored_by_the_same_kernel(rsl):
    """An interior value that something else holds is an extra output of the
    root's kernel when it has the root's shape, and a separate kernel (a leaf)
    when it is broadcast, as b + 1 here."""
    rng = np.random.default_rng(11)
    a_np = rng.random((300, 128), dtype=np.float32)
    b_np = rng.random((300, 1), dtype=np.float32)
    a, b = V(rsl, a_np), V(rsl, b_np)
    eager = [(a * b), (b + 1.0), (a * b) / (b + 1.0) - a]
    s0 = rsl._stats()["fused_launches"]
    with rsl.capture_on():
        t = a * b
        u = b + 1.0
        c = t / u - a
    c.realize()
    assert rsl._stats()["fused_launches"] - s0 == 2
    assert not rsl._is_deferred(t) and not rsl._is_deferred(u)
    for got, want in zip([t, u, c], eager):
        assert np.array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32))
    # float64, indexed path (no float4 plan)
    a64, b64 = V(rsl, a_np.astype(np.float64)), V(rsl, b_np.astype(np.float64))
    want = [(a64 * a64), (a64 * a64) * b64 + 1.0]
    s0 = rsl._stats()["fused_launches"]
    with rsl.capture_on():
        t = a64 * a64
        c = t * b64 + 1.0
    c.realize()
    assert rsl._stats()["fused_launches"] - s0 == 1
    for got, w in zip([t, c], want):
        assert np.array_equal(got.numpy().view(np.uint64), w.numpy().view(np.uint64))


def test_long_held_chain_splits_into_few_regions(rsl):
    """48 captured ops whose every intermediate is held (as autograd holds
    forward values) exceed one kernel's output limit: the chain splits into a
    few regions, each storing its part, and every value equals eager."""
    rng = np.random.default_rng(13)
    a, b = V(rsl, rng.random((64, 96), dtype=np.float32)), V(rsl, rng.random((64, 96), dtype=np.float32))

    def chain():
        held, t = [], a
        for i in range(32):
            t = t * b + a if i % 2 == 0 else t - b
            held.append(t)
        return held

    eager = [t.numpy() for t in chain()]
    s0 = rsl._stats()["fused_launches"]
    with rsl.capture_on():
        held = chain()
    held[-1].realize()
    assert rsl._stats()["fused_launches"] - s0 <= 4
    for i, (t, w) in enumerate(zip(held, eager)):
        assert not rsl._is_deferred(t), i
        assert np.array_equal(t.numpy().view(np.uint32), w.view(np.uint32)), i


def test_broadcast_add_backward_folds_and_accumulates_in_place(rsl):
    """The backward of A + B + C (B [1, N], C [M, 1]) reduces the ones seed
    over each broadcast axis: a sum of ones is exact in any order, so it is
    folded to a constant instead of a pass over the seed, and the gradients
    stay constants until read.  Accumulation keeps the gradient tensors'
    identity throughout -- the in-place accumulation Lamp3 tests in
    autograd_tests.cpp:487-514."""
    m, n = 300, 257
    rng = np.random.default_rng(27)
    A = rsl.Variable(rng.standard_normal((m, n)).astype(np.float32), requires_grad=True)
    B = rsl.Variable(rng.standard_normal((1, n)).astype(np.float32), requires_grad=True)
    C = rsl.Variable(rng.standard_normal((m, 1)).astype(np.float32), requires_grad=True)
    (A + B + C).backward()
    held = [v.grad for v in (A, B, C)]  # handles taken before any read
    s0 = rsl._stats()
    y = A + B + C
    y.backward()
    s1 = rsl._stats()
    # The gradients are constants until read: the second backward launches
    # nothing (the forward's two adds are eager), and the held handles see the
    # accumulated values.
    assert s1["eager_launches"] - s0["eager_launches"] == 2
    assert s1["fused_launches"] - s0["fused_launches"] == 0
    assert np.all(held[0].numpy() == 2.0)
    assert np.all(held[1].numpy() == 2.0 * m) and np.all(held[2].numpy() == 2.0 * n)
    assert np.all(y.grad.numpy() == 1.0)
    # Read (materialised) gradients accumulate in place: one fused kernel each
    # computes g + the pending term into the existing buffer.
    ptrs = [rsl._storage_ptr(v.grad) for v in (A, B, C)]
    s0 = rsl._stats()
    (A + B + C).backward()
    s1 = rsl._stats()
    assert [rsl._storage_ptr(v.grad) for v in (A, B, C)] == ptrs
    assert s1["fused_launches"] - s0["fused_launches"] == 3
    assert np.all(held[0].numpy() == 3.0)
    assert np.all(B.grad.numpy() == 3.0 * m) and np.all(C.grad.numpy() == 3.0 * n)


def test_realize_all_groups_independent_updates(rsl):
    """realize_all runs the pending elementwise updates of several tensors
    (different shapes, float4 and indexed plans, float32 and float64, as an
    optimizer's per-parameter p - lr * g) as one kernel, each equal to
    realising it alone; a row reduction among them runs on its own, and
    updates sharing a pending subexpression fall back to one by one."""
    rng = np.random.default_rng(23)
    shapes = [(256, 64), (64,), (64, 10), (10,), (33, 7)]
    ps = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    gs = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]

    def updates(dt=np.float32):
        out = []
        rdt = rsl.dtype.float64 if dt == np.float64 else rsl.dtype.float32
        for p_np, g_np in zip(ps, gs):
            p, g = rsl.Variable(p_np.astype(dt), dtype=rdt), rsl.Variable(g_np.astype(dt), dtype=rdt)
            with rsl.capture_on():
                out.append(p - 1e-3 * g)
        return out

    want = [u.numpy() for u in updates()]
    want64 = [u.numpy() for u in updates(np.float64)]
    got = updates()
    s0 = rsl._stats()["fused_launches"]
    rsl.realize_all(got)
    assert rsl._stats()["fused_launches"] - s0 == 1
    for g, w in zip(got, want):
        assert not rsl._is_deferred(g)
        assert np.array_equal(g.numpy().view(np.uint32), w.view(np.uint32))
    # float64 updates join the group; a row reduction runs on its own
    mixed = updates() + updates(np.float64)
    x = rsl.Variable(rng.standard_normal((8, 30)).astype(np.float32))
    with rsl.capture_on():
        row = rsl.sum(x * 2.0, 1)
    want_row = rsl.sum(x * 2.0, 1).numpy()
    s0 = rsl._stats()["fused_launches"]
    rsl.realize_all(mixed + [row])
    assert rsl._stats()["fused_launches"] - s0 == 2
    for g, w in zip(mixed[:len(shapes)], want):
        assert np.array_equal(g.numpy().view(np.uint32), w.view(np.uint32))
    for g, w in zip(mixed[len(shapes):], want64):
        assert np.array_equal(g.numpy().view(np.uint64), w.view(np.uint64))
    assert np.array_equal(row.numpy(), want_row)
    # two roots sharing a pending value: realised one by one, still correct
    a = rsl.Variable(ps[0])
    with rsl.capture_on():
        t = a * 3.0
        r1, r2 = t + 1.0, t - 1.0
    rsl.realize_all([r1, r2])
    assert np.array_equal(r1.numpy(), (ps[0] * np.float32(3)) + np.float32(1))
    assert np.array_equal(r2.numpy(), (ps[0] * np.float32(3)) - np.float32(1))


def test_leaf_region_storing_a_shared_node(rsl):
    """Rows of 4096 are too long for a row kernel, so the row sum L below is a
    leaf of c's region, and realising it first reaches n, which c's region
    also holds; c's region is then rebuilt with n as a leaf.  Values equal
    eager."""
    rng = np.random.default_rng(12)
    a_np = rng.standard_normal((4, 4096), dtype=np.float32)
    a = V(rsl, a_np)
    n_e = a * 2.0
    want = [n_e.numpy(), (n_e - rsl.sum(n_e, 1)).numpy()]
    with rsl.capture_on():
        n = a * 2.0
        c = n - rsl.sum(n, 1)
    got = [n.numpy(), c.numpy()]
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
    # Here L's own region is a row kernel and stores n as one of its outputs
    # (the [2, 1, 200] operand d, whose rows are not evenly spaced in the
    # [2, 64, 200] row layout, keeps c's region off the row path).
    a_np = rng.standard_normal((2, 64, 200), dtype=np.float32)
    d_np = rng.standard_normal((2, 1, 200), dtype=np.float32)
    a, d = V(rsl, a_np), V(rsl, d_np)
    n_e = a * 2.0
    want = [n_e.numpy(), ((n_e - rsl.sum(n_e, 2)) * d).numpy()]
    s0 = rsl._stats()["fused_launches"]
    with rsl.capture_on():
        n = a * 2.0
        c = (n - rsl.sum(n, 2)) * d
    got = [c.numpy(), n.numpy()][::-1]
    assert rsl._stats()["fused_launches"] - s0 == 2
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("x_grad", [True, False], ids=["x_grad", "x_const"])
@pytest.mark.parametrize("dt", ["float32", "float64"])
@pytest.mark.parametrize("m,k,n", [(32, 256, 64), (20, 70, 10), (512, 2048, 2048), (64, 130, 33)],
                         ids=str)
def test_linear_relu_node_matches_linear_then_relu(rsl, m, k, n, dt, x_grad):
    """linear_relu (Sequential's Linear -> ReLU as one node, ReLU in the GEMM
    epilogue for float32) gives the values and the x, w, b gradients of linear
    followed by clamp(., 0, DBL_MAX), bit for bit, with infinities and NaN in
    x (the backward masks by the output, which must equal masking by the
    input).  With x needing no gradient (a first layer) the float32 weight and
    bias gradients apply ReLU's mask inside the column-sum GEMM."""
    rng = np.random.default_rng(m * k + n + 1)
    x_np = rng.standard_normal((m, k)).astype(dt)
    x_np[0, :3] = [np.inf, -np.inf, np.nan] if m > 1 else x_np[0, :3]
    w_np = rng.standard_normal((k, n)).astype(dt)
    b_np = rng.standard_normal(n).astype(dt)
    view = np.uint32 if dt == "float32" else np.uint64
    outs, grads = [], []
    for fused in (True, False):
        x = rsl.Variable(x_np, dtype=getattr(rsl.dtype, dt), requires_grad=x_grad)
        w = rsl.Variable(w_np, dtype=getattr(rsl.dtype, dt), requires_grad=True)
        b = rsl.Variable(b_np, dtype=getattr(rsl.dtype, dt), requires_grad=True)
        y = rsl._C.linear_relu(x, w, b) if fused else rsl.clamp(rsl.linear(x, w, b), 0, DBL_MAX)
        (y * 0.5 + 1.0).sum(1).sum(0).backward()
        outs.append(y.numpy())
        grads.append(([x.grad.numpy()] if x_grad else []) + [w.grad.numpy(), b.grad.numpy()])
    assert np.array_equal(outs[0].view(view), outs[1].view(view))
    for g0, g1 in zip(*grads):
        assert np.array_equal(g0.view(view), g1.view(view))


def test_sequential_fuses_linear_relu_pairs(rsl):
    """Sequential runs Linear -> ReLU as one node; a model whose ReLU is a
    subclass (not fused) gives the same loss and gradients bit for bit."""
    from rushlite_amd.nets import layers

    class PlainReLU(layers.ReLU):
        pass

    rng = np.random.default_rng(17)
    x_np = rng.standard_normal((48, 96)).astype(np.float32)
    ws = [rng.standard_normal((96, 80)).astype(np.float32), rng.standard_normal((80, 10)).astype(np.float32)]
    bs = [rng.standard_normal(80).astype(np.float32), rng.standard_normal(10).astype(np.float32)]
    results = []
    for relu_cls in (layers.ReLU, PlainReLU):
        model = layers.Sequential([layers.Linear(96, 80), relu_cls(), layers.Linear(80, 10)])
        for i, idx in enumerate((0, 2)):
            model.params[f"{idx}.weights"] = rsl.Variable(ws[i], requires_grad=True)
            model.params[f"{idx}.bias"] = rsl.Variable(bs[i], requires_grad=True)
        s0 = rsl._stats()["eager_launches"]
        out = model(rsl.Variable(x_np))
        launches = rsl._stats()["eager_launches"] - s0
        out.sum(1).sum(0).backward()
        results.append((out.numpy(), [p.grad.numpy() for _, p in model.named_parameters()], launches))
    (o0, g0, n0), (o1, g1, n1) = results
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    for a, b in zip(g0, g1):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert n0 == n1 - 1  # the ReLU launch is gone


@pytest.mark.parametrize("m,k,n", [(32, 256, 64), (20, 70, 10), (512, 2048, 2048), (64, 130, 33)],
                         ids=str)
def test_linear_op_matches_matmul_plus_bias(rsl, m, k, n):
    """rsl.linear (Linear's forward: one GEMM with the bias in its epilogue)
    gives the values and the x and w gradients of matmul followed by the
    broadcast add, bit for bit.  Its bias gradient comes from the weight
    gradient's GEMM (column sums of the output gradient, summed in the GEMM's
    own order on the single-launch path), so it is held to the reductions'
    bar against float64 instead."""
    rng = np.random.default_rng(m * k + n)
    x_np = rng.standard_normal((m, k)).astype(np.float32)
    w_np = rng.standard_normal((k, n)).astype(np.float32)
    b_np = rng.standard_normal(n).astype(np.float32)
    outs, grads = [], []
    for fused in (True, False):
        x = rsl.Variable(x_np, requires_grad=True)
        w = rsl.Variable(w_np, requires_grad=True)
        b = rsl.Variable(b_np, requires_grad=True)
        y = rsl.linear(x, w, b) if fused else rsl.matmul(x, w) + b
        (rsl.exp(y * 0.01) * 2.0).sum(1).sum(0).backward()
        outs.append(y.numpy())
        grads.append([x.grad.numpy(), w.grad.numpy(), b.grad.numpy()])
        gy = (rsl.exp(y * 0.01) * 2.0 * 0.01).numpy().astype(np.float64)
    assert np.array_equal(outs[0], outs[1])
    for g0, g1 in zip(grads[0][:2], grads[1][:2]):
        assert np.array_equal(g0, g1)
    db = gy.sum(0)
    for g in (grads[0][2], grads[1][2]):
        assert np.max(np.abs(g - db)) <= 1e-5 * np.max(np.abs(db))
