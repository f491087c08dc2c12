"""Whole-step HIP graphs (rsl.hip.Graph): a captured step replays the exact
kernels of the eager step, so every replay must equal the eager step bit for
bit.  Each replay is checked against an eager twin run in between replays,
with unrelated eager allocations and synchronisations interleaved, so a graph
that wrote outside its own pool or left stale state would show up.  The
reference has no graphs; the eager path these are compared with is itself
held to the oracle in test_gpu_framework.py.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rsl(hip):
    import rushlite_amd
    return rushlite_amd


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


def _problem(dims, batch, seed=2):
    rng = np.random.default_rng(seed)
    x = rng.random((batch, dims[0]), dtype=np.float32)
    y = rng.random((batch, dims[-1]), dtype=np.float32)
    ws = [rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32)
          for i in range(len(dims) - 1)]
    bs = [rng.standard_normal(dims[i + 1], dtype=np.float32) for i in range(len(dims) - 1)]
    return x, y, ws, bs


def _stepper(rsl, model, x, y, lr=1e-3, fused_update=False):
    @rsl.capture()
    def forward(inp):
        return model(inp)

    def step():
        probs = forward(x)
        loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        with rsl.capture_on(fused_update):
            for name, p in list(model.named_parameters()):
                model.params[name] = rsl.Variable(p.data - lr * p.grad, requires_grad=True)
        loss.realize()  # inside a capture, so each replay recomputes it
        return loss
    return step


def _params(model):
    return {n: p.numpy() for n, p in model.named_parameters()}


# README MLP (config 0); a wider net whose GEMMs take the split-K and
# register-direct paths (batch 32, K up to 1024).
CASES = [((256, 64, 10), 32), ((1024, 512, 256, 10), 32)]


def test_graph_replays_equal_eager_steps_at_config4_size(rsl):
    """Config 4 (batch 512, 4096-4096-4096-1000, x normal(0, 1), one-hot y):
    the captured step replays the LDS-tile GEMMs with their split-K folds, the
    paired weight and input gradient launches and the grouped update.
    Parameters at a 1/64 scale, so the gradients are dense (at randn(0, 1) the
    softmax is one-hot and every gradient is zero); the loss must equal the
    eager twin's at every replay and the parameters after the last."""
    dims, batch = (4096, 4096, 4096, 1000), 512
    rng = np.random.default_rng(5)
    x_np = rng.standard_normal((batch, dims[0]), dtype=np.float32)
    y_np = np.zeros((batch, dims[-1]), np.float32)
    y_np[np.arange(batch), rng.integers(0, dims[-1], batch)] = 1.0
    ws = [rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32) / np.float32(64)
          for i in range(len(dims) - 1)]
    bs = [rng.standard_normal(dims[i + 1], dtype=np.float32) / np.float32(64)
          for i in range(len(dims) - 1)]
    eager = _mlp(rsl, ws, bs)
    graphed = _mlp(rsl, ws, bs)
    xe, ye = rsl.Variable(x_np), rsl.Variable(y_np)
    xg, yg = rsl.Variable(x_np), rsl.Variable(y_np)
    step_e = _stepper(rsl, eager, xe, ye, fused_update=True)
    step_g = _stepper(rsl, graphed, xg, yg, fused_update=True)
    l_e, l_g = step_e(), step_g()
    rsl.realize_all(p for _, p in eager.named_parameters())
    rsl.realize_all(p for _, p in graphed.named_parameters())
    assert np.array_equal(l_e.numpy(), l_g.numpy())
    graph = rsl.hip.Graph()
    with graph.capture(carry=graphed):
        loss_g = step_g()
    losses = []
    for i in range(4):
        graph.replay()
        l_e = step_e()
        rsl.realize_all(p for _, p in eager.named_parameters())
        got, want = loss_g.numpy(), l_e.numpy()
        assert np.array_equal(got, want), (i, got, want)
        losses.append(float(want.ravel()[0]))
    assert losses[-1] < losses[0]  # the dense gradients move the loss
    pg, pe = _params(graphed), _params(eager)
    for name in pe:
        assert np.array_equal(pg[name], pe[name]), name


@pytest.mark.parametrize("fused_update", [False, True], ids=["eager_sgd", "fused_sgd"])
@pytest.mark.parametrize("dims,batch", CASES)
def test_graph_replays_equal_eager_steps(rsl, dims, batch, fused_update):
    """With the SGD update eager the capture ends with a copy of each new
    parameter into the buffer the graph reads; with the update captured it is
    computed straight into that buffer.  Both must equal the eager steps."""
    x_np, y_np, ws, bs = _problem(dims, batch)
    eager = _mlp(rsl, ws, bs)
    graphed = _mlp(rsl, ws, bs)
    xe, ye = rsl.Variable(x_np), rsl.Variable(y_np)
    xg, yg = rsl.Variable(x_np), rsl.Variable(y_np)
    step_e = _stepper(rsl, eager, xe, ye, fused_update=fused_update)
    step_g = _stepper(rsl, graphed, xg, yg, fused_update=fused_update)

    # step 1: both eager (compiles every kernel the capture will record)
    l_e, l_g = step_e(), step_g()
    assert np.array_equal(l_e.numpy(), l_g.numpy())

    graph = rsl.hip.Graph()
    with graph.capture(carry=graphed):
        loss_g = step_g()
    assert graph.captured
    # a captured update writes the parameters in place: no copy-back buffers
    held = graph._hold[0]
    same = [rsl._storage_ptr(p.data) == rsl._storage_ptr(held[n].data)
            for n, p in graphed.named_parameters()]
    assert all(same) == fused_update and any(same) == fused_update

    scratch = []
    for i in range(6):
        graph.replay()
        l_e = step_e()
        # unrelated eager work and host round trips between replays
        scratch.append(rsl.Variable(np.full((64, 64), float(i), np.float32)) * 2.0)
        rsl.hip.sync()
        assert np.array_equal(loss_g.numpy(), l_e.numpy()), i
        pg, pe = _params(graphed), _params(eager)
        for name in pe:
            assert np.array_equal(pg[name], pe[name]), (i, name)
    for i, t in enumerate(scratch):
        assert np.all(t.numpy() == 2.0 * i)


def test_graph_reads_inputs_updated_in_place(rsl):
    rng = np.random.default_rng(5)
    a_np = rng.random((256, 512), dtype=np.float32)
    b_np = rng.random((256, 1), dtype=np.float32)
    a, b = rsl.Variable(a_np), rsl.Variable(b_np)
    graph = rsl.hip.Graph()
    with graph.capture():
        with rsl.capture_on():
            c = rsl.exp(a) * b - rsl.clamp(a, 0, 1e30) / (b + 1)
        c.realize()
    for trial in range(3):
        new_a = rng.random((256, 512), dtype=np.float32)
        a.data.copy(rsl.Variable(new_a).data)
        junk = [rsl.Variable(np.ones((128, 128), np.float32)) + float(k) for k in range(4)]
        graph.replay()
        with rsl.capture_on():
            want = rsl.exp(a) * b - rsl.clamp(a, 0, 1e30) / (b + 1)
        assert np.array_equal(c.numpy(), want.numpy()), trial
        assert all(np.all(j.numpy() == 1.0 + k) for k, j in enumerate(junk))


def test_capture_rejects_host_round_trips_and_recovers(rsl):
    a = rsl.Variable(np.ones((8, 8), np.float32))
    graph = rsl.hip.Graph()
    with pytest.raises(RuntimeError, match="graph is being captured"):
        with graph.capture():
            b = a * 3.0
            b.tolist()  # device -> host inside a capture
    assert not graph.captured
    with pytest.raises(RuntimeError, match="graph is being captured"):
        with rsl.hip.Graph().capture():
            rsl.Variable(np.zeros((4, 4), np.float32))  # host -> device
    # eager work after aborted captures
    c = a * 2.0 + 1.0
    assert np.all(c.numpy() == 3.0)
    # a graph cannot be captured twice
    g = rsl.hip.Graph()
    with g.capture():
        d = a + 1.0
    with pytest.raises(RuntimeError, match="already captured"):
        with g.capture():
            pass
    g.replay()
    assert np.all(d.numpy() == 2.0)


def test_graph_memory_returns_after_release(rsl):
    """Dropping the graph and its outputs returns its pool to HIP; the same
    capture can then be repeated without growth."""
    import gc
    a = rsl.Variable(np.ones((1024, 1024), np.float32))

    def once():
        g = rsl.hip.Graph()
        with g.capture():
            out = (a * 2.0) + 1.0
        g.replay()
        v = out.numpy()
        del g, out
        gc.collect()
        return v

    first = once()
    base = rsl._stats()["pool_device_mallocs"]
    for _ in range(3):
        assert np.all(once() == first)
    # each capture grows its own pool by one segment and frees it afterwards
    assert rsl._stats()["pool_device_mallocs"] - base == 3


@pytest.mark.parametrize("capture_on", [False, True], ids=["eager_ops", "fused_ops"])
@pytest.mark.parametrize("shape", [(64, 128), (33, 7)], ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("seed", range(4))
def test_random_program_graph_replays_equal_eager(rsl, seed, shape, capture_on):
    """A random program of the differential suite (broadcast binary ops,
    unary ops, reductions, matmul, transpose), forward and backward, captured
    into a graph; after the inputs are updated in place, every replay equals
    an eager run on the new inputs bit for bit, output and every gradient."""
    import test_gpu_graphs as TG
    leaves, steps, shapes = TG.make_program_rc(seed, *shape)
    rng = np.random.default_rng(1000 + seed)
    lv = [rsl.Variable(rng.uniform(-1, 1, s).astype(np.float32), requires_grad=True)
          for s in leaves]
    base = TG.lamp_ops(rsl, rsl.dtype.float32)
    consts = {v: rsl.Variable(np.array([v], np.float32)) for v in (1.0, 0.5)}

    class ops(base):  # constants made before the capture: no upload inside it
        @staticmethod
        def const(like, v):
            return consts[v]

    def step():
        for v in lv:
            v.zero_grad()
        with rsl.capture_on(capture_on):
            out = TG.run(ops, lv, steps, shapes)
        out.backward()
        for v in lv:
            v.grad.realize()
        out.realize()
        return out

    step()  # compiles every kernel the capture records
    graph = rsl.hip.Graph()
    with graph.capture():
        out_g = step()
    grads_g = [v.grad for v in lv]
    for rep in range(3):
        new = [np.random.default_rng(7 * rep + seed).uniform(-1, 1, s).astype(np.float32)
               for s in leaves]
        for v, a in zip(lv, new):
            v.data.copy(rsl.Variable(a).data)
        graph.replay()
        ev = [rsl.Variable(a, requires_grad=True) for a in new]
        with rsl.capture_on(capture_on):
            oe = TG.run(ops, ev, steps, shapes)
        oe.backward()
        assert np.array_equal(out_g.numpy(), oe.numpy()), rep
        for i, (g, v) in enumerate(zip(grads_g, ev)):
            assert np.array_equal(g.numpy(), v.grad.numpy()), (rep, i)
