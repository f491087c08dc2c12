"""Wider randomized runs of the GPU parity checks (a GPU box; not collected by
pytest).  Each suite draws many more cases than the committed tests from the
same generators and checks them to the same bars, printing a progress line
every few dozen cases and every mismatch:

    python tests/fuzz_wide.py programs 100 200   # random programs, seeds 100..199
    python tests/fuzz_wide.py gemm 888 3000      # random GEMM shapes (+ 100 Linear backward pairs)
    python tests/fuzz_wide.py strided 51 1500    # strided, offset operands; padding poisoned
    python tests/fuzz_wide.py ops 31 600         # reductions (and 2000 broadcast binaries)
    python tests/fuzz_wide.py typed 41 400       # bool / int / float64 GEMM, reduce, binary
    python tests/fuzz_wide.py noalloc 61 400     # the no-allocation GEMM against the allocating one
    python tests/fuzz_wide.py mlp 71 300         # one training step of random MLPs against the oracle
    python tests/fuzz_wide.py graphs 81 100      # random MLP steps in HIP graphs against eager twins
    python tests/fuzz_wide.py specials 91 600    # fused against eager on special-value inputs
    python tests/fuzz_wide.py bits 101 600       # captured programs against eager, bit for bit
    python tests/fuzz_wide.py copies 111 400     # host-device copies of random sizes and offsets
    python tests/fuzz_wide.py held 121 500       # captured programs with intermediates held, bit for bit
    python tests/fuzz_wide.py large 131 100      # GEMMs of 2^30+ multiply-adds, sampled rows and columns

The generators and checks are the committed tests' own (test_gpu_graphs,
test_gpu_hip_graph, test_gpu_kernels, test_gpu_typed); `strided` adds GEMMs
whose operands sit at odd offsets inside wider rows filled with NaN, whose
output rows are wider than N and prefilled with a sentinel: no NaN may reach
C and no element outside C may change.
"""
import sys
import time
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE))

from rushlite_amd import abi  # noqa: E402
from _helpers import rel_err  # noqa: E402

T0 = time.time()
COUNTS = {"ok": 0, "skip": 0, "fail": 0}


def attempt(name, fn, *args):
    try:
        fn(*args)
        COUNTS["ok"] += 1
    except pytest.skip.Exception:
        COUNTS["skip"] += 1
    except AssertionError as e:
        COUNTS["fail"] += 1
        print("FAIL", name, [a for a in args if not hasattr(a, "__dict__")], str(e)[:300],
              flush=True)


def progress(what):
    print(f"{what}: {COUNTS} {time.time() - T0:.0f} s", flush=True)


def programs(lo, hi):
    import rushlite_amd as rsl
    from oracle import lamp_oracle
    lamp_oracle.load()
    import test_gpu_graphs as TG
    import test_gpu_hip_graph as TH
    for seed in range(lo, hi):
        for cap in (False, True):
            attempt("f64", TG.check_graph, rsl, seed, cap, np.float64, TG.TOL)
            attempt("f32", TG.check_graph, rsl, seed, cap, np.float32, 1e-4)
            for shape in TG.RC_SHAPES:
                attempt("rc", TG.test_random_graph_float32_shapes_vs_oracle, rsl, lamp_oracle,
                        seed, shape, cap)
            for shape in TG.D3_SHAPES:
                attempt("3d", TG.test_random_graph_3d, rsl, lamp_oracle, seed, shape, cap)
            for shape in [(64, 128), (33, 7)]:
                attempt("graph", TH.test_random_program_graph_replays_equal_eager, rsl, seed,
                        shape, cap)
        if seed % 10 == 0:
            progress(f"seed {seed}")


def gemm(seed, count, pairs=100):
    import test_gpu_kernels as TK
    for i, (m, n, k) in enumerate(TK._random_gemm_shapes(count, seed)):
        for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
            attempt("gemm", TK.test_gemm_random_shapes_every_path, abi, m, n, k, ta, tb)
        if i % 100 == 0:
            progress(f"gemm shape {i}")
    rng = np.random.default_rng(seed + 1)
    for i in range(pairs):
        shape = (int(rng.integers(130, 2700)), 4 * int(rng.integers(129, 1026)),
                 4 * int(rng.integers(129, 1026)))
        attempt("pair", TK.test_linear_backward_random_shapes_equal_separate_calls, abi, *shape)
        if i % 20 == 0:
            progress(f"pair {i}")


def _strided_case(L, rng):
    c = rng.random()
    m = int(rng.integers(1, 33) if c < 0.25 else rng.integers(33, 300) if c < 0.6
            else rng.integers(300, 1500))
    n = int(rng.integers(1, 130) if rng.random() < 0.3 else rng.integers(130, 2500))
    k = int(rng.integers(1, 33) if rng.random() < 0.3 else rng.integers(33, 1500))
    if m * n * k > (1 << 30):
        return
    ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    kind = str(rng.choice(["gemm", "acc", "relu", "colsum"]))
    if kind == "colsum":
        tb = 0
    ar, ac = (k, m) if ta else (m, k)
    br, bc = (n, k) if tb else (k, n)
    lda, ldb, ldc = (ac + int(rng.integers(0, 10)), bc + int(rng.integers(0, 10)),
                     n + int(rng.integers(0, 10)))
    oa, ob, oc = (int(rng.integers(0, 4)) for _ in range(3))
    a = rng.standard_normal((ar, ac)).astype(np.float32)
    b = rng.standard_normal((br, bc)).astype(np.float32)
    sentinel = np.float32(12345.0)
    ha = np.full(oa + ar * lda + 8, np.nan, np.float32)
    hb = np.full(ob + br * ldb + 8, np.nan, np.float32)
    hc = np.full(oc + m * ldc + 8, sentinel, np.float32)
    for r in range(ar):
        ha[oa + r * lda: oa + r * lda + ac] = a[r]
    for r in range(br):
        hb[ob + r * ldb: ob + r * ldb + bc] = b[r]
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    if kind == "acc":
        for r in range(m):
            hc[oc + r * ldc: oc + r * ldc + n] = c0[r]
    da, db, dc = (abi.DeviceBuffer.from_numpy(x) for x in (ha, hb, hc))
    pa, pb, pc = da.ptr + 4 * oa, db.ptr + 4 * ob, dc.ptr + 4 * oc
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    bias = rng.standard_normal(n).astype(np.float32)
    dbias = abi.DeviceBuffer.from_numpy(bias)
    dcs = abi.DeviceBuffer((n,), np.float32)
    if kind in ("gemm", "acc"):
        st = L.lmp_k_gemm_f32(ta, tb, m, n, k, pa, lda, pb, ldb, pc, ldc, int(kind == "acc"))
        if kind == "acc":
            want = want + c0
    elif kind == "relu":
        st = L.lmp_k_linear_relu_f32(ta, tb, m, n, k, pa, lda, pb, ldb, dbias.ptr, pc, ldc)
        want = np.maximum(want + bias, 0.0)
    else:
        st = L.lmp_k_gemm_colsum_f32(ta, 0, m, n, k, pa, lda, pb, ldb, pc, ldc, 0, dcs.ptr, 0)
    case = (kind, m, n, k, ta, tb, lda, ldb, ldc, oa, ob, oc)
    if st == abi.ERR_UNSUPPORTED:
        return
    assert st == abi.OK, (case, st, L.lmp_rt_last_error())
    got = dc.numpy()
    inner = np.stack([got[oc + r * ldc: oc + r * ldc + n] for r in range(m)])
    mask = np.ones(got.shape, bool)
    for r in range(m):
        mask[oc + r * ldc: oc + r * ldc + n] = False
    assert np.all(np.isfinite(inner)), (case, "NaN from the padding reached C")
    assert rel_err(inner, want) <= 1e-5, (case, rel_err(inner, want))
    assert np.array_equal(got[mask], hc[mask]), (case, "an element outside C changed")
    if kind == "colsum":
        assert rel_err(dcs.numpy(), b.astype(np.float64).sum(0)) <= 1e-5, case


def strided(seed, count):
    L = abi.lib()
    rng = np.random.default_rng(seed)
    for i in range(count):
        attempt("strided", _strided_case, L, rng)
        if i % 100 == 0:
            progress(f"strided {i}")


def large(seed, count):
    """Random GEMMs of 2^30 to 7.3e11 multiply-adds (extents up to 9000, every
    orientation, plain, accumulating and bias + ReLU): 26 sampled rows and 26
    sampled columns of each against float64 at 1e-4."""
    import test_gpu_kernels as TK
    rng = np.random.default_rng(seed)
    for i in range(count):
        attempt("large", TK.gemm_large_case, abi, rng)
        if i % 10 == 0:
            progress(f"large {i}")


def _random_shape(rng):
    dims = []
    for _ in range(int(rng.integers(1, 4))):
        c = rng.random()
        dims.append(int(rng.integers(1, 8) if c < 0.3 else rng.integers(8, 300) if c < 0.8
                        else rng.integers(300, 5000)))
    while np.prod(dims) > (1 << 24):
        dims[int(np.argmax(dims))] //= 2
    return tuple(max(1, d) for d in dims)


def ops(seed, nred, nbin=2000):
    from oracle import lamp_oracle as oracle
    oracle.load()
    import test_gpu_kernels as TK
    rng = np.random.default_rng(seed)
    for i in range(nred):
        shape = _random_shape(rng)
        attempt("reduce", TK.test_reduce, abi, oracle, shape, int(rng.integers(0, len(shape))))
        if i % 100 == 0:
            progress(f"reduce {i}")
    for i in range(nbin):
        sa = _random_shape(rng)
        sb = tuple(1 if rng.random() < 0.4 else d for d in sa[int(rng.integers(0, len(sa))):])
        if rng.random() < 0.5:
            sa, sb = sb, sa
        attempt("binary", TK.test_binary_bitexact, abi, oracle, str(rng.choice(TK.EXACT_BIN)), sa,
                sb)
        if i % 200 == 0:
            progress(f"binary {i}")


def typed(seed, ngemm, nred=300, nbin=1500):
    import test_gpu_typed as TT
    rng = np.random.default_rng(seed)
    dims = lambda lo, hi: int(rng.integers(lo, hi))  # noqa: E731
    pick = lambda: TT.TYPED[int(rng.integers(0, len(TT.TYPED)))]  # noqa: E731
    for i in range(ngemm):
        attempt("typed gemm", TT.test_typed_gemm, abi, pick(), dims(1, 300), dims(1, 300),
                dims(1, 300), dims(0, 2), dims(0, 2))
        if i % 100 == 0:
            progress(f"typed gemm {i}")
    for i in range(nred):
        nd = dims(1, 4)
        shape = tuple(dims(1, 400 if nd < 3 else 120) for _ in range(nd))
        attempt("typed reduce", TT.test_typed_reduce, abi, pick(), shape, dims(0, nd))
        if i % 100 == 0:
            progress(f"typed reduce {i}")
    names = ["add", "sub", "mul", "div", "eq", "ne", "ge", "le", "gt", "lt"]
    for i in range(nbin):
        nd = dims(1, 4)
        sa = tuple(dims(1, 200) for _ in range(nd))
        sb = tuple(1 if rng.random() < 0.4 else d for d in sa[dims(0, nd):])
        if rng.random() < 0.5:
            sa, sb = sb, sa
        attempt("typed binary", TT.test_typed_binary_exact, abi, str(rng.choice(names)), pick(),
                sa, sb)
        if i % 200 == 0:
            progress(f"typed binary {i}")


def _noalloc_case(L, rng):
    m, n, k = (int(rng.integers(1, 2100)), int(rng.integers(1, 4200)), int(rng.integers(1, 4200)))
    if m * n * k > (1 << 32):
        return
    ta, tb, acc = int(rng.integers(0, 2)), int(rng.integers(0, 2)), int(rng.integers(0, 2))
    a = (rng.standard_normal((k, m) if ta else (m, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((n, k) if tb else (k, n)) * 0.02).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    da, db = abi.DeviceBuffer.from_numpy(a), abi.DeviceBuffer.from_numpy(b)
    ref, out = abi.DeviceBuffer.from_numpy(c0), abi.DeviceBuffer.from_numpy(c0)
    abi.check(L.lmp_k_gemm_f32(ta, tb, m, n, k, da.ptr, a.shape[1], db.ptr, b.shape[1], ref.ptr,
                               n, acc))
    st = L.lmp_k_gemm_f32_noalloc(ta, tb, m, n, k, da.ptr, a.shape[1], db.ptr, b.shape[1],
                                  out.ptr, n, acc)
    if st == abi.ERR_UNSUPPORTED:  # partials above the fixed workspace
        return
    assert st == abi.OK, ((m, n, k, ta, tb, acc), st)
    assert np.array_equal(out.numpy().view(np.uint32), ref.numpy().view(np.uint32)), \
        (m, n, k, ta, tb, acc)


def noalloc(seed, count):
    """lmp_k_gemm_f32_noalloc against lmp_k_gemm_f32 on random products, one
    after another on the shared workspace: the same bits."""
    L = abi.lib()
    rng = np.random.default_rng(seed)
    for i in range(count):
        attempt("noalloc", _noalloc_case, L, rng)
        if i % 50 == 0:
            progress(f"noalloc {i}")


def _mlp_case(rsl, oracle, rng):
    from rushlite_amd.nets import layers
    nl = int(rng.integers(1, 4))
    widths = [int(rng.choice([rng.integers(1, 80), rng.integers(80, 700)])) for _ in range(nl + 1)]
    batch = int(rng.choice([rng.integers(1, 40), rng.integers(40, 600)]))
    x = rng.random((batch, widths[0]), dtype=np.float32)
    y = rng.random((batch, widths[-1]), dtype=np.float32)
    ws = [(rng.standard_normal((widths[i], widths[i + 1])) / np.sqrt(widths[i])).astype(np.float32)
          for i in range(nl)]
    bs = [(rng.standard_normal(widths[i + 1]) * 0.1).astype(np.float32) for i in range(nl)]
    mods = []
    for i in range(nl):
        mods.append(layers.Linear(widths[i], widths[i + 1]))
        if i < nl - 1:
            mods.append(layers.ReLU())
    mods.append(layers.Softmax(dim=-1))
    model = layers.Sequential(mods)
    li = 0
    for i, m in enumerate(mods):
        if isinstance(m, layers.Linear):
            model.params[f"{i}.weights"] = rsl.Variable(ws[li], requires_grad=True)
            model.params[f"{i}.bias"] = rsl.Variable(bs[li], requires_grad=True)
            li += 1
    capture = bool(rng.integers(0, 2))
    xv, yv = rsl.Variable(x), rsl.Variable(y)
    with rsl.capture_on(capture):
        probs = model(xv)
        loss = (-yv * rsl.log(probs + 1e-3)).sum(1).sum(0)
    loss.backward()
    ref_loss, ref_gw, ref_gb = oracle.mlp_step(ws, bs, x, y)
    _, r64_gw, r64_gb = oracle.mlp_step(ws, bs, x, y, f64_gemm=True)
    case = (widths, batch, capture)
    # Skip a step that is ill-conditioned in float32: both oracle orders more
    # than half the bar from torch float64 (a cancelling column sum of a
    # saturated softmax's gradient, say), where valid float32 orders disagree.
    import torch
    from test_oracle import _torch_softmax_lamp
    tw = [torch.tensor(w, dtype=torch.float64, requires_grad=True) for w in ws]
    tb = [torch.tensor(b, dtype=torch.float64, requires_grad=True) for b in bs]
    h = torch.tensor(x, dtype=torch.float64)
    for i in range(nl):
        h = h @ tw[i] + tb[i]
        if i < nl - 1:
            # a pre-activation within float32 GEMM rounding of zero: the ReLU
            # mask there depends on the summation order
            hv = h.detach().abs()
            if float(hv.min()) < 2e-6 * float(hv.max()):
                pytest.skip(f"a ReLU input within rounding of zero: {case}")
            h = torch.clamp(h, min=0.0)
    tl = (-torch.tensor(y, dtype=torch.float64) * torch.log(_torch_softmax_lamp(h, -1) + 1e-3))
    tl.sum(1, keepdim=True).sum(0, keepdim=True).backward()
    truth = [t.grad.numpy() for pair in zip(tw, tb) for t in pair]
    refs_all = [t for pair in zip(ref_gw, ref_gb) for t in pair]
    refs64_all = [t for pair in zip(r64_gw, r64_gb) for t in pair]
    for r, r64, t in zip(refs_all, refs64_all, truth):
        if min(rel_err(r, t), rel_err(r64, t)) > 5e-5:
            pytest.skip(f"ill-conditioned in float32: {case}")
    assert abs(loss.tolist()[0] - ref_loss) <= 1e-4 * max(abs(ref_loss), 1e-30), case
    grads = [p.grad.numpy() for _, p in model.named_parameters()]
    refs = [t for pair in zip(ref_gw, ref_gb) for t in pair]
    refs64 = [t for pair in zip(r64_gw, r64_gb) for t in pair]
    for i, (g, r, r64) in enumerate(zip(grads, refs, refs64)):
        assert min(rel_err(g, r), rel_err(g, r64)) <= 1e-4, (case, i)


def mlp(seed, count):
    """One training step of random Linear-ReLU-...-Softmax nets (1-3 layers,
    widths and batches across the GEMM kernels' thresholds, the forward
    captured or eager) against the oracle's step in two GEMM orders."""
    import rushlite_amd as rsl
    from oracle import lamp_oracle as oracle
    oracle.load()
    rng = np.random.default_rng(seed)
    for i in range(count):
        attempt("mlp", _mlp_case, rsl, oracle, rng)
        if i % 25 == 0:
            progress(f"mlp {i}")


def graphs(seed, count):
    """Random MLP training steps captured in a HIP graph (the update eager or
    captured), every replay against an eager twin bit for bit."""
    import rushlite_amd as rsl
    import test_gpu_hip_graph as TH
    rng = np.random.default_rng(seed)
    for i in range(count):
        nl = int(rng.integers(1, 4))
        dims = tuple(int(rng.choice([rng.integers(1, 80), rng.integers(80, 1100)]))
                     for _ in range(nl + 1))
        batch = int(rng.choice([rng.integers(1, 40), rng.integers(40, 600)]))
        attempt("graph", TH.test_graph_replays_equal_eager_steps, rsl, dims, batch,
                bool(rng.integers(0, 2)))
        if i % 10 == 0:
            progress(f"graphs {i}")


def _same_or_both_nan(got, want):
    got, want = np.asarray(got), np.asarray(want)
    nan = np.isnan(want)
    return (got.shape == want.shape and np.array_equal(np.isnan(got), nan)
            and np.array_equal(got[~nan].view(np.uint8), want[~nan].view(np.uint8)))


def _specials_case(rsl, rng, seed, shape, dtype):
    import test_gpu_graphs as TG
    from _helpers import SPECIALS
    leaves, steps, shapes = TG.make_program_3d(seed, *shape)
    arrs = []
    for s in leaves:
        v = rng.uniform(-1.0, 1.0, s)
        pick = rng.random(s) < 0.3
        v[pick] = rng.choice(SPECIALS.astype(np.float64), int(pick.sum()))
        arrs.append(v.astype(dtype))
    kind = rsl.dtype.float64 if dtype == np.float64 else rsl.dtype.float32
    ops = TG.lamp_ops(rsl, kind)
    outs = []
    for capture in (False, True):
        lv = [rsl.Variable(a, dtype=kind) for a in arrs]
        with rsl.capture_on(capture):
            out = TG._run_steps(ops, lv, steps)
        outs.append(out.numpy())
    assert _same_or_both_nan(outs[1], outs[0]), (seed, shape, np.dtype(dtype).name, steps)


def _bits_case(rsl, rng, seed, shape, dtype):
    import test_gpu_graphs as TG
    leaves, steps, shapes = TG.make_program_rc(seed, *shape)
    arrs = [rng.uniform(-1.0, 1.0, s).astype(dtype) for s in leaves]
    kind = rsl.dtype.float64 if dtype == np.float64 else rsl.dtype.float32
    ops = TG.lamp_ops(rsl, kind)
    outs, grads = [], []
    for capture in (False, True):
        lv = [rsl.Variable(a, requires_grad=True, dtype=kind) for a in arrs]
        with rsl.capture_on(capture):
            out = TG._run_steps(ops, lv, steps)
            total = TG.run(ops, lv, steps, shapes)
        outs.append(out.numpy())
        total.backward()
        grads.append([v.grad.numpy() for v in lv])
    assert _same_or_both_nan(outs[1], outs[0]), (seed, shape, "value", steps)
    for i, (g1, g0) in enumerate(zip(grads[1], grads[0])):
        assert _same_or_both_nan(g1, g0), (seed, shape, "grad", i, steps)


def _held_case(rsl, rng, seed, shape, dtype):
    import test_gpu_graphs as TG
    leaves, steps, shapes = TG.make_program_rc(seed, *shape)
    arrs = [rng.uniform(-1.0, 1.0, s).astype(dtype) for s in leaves]
    kind = rsl.dtype.float64 if dtype == np.float64 else rsl.dtype.float32
    ops = TG.lamp_ops(rsl, kind)
    first = len(leaves)
    keep = sorted(set(int(i) for i in rng.integers(first, first + len(steps), int(rng.integers(1, 24)))))
    results = []
    for capture in (False, True):
        # one step at a time over a growing pool (the step's operands index
        # it), so every intermediate has a Python owner while the rest of the
        # program is recorded; those in `keep` outlive the region
        pool = [rsl.Variable(a, dtype=kind) for a in arrs]
        with rsl.capture_on(capture):
            for st in steps:
                pool.append(TG._run_steps(ops, pool, [st]))
        held = {i: pool[i] for i in keep}
        held[-1] = pool[-1]
        del pool
        results.append({i: v.numpy() for i, v in held.items()})
    for i in results[0]:
        assert _same_or_both_nan(results[1][i], results[0][i]), (seed, shape, "value", i, keep, steps)


def held(seed, count):
    """Random programs run with some intermediates held by the caller (so the
    fused regions store them as extra outputs, split at the output limit, or
    cut there), captured against eager: every held value and the result bit
    for bit."""
    import rushlite_amd as rsl
    import test_gpu_graphs as TG
    rng = np.random.default_rng(seed)
    shapes = TG.RC_SHAPES + [(512, 1000), (7, 5)]
    for i in range(count):
        shape = shapes[int(rng.integers(0, len(shapes)))]
        dt = np.float64 if rng.random() < 0.3 else np.float32
        attempt("held", _held_case, rsl, rng, int(rng.integers(0, 1 << 30)), shape, dt)
        if i % 50 == 0:
            progress(f"held {i}")


def bits(seed, count):
    """Random programs over [R, C] leaves (matmul and transpose included),
    captured against eager: values and every input gradient bit for bit."""
    import rushlite_amd as rsl
    import test_gpu_graphs as TG
    rng = np.random.default_rng(seed)
    shapes = TG.RC_SHAPES + [(512, 1000), (7, 5)]
    for i in range(count):
        shape = shapes[int(rng.integers(0, len(shapes)))]
        dt = np.float64 if rng.random() < 0.3 else np.float32
        attempt("bits", _bits_case, rsl, rng, int(rng.integers(0, 1 << 30)), shape, dt)
        if i % 50 == 0:
            progress(f"bits {i}")


def _copies_case(L, rng):
    nbytes = int(np.exp(rng.uniform(0, np.log(96 << 20))))
    so, do = int(rng.integers(0, 64)), int(rng.integers(0, 64))
    src = rng.integers(0, 256, so + nbytes + 64, dtype=np.uint8)
    dev = abi.DeviceBuffer((do + nbytes + 64,), np.uint8)
    guard = rng.integers(0, 256, do + nbytes + 64, dtype=np.uint8)
    abi.check(L.lmp_rt_memcpy_h2d(dev.ptr, guard.ctypes.data, guard.nbytes))
    abi.check(L.lmp_rt_memcpy_h2d(dev.ptr + do, src.ctypes.data + so, nbytes))
    back = np.empty(do + nbytes + 64, np.uint8)
    abi.check(L.lmp_rt_memcpy_d2h(back.ctypes.data, dev.ptr, back.nbytes))
    want = guard.copy()
    want[do:do + nbytes] = src[so:so + nbytes]
    assert np.array_equal(back, want), ("h2d", nbytes, so, do)
    # device to device into another offset, then a partial download
    dev2 = abi.DeviceBuffer((nbytes + 128,), np.uint8)
    o2 = int(rng.integers(0, 64))
    abi.check(L.lmp_rt_memcpy_d2d(dev2.ptr + o2, dev.ptr + do, nbytes))
    part = np.empty(nbytes + 8, np.uint8)
    part[-8:] = 7
    abi.check(L.lmp_rt_memcpy_d2h(part.ctypes.data, dev2.ptr + o2, nbytes))
    assert np.array_equal(part[:nbytes], src[so:so + nbytes]), ("d2d/d2h", nbytes, so, do, o2)
    assert np.all(part[-8:] == 7), ("d2h wrote past its end", nbytes)


def copies(seed, count):
    """Host-device copies of random sizes (1 byte to 96 MiB, across the staging
    threshold and chunk boundaries) at random byte offsets on both sides: the
    bytes arrive, nothing around them changes."""
    L = abi.lib()
    rng = np.random.default_rng(seed)
    for i in range(count):
        attempt("copies", _copies_case, L, rng)
        if i % 50 == 0:
            progress(f"copies {i}")


def specials(seed, count):
    """Random elementwise and reduction programs (the 3-d generator: every
    broadcast kind, reductions over any axis) on inputs 30% special values
    (signed zeros, infinities, NaN, subnormals, extremes): the fused kernels
    against the eager ones, bit for bit, NaN by position."""
    import rushlite_amd as rsl
    import test_gpu_graphs as TG
    rng = np.random.default_rng(seed)
    shapes = TG.D3_SHAPES + [(1, 64, 128), (2, 33, 7)]
    for i in range(count):
        shape = shapes[int(rng.integers(0, len(shapes)))]
        dt = np.float64 if rng.random() < 0.3 else np.float32
        attempt("specials", _specials_case, rsl, rng, int(rng.integers(0, 1 << 30)), shape, dt)
        if i % 50 == 0:
            progress(f"specials {i}")


def main():
    suite, a, b = sys.argv[1], int(sys.argv[2]), int(sys.argv[3])
    abi.check(abi.lib().lmp_rt_init(0))
    {"programs": programs, "gemm": gemm, "strided": strided, "ops": ops,
     "typed": typed, "noalloc": noalloc, "mlp": mlp, "graphs": graphs,
     "specials": specials, "bits": bits, "copies": copies, "held": held, "large": large}[suite](a, b)
    print("DONE", suite, COUNTS, flush=True)
    sys.exit(1 if COUNTS["fail"] else 0)


if __name__ == "__main__":
    main()
