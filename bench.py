#!/usr/bin/env python3
"""Benchmark of the Lamp3 MI355X backend; prints ONE JSON line.

Headline: the captured, fused broadcast chain
c = a*a + b with a [8192,8192] and b [8192,1] fp32, uniform[0,1) inputs from
fixed seeds, resident in HBM.  One step = one realisation of the captured
graph = one fused kernel launch.  `value` is HBM GB/s counted on algorithmic
bytes (read a and b once, write c once: 536,903,680 B per step) over the
steps timed back to back between two HIP events on the library stream.

MI355X's 256 MB memory-side cache (MALL) could hold part of `a` from the
previous step, so the timed steps rotate over three copies of `a` (three
256 MiB buffers with the same values): between two uses of one copy the
other two stream 512 MiB of reads and 512 MiB of writes, so every step reads
its `a` from HBM, and the steps still run back to back (no event pair or
synchronisation per step).  `evicted_per_step` times each step alone after a
1 GiB read (HIP events around every step); `warm_loop` repeats one copy.
(The fused kernel reads operands of 256 MiB or more with nontemporal loads,
which do not allocate in the MALL, so today all three read HBM.)

`extra` carries the other configs measured in the same process: the 6-op
chain, the [16384,16384] dim reductions and broadcast-add backwards, the
fp32 GEMMs (TFLOP/s; the skinny ones also in TB/s, cold), and the MLP
training loops (steps/s).  `cpu_baseline` times the CPU oracle (a
from-scratch restatement of Lamp3's CPU backend, built with the reference's
-O3 -ffast-math flags and OpenMP) on the host cores of the same machine, for
every config, on bounded samples stated in each entry.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

# The CPU baseline's OpenMP threads stay on neighbouring cores (the reference
# baseline plan); set before any OpenMP runtime is loaded.
os.environ.setdefault("OMP_PROC_BIND", "close")

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

METRIC = "fused-kernel HBM GB/s (% of peak); fp32 matmul TFLOP/s; MLP train steps/s"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
FP64_MFMA_PEAK_TFLOPS = 78.6
N8K = 8192
N16K = 16384
BYTES_C1 = 4 * (2 * N8K * N8K + N8K)          # 536,903,680
BYTES_C2 = 4 * (N16K * N16K + N16K)           # 1,073,807,360
TRAFFIC_FILE = ROOT / "profiles" / "fused_a2b_8192_traffic.json"
ROTATE_C1 = 3      # copies of a (256 MiB each) the config-1 steps rotate over
ROTATE_THIN = 4    # copies of W (128 MiB each) the skinny GEMMs rotate over
C4_DIMS, C4_BATCH = (4096, 4096, 4096, 1000), 512
C0_DIMS, C0_BATCH = (256, 64, 10), 32


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=5.0,
                   help="CPU time budget of the config-1 baseline sample")
    p.add_argument("--only", nargs="+",
                   choices=["c1", "c2", "c3", "c3thin", "f64", "mlp"],
                   help="run only these extra sections (for per-config profiles)")
    p.add_argument("--copy-probe", action="store_true",
                   help="also launch a known-size copy kernel (x + 0 over 64 Mi "
                        "floats: 256 MiB read, 256 MiB written) to calibrate "
                        "rocprof FETCH_SIZE/WRITE_SIZE")
    return p.parse_args()


def ensure_built():
    lib = ROOT / "rushlite_amd" / "lib" / "liblmp_hip.so"
    if not lib.exists() or not list((ROOT / "rushlite_amd").glob("_C*.so")):
        from rushlite_amd import build as b
        b.build_all()


class Events:
    """HIP events recorded on the stream every backend kernel runs on."""

    def __init__(self, abi):
        self.abi = abi
        self.t = abi.Timer()

    def __enter__(self):
        self.abi.synchronize()
        self.t.begin()
        return self

    def __exit__(self, *exc):
        self.ms = self.t.end()
        self.abi.synchronize()


def time_steps(abi, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    abi.synchronize()
    with Events(abi) as ev:
        for _ in range(steps):
            fn()
    return ev.ms


def time_rotating(abi, fns, steps, warmup):
    """Steps run back to back, cycling over `fns` (one closure per copy of
    the large operand); one event pair around all of them."""
    k = len(fns)
    for i in range(warmup):
        fns[i % k]()
    abi.synchronize()
    with Events(abi) as ev:
        for i in range(steps):
            fns[i % k]()
    return ev.ms


class Evictor:
    """Empties the MALL of a step's operands: a dim-1 sum over a 1 GiB tensor
    (four times the cache) streams unrelated lines through it."""

    def __init__(self, rsl):
        self.rsl = rsl
        self.big = rsl.ones([N16K, N16K])

    def __call__(self):
        with self.rsl.no_grad():
            self.rsl.sum(self.big, 1).realize()


def time_steps_cold(abi, fn, evict, steps, warmup):
    """Sum of per-step HIP-event times of `fn`, each step preceded (outside
    its timed interval) by `evict`."""
    for _ in range(warmup):
        evict()
        fn()
    abi.synchronize()
    t = abi.Timer()
    total = 0.0
    for _ in range(steps):
        evict()
        t.begin()
        fn()
        total += t.end()
    abi.synchronize()
    return total


def c1_inputs(rsl):
    a_np = np.random.default_rng(0).random((N8K, N8K), dtype=np.float32)
    b_np = np.random.default_rng(1).random((N8K, 1), dtype=np.float32)
    a_list = [rsl.Variable(a_np) for _ in range(ROTATE_C1)]
    return a_list, rsl.Variable(b_np)


def headline(rsl, abi, a_list, b, steps, warmup, evict):
    def make(a):
        def step():
            with rsl.capture_on():
                c = a * a + b
            c.realize()
        return step

    fns = [make(a) for a in a_list]
    s0 = rsl._stats()
    ms = time_rotating(abi, fns, steps, warmup)
    s1 = rsl._stats()
    launches = (s1["fused_launches"] - s0["fused_launches"]) / (steps + warmup)
    per_step_ms = ms / steps
    evicted_ms = time_steps_cold(abi, fns[0], evict, max(5, steps // 4), 2) / max(5, steps // 4)
    warm_ms = time_steps(abi, fns[0], steps, warmup) / steps
    return per_step_ms, evicted_ms, warm_ms, launches


def extras(rsl, abi, a_list, b, steps, warmup, only=None):
    out = {}
    want = lambda tag: only is None or tag in only  # noqa: E731
    L = abi.lib()
    dbl_max = sys.float_info.max

    if want("c1"):
        # --- config 1b: 6-op chain, fused, and the reference-style unfused path
        def make_chain(a):
            def chain():
                with rsl.capture_on():
                    c = rsl.exp(a) * b - rsl.clamp(a, 0, dbl_max) / (b + 1)
                c.realize()
            return chain
        ms = time_rotating(abi, [make_chain(a) for a in a_list], steps, warmup) / steps
        warm = time_steps(abi, make_chain(a_list[0]), steps, warmup) / steps
        out["c1b_chain6_fused"] = {"us": round(ms * 1e3, 2),
                                   "GB/s": round(BYTES_C1 / ms / 1e6, 1),
                                   "warm_loop_us": round(warm * 1e3, 2)}

        def make_unfused(a):
            return lambda: (a * a + b).realize()
        r = steps // 4 + 1
        ms = time_rotating(abi, [make_unfused(a) for a in a_list], r, 2) / r
        out["c1a_eager_unfused_2_launches"] = {"us": round(ms * 1e3, 2),
                                               "GB/s_algorithmic": round(BYTES_C1 / ms / 1e6, 1)}

        # The 6-op chain outside capture_on: one eager kernel per op (exp, mul,
        # clamp, the [8192,1] b + 1, div, sub), every intermediate written to
        # and read back from HBM
        def make_chain_eager(a):
            return lambda: (rsl.exp(a) * b - rsl.clamp(a, 0, dbl_max) / (b + 1)).realize()
        s0 = rsl._stats()
        ms = time_rotating(abi, [make_chain_eager(a) for a in a_list], r, 2) / r
        s1 = rsl._stats()
        out["c1b_chain6_eager_unfused"] = {
            "us": round(ms * 1e3, 2),
            "GB/s_algorithmic": round(BYTES_C1 / ms / 1e6, 1),
            "launches_per_step": (s1["kernels"] - s0["kernels"]) / (r + 2)}

        # Host <-> device around the path (the boundary takes device buffers;
        # `value` never includes these): upload of a and b from pageable
        # numpy arrays (Variable(ndarray)), download of c (.numpy()), and the
        # config-1 rate with both included.
        a_np = np.random.default_rng(0).random((N8K, N8K), dtype=np.float32)
        b_np = np.random.default_rng(1).random((N8K, 1), dtype=np.float32)
        ups, downs, ends = [], [], []
        for _ in range(3):
            abi.synchronize()
            t0 = time.perf_counter()
            av, bv = rsl.Variable(a_np), rsl.Variable(b_np)
            abi.synchronize()
            t1 = time.perf_counter()
            with rsl.capture_on():
                cv = av * av + bv
            cv.realize()
            abi.synchronize()
            t2 = time.perf_counter()
            c_np = cv.numpy()
            t3 = time.perf_counter()
            ups.append(t1 - t0)
            downs.append(t3 - t2)
            ends.append(t3 - t0)
            del av, bv, cv, c_np
        up, down, end = min(ups), min(downs), min(ends)
        out["c1_host_device"] = {
            "h2d_GB/s": round((a_np.nbytes + b_np.nbytes) / up / 1e9, 2),
            "d2h_GB/s": round(a_np.nbytes / down / 1e9, 2),
            "end_to_end_ms": round(end * 1e3, 2),
            "end_to_end_GB/s_algorithmic": round(BYTES_C1 / end / 1e9, 2),
            "note": "best of 3: upload a and b from pageable host arrays, fused kernel, download "
                    "c to a new host array; wall clock with a synchronisation after each part"}
        del a_np, b_np

    if want("c2"):
        # --- config 2: dim reductions and the broadcast-add backward (1 GiB
        # operands, four times the MALL: every pass reads HBM)
        A_np = np.random.default_rng(3).standard_normal((N16K, N16K), dtype=np.float32)
        A = rsl.Variable(A_np, requires_grad=True)
        del A_np
        reps = max(5, steps // 10)
        for name, fn in (("sum_dim0", lambda: rsl.sum(A, 0).realize()),
                         ("sum_dim1", lambda: rsl.sum(A, 1).realize()),
                         ("max_dim1", lambda: rsl.max(A, 1).realize())):
            with rsl.no_grad():
                ms = time_steps(abi, fn, reps, 2) / reps
            out["c2_" + name] = {"us": round(ms * 1e3, 2), "GB/s": round(BYTES_C2 / ms / 1e6, 1)}
        B = rsl.Variable(np.zeros((1, N16K), np.float32), requires_grad=True)

        def bwd():
            (A + B).backward()
            # materialise the gradients every step, as a reader of .grad would
            A.grad.realize()
            B.grad.realize()
        # two warm-up steps: the first leaves the gradients constant, the
        # second compiles the in-place accumulation kernels
        n_bwd = max(3, reps // 2)
        ms = time_steps(abi, bwd, n_bwd, 2) / n_bwd
        out["c2_broadcast_add_backward"] = {
            "ms": round(ms, 3),
            "note": "forward A + B (read 1 GiB, write 1 GiB) and backward with both gradients "
                    "materialised each step: A.grad += 1 in place by one fused kernel (read and "
                    "write 1 GiB); B.grad's dim-0 sum of the ones seed is exact in any order and "
                    "folds to a constant, so this line runs no dim-0 reduction kernel "
                    "(c2_broadcast_add_backward_upstream does)"}
        G = rsl.Variable(np.random.default_rng(4).standard_normal((N16K, N16K),
                                                                  dtype=np.float32))
        A.zero_grad()
        B.zero_grad()

        def bwd_up():
            ((A + B) * G).backward()
            A.grad.realize()
            B.grad.realize()
        ms = time_steps(abi, bwd_up, n_bwd, 2) / n_bwd
        out["c2_broadcast_add_backward_upstream"] = {
            "ms": round(ms, 3),
            "note": "forward (A + B) * G with G [16384,16384] normal(0,1): the gradient reaching "
                    "A + B is G, not a constant, so backward runs A.grad += G in place and "
                    "B.grad += the dim-0 reduction of G over 16384 rows (the col_reduce kernel "
                    "of c2_sum_dim0) each step"}
        del A, B, G

    if want("c3") or want("c3thin"):
        # --- config 3: fp32 GEMMs through the C ABI (the same kernels Linear uses)
        gemm = {}
        zero_fns = []
        shapes = ((32, 4096, 8192),) if not want("c3") else \
            ((4096, 4096, 4096), (8192, 8192, 8192), (32, 4096, 8192))
        for (m, n, k) in shapes:
            thin = m <= 32
            copies = ROTATE_THIN if thin else 1
            rng_x, rng_w, rng_y = (np.random.default_rng(s) for s in (2, 10, 3))
            # entries normal(0, 0.02) from fixed seeds (x 2, weights 10, dY 3)
            X = abi.DeviceBuffer.from_numpy(rng_x.standard_normal((m, k), dtype=np.float32) * 0.02)
            W_np = rng_w.standard_normal((k, n), dtype=np.float32) * 0.02
            Ws = [abi.DeviceBuffer.from_numpy(W_np) for _ in range(copies)]
            del W_np
            dY = abi.DeviceBuffer.from_numpy(rng_y.standard_normal((m, n), dtype=np.float32) * 0.02)
            Y, dX = abi.DeviceBuffer((m, n)), abi.DeviceBuffer((m, k))
            dWs = [abi.DeviceBuffer((k, n)) for _ in range(copies)]
            # Linear: Y = X W ; dX = dY W^T ; dW = X^T dY   (each 2*m*n*k flop)
            cases = (("fwd", 0, 0, m, n, k, lambda i: X, k, lambda i: Ws[i], n, lambda i: Y),
                     ("dX", 0, 1, m, k, n, lambda i: dY, n, lambda i: Ws[i], n, lambda i: dX),
                     ("dW", 1, 0, k, n, m, lambda i: X, k, lambda i: dY, n, lambda i: dWs[i]))
            for label, ta, tb, mm, nn, kk, A_, lda, B_, ldb, C_ in cases:
                def make(i, ta=ta, tb=tb, mm=mm, nn=nn, kk=kk, A_=A_, lda=lda, B_=B_, ldb=ldb,
                         C_=C_):
                    a_, b_, c_ = A_(i).ptr, B_(i).ptr, C_(i).ptr
                    return lambda: abi.check(L.lmp_k_gemm_f32(ta, tb, mm, nn, kk, a_, lda, b_,
                                                              ldb, c_, nn, 0))
                fns = [make(i) for i in range(copies)]
                flop = 2.0 * mm * nn * kk
                key = f"{m}x{n}x{k}_{label}"
                if thin:
                    # the weight (or weight gradient) is 128 MiB: rotate over
                    # four copies so each call reads (writes) it in HBM, not
                    # in the 256 MB MALL; 200 calls back to back
                    r = 200
                    ms = time_rotating(abi, fns, r, 40) / r
                    warm = time_steps(abi, fns[0], r, 40) / r
                    algo = 4.0 * (mm * kk + kk * nn + mm * nn)
                    gemm[key] = {
                        "us": round(ms * 1e3, 2), "TFLOP/s": round(flop / ms / 1e9, 1),
                        "frac_of_fp32_peak": round(flop / ms / 1e9 / FP32_MFMA_PEAK_TFLOPS, 3),
                        "algorithmic_bytes": int(algo), "TB/s": round(algo / ms / 1e9, 3),
                        "frac_of_hbm_peak": round(algo / ms / 1e6 / HBM_PEAK_GBS, 3),
                        "warm_loop_us": round(warm * 1e3, 2)}
                    zero_fns.append((key, ta, tb, mm, nn, kk, lda, ldb))
                else:
                    r = 3 if m >= 8192 else 10
                    # about 25 ms of warm-up so the clocks have settled
                    ms = time_steps(abi, fns[0], r, 3 if m >= 8192 else 20) / r
                    gemm[key] = {
                        "us": round(ms * 1e3, 1), "TFLOP/s": round(flop / ms / 1e9, 1),
                        "frac_of_fp32_peak": round(flop / ms / 1e9 / FP32_MFMA_PEAK_TFLOPS, 3)}
            del X, Ws, dY, Y, dX, dWs
            if zero_fns:
                # The same calls on all-zero operands: the same kernels, bytes
                # and instructions; only the values the MFMAs see differ.  The
                # gap is what the part's power limit costs these kernels
                # (random operands lower the clock while HBM streams).
                Z = [abi.DeviceBuffer((k, n)) for _ in range(copies)]
                Zx, Zy = abi.DeviceBuffer((m, k)), abi.DeviceBuffer((m, n))
                for buf in (*Z, Zx, Zy):
                    abi.check(L.lmp_k_fill(abi.FLOAT32, buf.ptr, buf.nbytes // 4, 0.0))
                out_y, out_x = abi.DeviceBuffer((m, n)), abi.DeviceBuffer((m, k))
                outs = [abi.DeviceBuffer((k, n)) for _ in range(copies)]
                for key, ta, tb, mm, nn, kk, lda, ldb in zero_fns:
                    def make_zero(i, ta=ta, tb=tb, mm=mm, nn=nn, kk=kk, lda=lda, ldb=ldb, key=key):
                        if key.endswith("_fwd"):
                            a_, b_, c_ = Zx.ptr, Z[i].ptr, out_y.ptr
                        elif key.endswith("_dX"):
                            a_, b_, c_ = Zy.ptr, Z[i].ptr, out_x.ptr
                        else:
                            a_, b_, c_ = Zx.ptr, Zy.ptr, outs[i].ptr
                        return lambda: abi.check(L.lmp_k_gemm_f32(ta, tb, mm, nn, kk, a_, lda, b_,
                                                                  ldb, c_, nn, 0))
                    r = 200
                    zms = time_rotating(abi, [make_zero(i) for i in range(copies)], r, 40) / r
                    gemm[key]["zero_operands_us"] = round(zms * 1e3, 2)
                del Z, Zx, Zy, out_y, out_x, outs
                zero_fns.clear()
        out["c3_gemm"] = gemm
        if any(s[0] <= 32 for s in shapes):
            out["c3_gemm"]["note"] = (
                "skinny GEMMs: algorithmic bytes = 4*(M*K + K*N + M*N) per call; timed over 200 "
                "calls back to back rotating over four copies of the 128 MiB weight (weight "
                "gradient), so each call moves it through HBM; warm_loop_us repeats one copy; "
                "zero_operands_us runs the same calls on all-zero operands (same kernels and "
                "bytes: the difference is the clock the power limit leaves random operands)")

    if want("f64"):
        # float64 GEMM (the reference's float64 suites run matmul on the device)
        n = 4096
        A64, B64 = (abi.DeviceBuffer.from_numpy(
            np.random.default_rng(seed).standard_normal((n, n)) * 0.02) for seed in (2, 10))
        C64 = abi.DeviceBuffer((n, n), np.float64)

        def run64():
            abi.check(L.lmp_k_gemm(abi.FLOAT64, 0, 0, n, n, n, A64.ptr, n, B64.ptr, n, C64.ptr, n, 0))
        ms = time_steps(abi, run64, 5, 1) / 5
        flop = 2.0 * n ** 3
        out["gemm_f64_4096"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(flop / ms / 1e9, 1),
                                "frac_of_fp64_peak": round(flop / ms / 1e9 / FP64_MFMA_PEAK_TFLOPS, 3)}
        # 1024^3: too few 128 x 128 tiles to cover the CUs, so the 64 x 64 kernel
        m = 1024

        def run64s():
            abi.check(L.lmp_k_gemm(abi.FLOAT64, 0, 0, m, m, m, A64.ptr, n, B64.ptr, n, C64.ptr, n, 0))
        ms = time_steps(abi, run64s, 20, 3) / 20
        flop = 2.0 * m ** 3
        out["gemm_f64_1024"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(flop / ms / 1e9, 1),
                                "frac_of_fp64_peak": round(flop / ms / 1e9 / FP64_MFMA_PEAK_TFLOPS, 3),
                                "note": "the top-left 1024 x 1024 blocks of the 4096 x 4096 operands "
                                        "(leading dimension 4096), on the 64 x 64-tile kernel"}
        del A64, B64, C64

    if want("mlp"):
        # --- config 4 and config 0: MLP training loops
        # Config 4's throughput is quoted from a run whose gradients are dense:
        # at the stated randn(0, 1) init the softmax saturates to exact one-hot
        # rows and every gradient is exactly zero, so the backward GEMMs run on
        # all-zero operands (faster: less power).  The 1/64 (fan-in) init runs
        # them on dense gradients; the stated-init runs follow, labelled.
        out["c4_wide_mlp_fan_in_init"] = mlp_bench(rsl, abi, C4_DIMS, C4_BATCH, 50, onehot=True,
                                                   fused_update=True, scale=1.0 / 64)
        out["c4_wide_mlp_fan_in_init_hip_graph"] = mlp_bench(
            rsl, abi, C4_DIMS, C4_BATCH, 50, onehot=True, graph=True, fused_update=True,
            scale=1.0 / 64)
        out["c4_wide_mlp"] = mlp_bench(rsl, abi, C4_DIMS, C4_BATCH, 50, onehot=True)
        out["c0_readme_mlp"] = mlp_bench(rsl, abi, C0_DIMS, C0_BATCH, 100, onehot=False,
                                         keep_losses=True)
        # the SGD update captured (fused), then each step replayed from a HIP graph
        out["c4_wide_mlp_fused_update"] = mlp_bench(rsl, abi, C4_DIMS, C4_BATCH, 50,
                                                    onehot=True, fused_update=True)
        out["c4_wide_mlp_hip_graph"] = mlp_bench(rsl, abi, C4_DIMS, C4_BATCH, 50,
                                                 onehot=True, graph=True, fused_update=True)
        out["c0_readme_mlp_hip_graph"] = mlp_bench(rsl, abi, C0_DIMS, C0_BATCH, 100,
                                                   onehot=False, graph=True, fused_update=True)
    return out


def mlp_problem(dims, batch, onehot, scale=1.0):
    """Seeded inputs and parameters (one generator, seed 2): x normal(0, 1)
    with one-hot y (config 4) or x, y uniform[0, 1) (config 0), then each
    Linear's weights [in, out] and bias [out], normal(0, 1) * scale."""
    rng = np.random.default_rng(2)
    if onehot:
        x = rng.standard_normal((batch, dims[0]), dtype=np.float32)
        y = np.zeros((batch, dims[-1]), np.float32)
        y[np.arange(batch), rng.integers(0, dims[-1], batch)] = 1.0
    else:
        x = rng.random((batch, dims[0]), dtype=np.float32)
        y = rng.random((batch, dims[-1]), dtype=np.float32)
    ws, bs = [], []
    for i in range(len(dims) - 1):
        ws.append(rng.standard_normal((dims[i], dims[i + 1]), dtype=np.float32) * np.float32(scale))
        bs.append(rng.standard_normal(dims[i + 1], dtype=np.float32) * np.float32(scale))
    return x, y, ws, bs


def mlp_bench(rsl, abi, dims, batch, steps, onehot, graph=False, fused_update=False, scale=1.0,
              keep_losses=False):
    from rushlite_amd.nets import layers
    x_np, y_np, ws, bs = mlp_problem(dims, batch, onehot, scale)
    mods = []
    for i in range(len(dims) - 1):
        mods.append(layers.Linear(dims[i], dims[i + 1]))
        if i < len(dims) - 2:
            mods.append(layers.ReLU())
    mods.append(layers.Softmax(dim=-1))
    model = layers.Sequential(mods)
    li = 0
    for i, mod in enumerate(mods):
        if isinstance(mod, layers.Linear):
            model.params[f"{i}.weights"] = rsl.Variable(ws[li], requires_grad=True)
            model.params[f"{i}.bias"] = rsl.Variable(bs[li], requires_grad=True)
            li += 1
    x, y = rsl.Variable(x_np), rsl.Variable(y_np)

    @rsl.capture()
    def forward(inp):
        return model(inp)

    grads_seen = []

    def step():
        probs = forward(x)
        # with fused_update the loss and the SGD update are captured as well
        # (the reference README captures the forward only): the loss rows
        # become one fused row kernel, p - lr*g one kernel per parameter
        with rsl.capture_on(fused_update):
            loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        if not grads_seen:  # the first step's gradients, inspected after it
            grads_seen.extend(p.grad for _, p in model.named_parameters())
        with rsl.capture_on(fused_update):
            for name, p in list(model.named_parameters()):
                model.params[name] = rsl.Variable(p.data - 1e-3 * p.grad, requires_grad=True)
        if fused_update and not graph:
            # the pending updates together (one kernel for the independent
            # ones); a graph capture does this for the carried parameters
            rsl.realize_all(p for _, p in model.named_parameters())
        loss.realize()
        return loss

    first = step()
    first_loss = first.tolist()[0]
    nonzero_grads = sum(int(np.count_nonzero(g.numpy())) for g in grads_seen)
    grad_entries = sum(int(np.prod(g.shape)) for g in grads_seen)
    grads_seen.clear()
    kept = [first.data]  # keep_losses: every step's loss tensor, read after timing
    s2 = rsl._stats()
    for _ in range(2):
        kept.append(step().data)
    s3 = rsl._stats()
    # Kernels of a steady-state step (steps 2 and 3; the library's own count
    # of the kernels it launched): a pending update is launched by the next
    # step, so the first step alone can miss it.
    launches = round((s3["kernels"] - s2["kernels"]) / 2)
    if graph:
        # the whole step (forward, backward, SGD) as one HIP graph launch; its
        # kernels are those the capture records (the carried updates included)
        g = rsl.hip.Graph()
        rsl.realize_all(p for _, p in model.named_parameters())  # the last eager step's updates
        sg = rsl._stats()
        with g.capture(carry=model):
            loss = step()
        sh = rsl._stats()
        launches = sh["kernels"] - sg["kernels"]
        run = g.replay
    else:
        run = step
    abi.synchronize()
    t0 = time.perf_counter()
    with Events(abi) as ev:
        for _ in range(steps):
            out = run()
            if not graph:
                loss = out
                if keep_losses:
                    kept.append(out.data)
    wall = time.perf_counter() - t0
    last = loss.tolist()[0]
    gemm_flop = 0
    for i in range(len(dims) - 1):
        f = 2 * batch * dims[i] * dims[i + 1]
        gemm_flop += f * (2 if i == 0 else 3)  # layer-1 dX is not needed
    return {"steps": steps, "steps/s": round(steps / wall, 2),
            "ms_per_step": round(wall * 1e3 / steps, 3),
            "gpu_event_ms_per_step": round(ev.ms / steps, 3),
            "kernel_launches_per_step": 1 if graph else launches,
            "kernels_per_step": launches,
            "gemm_TFLOP/s_effective": round(gemm_flop * steps / wall / 1e12, 2),
            "init": ("normal(0, 1) (Linear's own init, linear.py:25-29)" if scale == 1.0
                     else f"normal(0, 1) * {scale:g}"),
            "init_scale": scale,
            "gradients": (f"{nonzero_grads} of {grad_entries} first-step gradient entries nonzero"
                          if nonzero_grads else "exactly zero at this init (all "
                          f"{grad_entries} first-step gradient entries): the backward GEMMs "
                          "run on all-zero operands"),
            "first_step_loss": first_loss,
            "final_loss": last,
            "total_steps_run": steps + 3,
            **({"losses": [t.tolist()[0] for t in kept]} if keep_losses and not graph else {})}


# ----------------------------------------------------------- CPU baseline

def host_info():
    """CPU model and core counts of this host (from /proc/cpuinfo and the
    process's CPU affinity), and the OpenMP settings the oracle runs with."""
    model, cores = None, set()
    phys = core = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and model is None:
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not key and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return {"cpu_model": model, "physical_cores_on_host": len(cores) or None,
            "logical_cpus_on_host": os.cpu_count(),
            "cpus_in_affinity_mask": len(os.sched_getaffinity(0)),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OMP_PROC_BIND": os.environ.get("OMP_PROC_BIND")}


def _timed(fn, reps, warm=1):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), reps


def cpu_baseline(seconds, gpu_extra, host):
    """Every config on the oracle's fast build (-O3 -ffast-math, OpenMP), the
    way Lamp3's CPU backend runs it: eager ops, per-output sequential
    reductions, i-j-k GEMMs (cpu/binary.cpp, cpu/expand.cpp, cpu/reduct.cpp:7-19,
    cpu/matrix.cpp:26-33), with flush-to-zero and denormals-are-zero on, the
    mode a -ffast-math build's startup code sets.  Work is bounded to a few
    seconds per config; each entry states its sample and repetitions."""
    from oracle import lamp_oracle as O
    O.load(fast=True)
    # numpy computes its float limits once, on first use; doing that here
    # keeps it from meeting the flush-to-zero mode below
    np.finfo(np.float32), np.finfo(np.float64)
    with O.denormal_flush():
        return _cpu_baseline(O, seconds, gpu_extra, host)


def _c0_envelope(O, x0, y0, w0, b0, steps, fast_losses, gpu_losses):
    """The README MLP trajectory amplifies rounding differences chaotically, so
    the GPU's losses are placed in the band that valid summation orders span
    on the CPU: the strict (IEEE) oracle run with each GEMM order of
    O.GEMM_ORDERS (sequential fp32 as cpu/matrix.cpp, float64-accumulated,
    k reversed, k blocks of 32 and 128 folded in fp32, BLAS sgemm) plus the
    fast build (the reference's -O3 -ffast-math flags).  At step k the band is
    [min, max] of those losses and its width w_k = max - min; the GPU is
    within the envelope when at every step it lies in [min - w_k, max + w_k]
    (for an ensemble of seven, another valid order leaves the plain band at
    about a quarter of the steps).  Gaps are relative to the sequential
    order's loss."""
    orders = {name: np.array(O.mlp_train(w0, b0, x0, y0, steps=steps, f64_gemm=mm)[0])
              for name, mm in O.GEMM_ORDERS.items()}
    orders["fast_build"] = np.array(fast_losses)
    L = np.stack(list(orders.values()))
    lo, hi = L.min(0), L.max(0)
    seq = orders["seq"]
    width = (hi - lo) / np.abs(seq)
    marks = [k for k in (0, 9, 49, steps - 1) if k < steps]
    out = {"orders": list(orders),
           "steps": int(steps),
           "band_width_rel_at_step": {str(k + 1): float(width[k]) for k in marks},
           "band_width_rel_max_over_steps": float(width.max()),
           "final_loss_band": [float(lo[-1]), float(hi[-1])]}
    if gpu_losses is not None and len(gpu_losses) == steps:
        g = np.array(gpu_losses, np.float64)
        outside = np.maximum(lo - g, g - hi).clip(min=0) / np.abs(seq)
        gap_seq = np.abs(g - seq) / np.abs(seq)
        out.update({
            "gpu_final_loss": float(g[-1]),
            "gpu_gap_to_seq_at_step": {str(k + 1): float(gap_seq[k]) for k in marks},
            "max_gap_over_steps": float(gap_seq.max()),
            "gpu_first_step_loss_rel_gap": float(gap_seq[0]),
            "gpu_steps_inside_band": int(np.count_nonzero(outside == 0)),
            "gpu_outside_band_rel_max": float(outside.max()),
            "within_envelope": bool(np.all(outside <= width))})
    return out


def _cpu_baseline(O, seconds, gpu_extra, host):
    fast = dict(fast=True)
    configs = {}

    # config 1a (the headline sample): full workload, repeated for `seconds`
    a = np.random.default_rng(0).random((N8K, N8K), dtype=np.float32)
    b = np.random.default_rng(1).random((N8K, 1), dtype=np.float32)
    O.binary("add", O.binary("mul", a, a, **fast), b, **fast)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        O.binary("add", O.binary("mul", a, a, **fast), b, **fast)
        reps += 1
        c1_el = time.perf_counter() - t0
        if (c1_el >= seconds and reps >= 3) or reps >= 5000:
            break
    c1_value = BYTES_C1 * reps / c1_el / 1e9

    # config 1b: the 6-op chain as six eager ops
    def chain6():
        e = O.binary("mul", O.unary("exp", a, **fast), b, **fast)
        r = O.binary("div", O.unary("clamp", a, 0.0, sys.float_info.max, **fast),
                     O.binary("add", b, np.array([1.0], np.float32), **fast), **fast)
        return O.binary("sub", e, r, **fast)
    med, n = _timed(chain6, 3)
    configs["c1b_chain6"] = {"ms": round(med * 1e3, 1), "GB/s_algorithmic": round(BYTES_C1 / med / 1e9, 2),
                             "reps": n, "stat": "median", "sample": "full workload, six eager ops"}
    del a, b

    # config 2: reductions (median of 5) and the broadcast-add backward
    A = np.random.default_rng(3).standard_normal((N16K, N16K), dtype=np.float32)
    for name, op, ax in (("sum_dim0", "sum", 0), ("sum_dim1", "sum", 1), ("max_dim1", "max", 1)):
        med, n = _timed(lambda: O.reduce(op, A, ax, **fast), 5)
        configs["c2_" + name] = {"ms": round(med * 1e3, 2), "GB/s": round(BYTES_C2 / med / 1e9, 2),
                                 "reps": n, "stat": "median", "sample": "full [16384,16384]"}
    with O.fast_build():
        def bwd():
            Av = O.OVar(A, True)
            Bv = O.OVar(np.zeros((1, N16K), np.float32), True)
            (Av + Bv).backward()
            return Bv.grad
        med, n = _timed(bwd, 1)
    configs["c2_broadcast_add_backward"] = {
        "ms": round(med * 1e3, 1), "reps": n, "stat": "single timed run after one warm-up",
        "sample": "full workload through the oracle's autograd: forward add, ones seed, "
                  "A.grad += seed, B.grad = dim-0 sum of the seed"}
    del A

    # config 3: naive GEMMs.  4096^3 on a row sample (the i-j-k loop's time is
    # linear in the rows of A); the skinny forward in full
    m4 = 32
    X = np.random.default_rng(2).standard_normal((m4, 4096), dtype=np.float32) * 0.02
    W = np.random.default_rng(10).standard_normal((4096, 4096), dtype=np.float32) * 0.02
    med, n = _timed(lambda: O.matmul(X, W, **fast), 1)
    flop = 2.0 * m4 * 4096 * 4096
    configs["c3_gemm_4096_fwd"] = {
        "TFLOP/s": round(flop / med / 1e12, 5), "ms_full_product_est": round(med * 4096 / m4 * 1e3, 0),
        "reps": n, "stat": "single timed run after one warm-up",
        "sample": f"rows 0..{m4 - 1} of the 4096^3 product (i-j-k, cpu/matrix.cpp:26-33); "
                  "full-product time scaled by 4096/32"}
    Xs = np.random.default_rng(2).standard_normal((32, 8192), dtype=np.float32) * 0.02
    Ws = np.random.default_rng(10).standard_normal((8192, 4096), dtype=np.float32) * 0.02
    med, n = _timed(lambda: O.matmul(Xs, Ws, **fast), 1)
    flop = 2.0 * 32 * 4096 * 8192
    configs["c3_gemm_32x4096x8192_fwd"] = {
        "ms": round(med * 1e3, 1), "TFLOP/s": round(flop / med / 1e12, 5), "reps": n,
        "stat": "single timed run after one warm-up", "sample": "full product"}
    del X, W, Xs, Ws

    # config 0: the README MLP from the bench's seeded parameters, as many SGD
    # steps as the GPU loop ran (three untimed, then 100 timed)
    gpu0 = (gpu_extra or {}).get("c0_readme_mlp")
    n0 = gpu0["total_steps_run"] if gpu0 else 103
    x0, y0, w0, b0 = mlp_problem(C0_DIMS, C0_BATCH, onehot=False)
    with O.fast_build():
        t0 = time.perf_counter()
        losses, _, _ = O.mlp_train(w0, b0, x0, y0, steps=n0)
        el = time.perf_counter() - t0
    entry = {"steps/s": round(n0 / el, 2), "steps": n0, "final_loss": losses[-1],
             "first_step_loss": losses[0], "sample": f"full workload, {n0} SGD steps"}
    if gpu0:
        entry["gpu_final_loss"] = gpu0["final_loss"]
        entry["gpu_final_loss_rel_gap_to_fast_build"] = (abs(gpu0["final_loss"] - losses[-1])
                                                        / abs(losses[-1]))
        entry["envelope"] = _c0_envelope(O, x0, y0, w0, b0, n0, losses, gpu0.get("losses"))
    configs["c0_readme_mlp"] = entry

    # config 4: one training step on a batch sample (every GEMM is linear in
    # the batch; the SGD update over 37.8M parameters is not)
    bsz = 16
    x4, y4, w4, b4 = mlp_problem(C4_DIMS, bsz, onehot=True)
    with O.fast_build():
        med, n = _timed(lambda: O.mlp_train(w4, b4, x4, y4, steps=1), 1)
    configs["c4_wide_mlp"] = {
        "ms_per_step_sample": round(med * 1e3, 0), "steps/s_sample": round(1 / med, 3),
        "ms_per_step_full_batch_est": round(med * C4_BATCH / bsz * 1e3, 0),
        "reps": n, "stat": "single timed run after one warm-up",
        "sample": f"one SGD step at batch {bsz} of the 512 (same architecture and init); the "
                  "full-batch estimate scales it by 512/16 (GEMM-dominated)"}

    return {"value": round(c1_value, 2), "unit": "GB/s",
            "cores": O.num_threads(fast=True), "kind": "port", "isa": O.host_isa(),
            "sample": f"full config-1 workload (c = a*a + b, a [8192,8192], b [8192,1]) "
                      f"x {reps} reps, eager mul then broadcast add as Lamp3's CPU path "
                      f"runs it, {O.fast_library_name()} (-O3 -ffast-math, OpenMP, "
                      f"{O.host_isa()}, flush-to-zero), {c1_el:.1f} s",
            "host": host,
            "configs": configs}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              f"(the Lamp3 path has no multi-GPU execution).", file=sys.stderr)
        sys.exit(2)
    ensure_built()
    import rushlite_amd as rsl
    from rushlite_amd import abi

    host = host_info()  # before an OpenMP runtime binds this thread
    abi.check(abi.lib().lmp_rt_init(0))
    info = rsl.hip.device_info()
    evict = Evictor(rsl)
    a_list, b = c1_inputs(rsl)
    per_step_ms, evicted_ms, warm_ms, launches = headline(rsl, abi, a_list, b, args.steps,
                                                          args.warmup, evict)
    value = BYTES_C1 / per_step_ms / 1e6
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config 1: c = a*a + b under capture_on, a [8192,8192], "
                               "b [8192,1] fp32 uniform[0,1) seeds 0/1, one fused "
                               "hipRTC kernel per step; steps rotate over three copies of a "
                               "so each reads it from HBM",
                   "algorithmic_bytes_per_step": BYTES_C1,
                   "fused_launches_per_step": launches,
                   "device": f"{info['arch']} x{info['cu_count']} CUs"},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "evicted_per_step": {"ms_per_step": round(evicted_ms, 5),
                             "GB/s": round(BYTES_C1 / evicted_ms / 1e6, 1),
                             "note": "each step timed alone (events around it) after a 1 GiB "
                                     "read has emptied the MALL"},
        "warm_loop": {"ms_per_step": round(warm_ms, 5),
                      "GB/s": round(BYTES_C1 / warm_ms / 1e6, 1),
                      "note": "one copy of a back to back; a (256 MiB) is read with nontemporal "
                              "loads, which do not allocate in the 256 MB MALL, so this loop "
                              "reads HBM as well"},
    }
    if args.copy_probe:
        zero = rsl.Variable(np.zeros(1, np.float32))
        for i in range(args.steps):
            (a_list[i % ROTATE_C1] + zero).realize()
        abi.synchronize()
        line["copy_probe"] = {"kernel": "bin2d_f32 (x + 0)", "read_bytes": 4 * N8K * N8K,
                              "write_bytes": 4 * N8K * N8K, "launches": args.steps}
    del evict
    if not args.no_extra:
        line["extra"] = extras(rsl, abi, a_list, b, args.steps, args.warmup, args.only)
    del a_list, b
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds, line.get("extra"), host)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
