#!/usr/bin/env python3
"""Benchmark of the Lamp3 MI355X backend; prints ONE JSON line.

Headline: the captured, fused broadcast chain
c = a*a + b with a [8192,8192] and b [8192,1] fp32, uniform[0,1) inputs from
fixed seeds, resident in HBM.  One step = one realisation of the captured
graph = one fused kernel launch.  `value` is HBM GB/s counted on algorithmic
bytes (read a and b once, write c once: 536,903,680 B per step) over
event-timed steps on the library stream.  MI355X's 256 MB memory-side cache
(MALL) would otherwise still hold part of `a` from the previous step, so each
timed step starts after a 1 GiB read has streamed unrelated data through it
(outside the timed interval): every byte then comes from HBM.  The
back-to-back loop, where some of `a` is served by the MALL, is reported
beside it as `warm_loop`.

`extra` carries the other configs measured in the same process: the 6-op
chain, the [16384,16384] dim reductions and the broadcast-add backward, the
fp32 GEMMs (TFLOP/s), and the two MLP training loops (steps/s).
`cpu_baseline` times the CPU oracle (a from-scratch restatement of Lamp3's
CPU backend, built with the reference's -O3 -ffast-math flags) on the host
cores of the same machine.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

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


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", nargs="+", choices=["c1", "c2", "c3", "f64", "mlp"],
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


def headline(rsl, abi, steps, warmup, evict):
    a_np = np.random.default_rng(0).random((N8K, N8K), dtype=np.float32)
    b_np = np.random.default_rng(1).random((N8K, 1), dtype=np.float32)
    a, b = rsl.Variable(a_np), rsl.Variable(b_np)
    del a_np

    def step():
        with rsl.capture_on():
            c = a * a + b
        c.realize()

    s0 = rsl._stats()
    ms = time_steps_cold(abi, step, evict, steps, warmup)
    s1 = rsl._stats()
    launches = (s1["fused_launches"] - s0["fused_launches"]) / (steps + warmup)
    per_step_ms = ms / steps
    warm_ms = time_steps(abi, step, steps, warmup) / steps
    return a, b, per_step_ms, warm_ms, launches


def extras(rsl, abi, a, b, steps, warmup, evict, only=None):
    out = {}
    want = lambda tag: only is None or tag in only  # noqa: E731
    L = abi.lib()
    dbl_max = sys.float_info.max

    if want("c1"):
        # --- config 1b: 6-op chain, fused, and the reference-style unfused path
        def chain():
            with rsl.capture_on():
                c = rsl.exp(a) * b - rsl.clamp(a, 0, dbl_max) / (b + 1)
            c.realize()
        ms = time_steps_cold(abi, chain, evict, steps, warmup) / steps
        warm = time_steps(abi, chain, steps, warmup) / steps
        out["c1b_chain6_fused"] = {"us": round(ms * 1e3, 2),
                                   "GB/s": round(BYTES_C1 / ms / 1e6, 1),
                                   "warm_loop_us": round(warm * 1e3, 2)}

        def unfused():
            (a * a + b).realize()
        r = steps // 4 + 1
        ms = time_steps_cold(abi, unfused, evict, r, 2) / r
        out["c1a_eager_unfused_2_launches"] = {"us": round(ms * 1e3, 2),
                                               "GB/s_algorithmic": round(BYTES_C1 / ms / 1e6, 1)}

    if want("c2"):
        # --- config 2: dim reductions and the broadcast-add backward
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
        ms = time_steps(abi, bwd, max(3, reps // 2), 2) / max(3, reps // 2)
        out["c2_broadcast_add_backward"] = {
            "ms": round(ms, 3),
            "note": "forward A + B (read 1 GiB, write 1 GiB) and backward with both gradients "
                    "materialised each step: A.grad += 1 in place by one fused kernel (read and "
                    "write 1 GiB); B.grad's dim-0 sum of the ones seed is exact in any order and "
                    "folds to a constant (the dim-0 reduction kernel itself is c2_sum_dim0)"}
        del A, B

    if want("c3"):
        # --- config 3: fp32 GEMMs through the C ABI (the same kernels Linear uses)
        gemm = {}
        L = abi.lib()
        for (m, n, k) in ((4096, 4096, 4096), (8192, 8192, 8192), (32, 4096, 8192)):
            # entries normal(0, 0.02) from fixed seeds (x 2, weights 10, dY 3)
            X, W, dY = (abi.DeviceBuffer.from_numpy(
                np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * 0.02)
                for seed, shape in ((2, (m, k)), (10, (k, n)), (3, (m, n))))
            Y, dX, dW = abi.DeviceBuffer((m, n)), abi.DeviceBuffer((m, k)), abi.DeviceBuffer((k, n))
            # Linear: Y = X W ; dX = dY W^T ; dW = X^T dY   (each 2*m*n*k flop)
            cases = (("fwd", 0, 0, m, n, k, X, k, W, n, Y),
                     ("dX", 0, 1, m, k, n, dY, n, W, n, dX),
                     ("dW", 1, 0, k, n, m, X, k, dY, n, dW))
            for label, ta, tb, mm, nn, kk, A_, lda, B_, ldb, C_ in cases:
                r = 3 if m >= 8192 else 10

                def run(ta=ta, tb=tb, mm=mm, nn=nn, kk=kk, A_=A_, lda=lda, B_=B_, ldb=ldb, C_=C_):
                    abi.check(L.lmp_k_gemm_f32(ta, tb, mm, nn, kk, A_.ptr, lda, B_.ptr, ldb,
                                               C_.ptr, nn, 0))
                # about 25 ms of warm-up so the clocks have settled
                ms = time_steps(abi, run, r, 3 if m >= 8192 else 20) / r
                flop = 2.0 * mm * nn * kk
                gemm[f"{m}x{n}x{k}_{label}"] = {
                    "us": round(ms * 1e3, 1), "TFLOP/s": round(flop / ms / 1e9, 1),
                    "frac_of_fp32_peak": round(flop / ms / 1e9 / FP32_MFMA_PEAK_TFLOPS, 3)}
            del X, W, dY, Y, dX, dW
        out["c3_gemm"] = gemm

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
        del A64, B64, C64

    if want("mlp"):
        # --- config 4 and config 0: MLP training loops
        out["c4_wide_mlp"] = mlp_bench(rsl, abi, (4096, 4096, 4096, 1000), 512, 50, onehot=True)
        out["c0_readme_mlp"] = mlp_bench(rsl, abi, (256, 64, 10), 32, 100, onehot=False)
        # the SGD update captured (fused), then each step replayed from a HIP graph
        out["c4_wide_mlp_fused_update"] = mlp_bench(rsl, abi, (4096, 4096, 4096, 1000), 512, 50,
                                                    onehot=True, fused_update=True)
        out["c4_wide_mlp_hip_graph"] = mlp_bench(rsl, abi, (4096, 4096, 4096, 1000), 512, 50,
                                                 onehot=True, graph=True, fused_update=True)
        out["c0_readme_mlp_hip_graph"] = mlp_bench(rsl, abi, (256, 64, 10), 32, 100,
                                                   onehot=False, graph=True, fused_update=True)
    return out


def mlp_bench(rsl, abi, dims, batch, steps, onehot, graph=False, fused_update=False):
    from rushlite_amd.nets import layers
    rng = np.random.default_rng(2)
    if onehot:
        x_np = rng.standard_normal((batch, dims[0]), dtype=np.float32)
        y_np = np.zeros((batch, dims[-1]), np.float32)
        y_np[np.arange(batch), rng.integers(0, dims[-1], batch)] = 1.0
    else:
        x_np = rng.random((batch, dims[0]), dtype=np.float32)
        y_np = rng.random((batch, dims[-1]), dtype=np.float32)
    mods = []
    for i in range(len(dims) - 1):
        mods.append(layers.Linear(dims[i], dims[i + 1]))
        if i < len(dims) - 2:
            mods.append(layers.ReLU())
    mods.append(layers.Softmax(dim=-1))
    model = layers.Sequential(mods)
    for li, mod in enumerate(mods):
        if isinstance(mod, layers.Linear):
            w = rng.standard_normal(mod.weights.shape, dtype=np.float32)
            model.params[f"{li}.weights"] = rsl.Variable(w, requires_grad=True)
            model.params[f"{li}.bias"] = rsl.Variable(
                rng.standard_normal(mod.bias.shape, dtype=np.float32), requires_grad=True)
    x, y = rsl.Variable(x_np), rsl.Variable(y_np)

    @rsl.capture()
    def forward(inp):
        return model(inp)

    def step():
        probs = forward(x)
        # with fused_update the loss and the SGD update are captured as well
        # (the reference README captures the forward only): the loss rows
        # become one fused row kernel, p - lr*g one kernel per parameter
        with rsl.capture_on(fused_update):
            loss = (-y * rsl.log(probs + 1e-3)).sum(1).sum(0)
        loss.backward()
        with rsl.capture_on(fused_update):
            for name, p in list(model.named_parameters()):
                model.params[name] = rsl.Variable(p.data - 1e-3 * p.grad, requires_grad=True)
        if fused_update and not graph:
            # the pending updates together (one kernel for the independent
            # ones); a graph capture does this for the carried parameters
            rsl.realize_all(p for _, p in model.named_parameters())
        loss.realize()
        return loss

    s0 = rsl._stats()
    step()
    s1 = rsl._stats()
    for _ in range(2):
        step()
    if graph:
        # the whole step (forward, backward, SGD) as one HIP graph launch
        g = rsl.hip.Graph()
        with g.capture(carry=model):
            loss = step()
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
    wall = time.perf_counter() - t0
    last = loss.tolist()[0]
    launches = (s1["eager_launches"] + s1["fused_launches"]
                - s0["eager_launches"] - s0["fused_launches"])
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
            "final_loss": last}


def cpu_baseline(seconds):
    from oracle import lamp_oracle as O
    a = np.random.default_rng(0).random((N8K, N8K), dtype=np.float32)
    b = np.random.default_rng(1).random((N8K, 1), dtype=np.float32)
    O.binary("add", O.binary("mul", a, a, fast=True), b, fast=True)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        O.binary("add", O.binary("mul", a, a, fast=True), b, fast=True)
        reps += 1
        el = time.perf_counter() - t0
        # about `seconds` of CPU work (the rep cap only bounds a very fast host)
        if (el >= seconds and reps >= 3) or reps >= 5000:
            break
    return {"value": round(BYTES_C1 * reps / el / 1e9, 2), "unit": "GB/s",
            "cores": O.num_threads(fast=True), "kind": "port",
            "sample": f"full config-1 workload (c = a*a + b, a [8192,8192], b [8192,1]) "
                      f"x {reps} reps, eager mul then broadcast add as Lamp3's CPU path "
                      f"runs it, liblamp_cpu_fast.so (-O3 -ffast-math, OpenMP), "
                      f"{el:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              f"(the Lamp3 path has no multi-GPU execution).", file=sys.stderr)
        sys.exit(2)
    ensure_built()
    import rushlite_amd as rsl
    from rushlite_amd import abi

    abi.check(abi.lib().lmp_rt_init(0))
    info = rsl.hip.device_info()
    evict = Evictor(rsl)
    a, b, per_step_ms, warm_ms, launches = headline(rsl, abi, args.steps, args.warmup, evict)
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
                               "hipRTC kernel per step",
                   "algorithmic_bytes_per_step": BYTES_C1,
                   "fused_launches_per_step": launches,
                   "device": f"{info['arch']} x{info['cu_count']} CUs"},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "warm_loop": {"ms_per_step": round(warm_ms, 5),
                      "GB/s": round(BYTES_C1 / warm_ms / 1e6, 1),
                      "note": "same steps back to back: part of a is still in the 256 MB "
                              "MALL from the previous step, so not all bytes come from HBM"},
    }
    if args.copy_probe:
        zero = rsl.Variable(np.zeros(1, np.float32))
        for _ in range(args.steps):
            evict()
            (a + zero).realize()
        abi.synchronize()
        line["copy_probe"] = {"kernel": "bin2d_f32 (x + 0)", "read_bytes": 4 * N8K * N8K,
                              "write_bytes": 4 * N8K * N8K, "launches": args.steps}
    if not args.no_extra:
        line["extra"] = extras(rsl, abi, a, b, args.steps, args.warmup, evict, args.only)
    del a, b, evict
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
