"""bench.py's CPU-side logic (no GPU): the README-MLP loss envelope that
places the GPU's trajectory among valid summation orders on the CPU, and the
--gpus guard.  The oracle here is the checker, as in bench.py's cpu_baseline."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from oracle import lamp_oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def problem():
    x0, y0, w0, b0 = bench.mlp_problem(bench.C0_DIMS, bench.C0_BATCH, onehot=False)
    steps = 40
    with O.fast_build():
        fast = O.mlp_train(w0, b0, x0, y0, steps=steps)[0]
    seq = O.mlp_train(w0, b0, x0, y0, steps=steps)[0]
    return x0, y0, w0, b0, steps, fast, np.array(seq)


def test_envelope_holds_a_valid_order(problem):
    """A trajectory that is one of the CPU orders lies in the band at every
    step, with no gap to that order."""
    x0, y0, w0, b0, steps, fast, seq = problem
    env = bench._c0_envelope(O, x0, y0, w0, b0, steps, fast, list(seq))
    assert env["within_envelope"] and env["gpu_steps_inside_band"] == steps
    assert env["gpu_outside_band_rel_max"] == 0.0 and env["max_gap_over_steps"] == 0.0
    assert len(env["orders"]) == len(O.GEMM_ORDERS) + 1
    # the band opens up as the orders drift apart
    w = env["band_width_rel_at_step"]
    assert w["1"] < 1e-6 < w[str(steps)]


def test_envelope_rejects_a_drifting_trajectory(problem):
    """A trajectory 20% off the sequential order from the first step is
    outside the band by more than the band's width and is reported so."""
    x0, y0, w0, b0, steps, fast, seq = problem
    env = bench._c0_envelope(O, x0, y0, w0, b0, steps, fast, list(seq * 1.2))
    assert not env["within_envelope"]
    assert env["gpu_steps_inside_band"] == 0
    assert env["max_gap_over_steps"] == pytest.approx(0.2, rel=1e-9)
    # without GPU losses the band is still reported
    bare = bench._c0_envelope(O, x0, y0, w0, b0, steps, fast, None)
    assert "within_envelope" not in bare and bare["band_width_rel_max_over_steps"] > 0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
