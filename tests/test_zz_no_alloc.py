"""The no-allocation GEMM entry point (lmp_k_gemm_f32_noalloc) against the
allocating one (lmp_k_gemm_f32), through the C ABI.

The two run the same kernels with the same split of K, so their results must
agree bit for bit; the no-allocation calls must leave the pool's allocation
counters unchanged, and a product whose split-K partials exceed the fixed
workspace must be refused with a clear error (and still be served by the
allocating entry point)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pool(hip):
    st = hip.PoolStats()
    hip.check(hip.lib().lmp_rt_pool_stats_get(C.byref(st)))
    return st.allocs, st.device_mallocs


def _case(hip, m, n, k, ta, tb, accumulate, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((k, m) if ta else (m, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((n, k) if tb else (k, n)) * 0.02).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    da, db = hip.DeviceBuffer.from_numpy(a), hip.DeviceBuffer.from_numpy(b)
    ref, out = hip.DeviceBuffer.from_numpy(c0), hip.DeviceBuffer.from_numpy(c0)
    lda, ldb = a.shape[1], b.shape[1]
    return da, db, ref, out, lda, ldb


# Two calls in a row, the second with a smaller product: config 4's layer
# (512 x 4096 x 4096, K split four ways: 32 MiB of partials, the workspace's
# whole size), then config 3's skinny forward (K split eight ways), then the
# same orientation with accumulation into C.
@pytest.mark.parametrize("calls", [
    [(512, 4096, 4096, 0, 0, 0), (32, 4096, 8192, 0, 0, 0)],
    [(512, 4096, 4096, 0, 1, 1), (33, 1000, 4096, 0, 0, 1)],
], ids=["fwd", "dX_accumulate"])
def test_noalloc_gemm_matches_allocating_entry(hip, calls):
    L = hip.lib()
    for i, (m, n, k, ta, tb, acc) in enumerate(calls):
        da, db, ref, out, lda, ldb = _case(hip, m, n, k, ta, tb, acc, 100 + i)
        hip.check(L.lmp_k_gemm_f32(ta, tb, m, n, k, da.ptr, lda, db.ptr, ldb, ref.ptr, n, acc))
        hip.synchronize()
        before = _pool(hip)
        hip.check(L.lmp_k_gemm_f32_noalloc(ta, tb, m, n, k, da.ptr, lda, db.ptr, ldb,
                                           out.ptr, n, acc))
        hip.synchronize()
        assert _pool(hip) == before, (m, n, k)
        got, want = out.numpy(), ref.numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, n, k)


def test_noalloc_gemm_refuses_partials_above_the_workspace(hip):
    """1920 x 1920 x 4096 with A's rows padded to 4097 values (no 16-byte
    rows, so the register-staged 128 x 128 tiles) splits K three ways: 44 MB
    of partials, more than the 32 MiB workspace."""
    L = hip.lib()
    m = n = 1920
    k, lda = 4096, 4097
    rng = np.random.default_rng(7)
    a = (rng.standard_normal((m, lda)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    da, db = hip.DeviceBuffer.from_numpy(a), hip.DeviceBuffer.from_numpy(b)
    ref, out = (hip.DeviceBuffer.from_numpy(np.zeros((m, n), np.float32)) for _ in range(2))
    before = _pool(hip)
    st = L.lmp_k_gemm_f32_noalloc(0, 0, m, n, k, da.ptr, lda, db.ptr, n, out.ptr, n, 0)
    assert st == hip.ERR_UNSUPPORTED
    msg = L.lmp_rt_last_error().decode()
    assert "no-allocation workspace" in msg and str(32 << 20) in msg, msg
    assert _pool(hip) == before
    hip.check(L.lmp_k_gemm_f32(0, 0, m, n, k, da.ptr, lda, db.ptr, n, ref.ptr, n, 0))
    want = a[:64, :k].astype(np.float64) @ b.astype(np.float64)
    got = ref.numpy()[:64]
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= 1e-4
