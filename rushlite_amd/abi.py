"""ctypes binding of the C ABI in include/lmp_hip.h.

This is the thinnest possible caller of liblmp_hip.so: kernel-level parity
tests and the benchmark drive the backend through it, exactly as a Lamp3
``*_hip`` adapter would through the C header.  It raises ``LmpError`` with the
library's thread-local message on any non-zero status.  Loading the library
needs no GPU; the first call that touches the device does.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "liblmp_hip.so"

MAX_DIMS = 16

# enums (include/lmp_hip.h)
OK, ERR_INVALID, ERR_RUNTIME, ERR_OOM, ERR_UNSUPPORTED, ERR_JIT = range(6)
BOOL, INT16, INT32, INT64, FLOAT32, FLOAT64 = range(6)
BIN = dict(add=0, sub=1, mul=2, div=3, pow=4, eq=5, ne=6, ge=7, le=8, gt=9,
           lt=10, abs_backward=11, clamp_backward=12)
UN = dict(neg=0, exp=1, log=2, sqrt=3, abs=4, sin=5, cos=6, tan=7, clamp=8)
RED = dict(sum=0, max=1, min=2, prod=3)

NP_DTYPE = {BOOL: np.bool_, INT16: np.int16, INT32: np.int32, INT64: np.int64,
            FLOAT32: np.float32, FLOAT64: np.float64}
CODE_OF = {np.dtype(v): k for k, v in NP_DTYPE.items()}


class LmpError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"lmp status {status}: {msg}")
        self.status = status


class Bcast(C.Structure):
    _fields_ = [("ndim", C.c_int32),
                ("shape", C.c_int64 * MAX_DIMS),
                ("stride_a", C.c_int64 * MAX_DIMS),
                ("stride_b", C.c_int64 * MAX_DIMS)]


class DeviceInfo(C.Structure):
    _fields_ = [("device", C.c_int32), ("cu_count", C.c_int32),
                ("simd_per_cu", C.c_int32), ("wave_size", C.c_int32),
                ("lds_bytes_per_cu", C.c_int64), ("total_mem_bytes", C.c_int64),
                ("clock_khz", C.c_int32), ("mem_clock_khz", C.c_int32),
                ("mem_bus_width", C.c_int32), ("arch", C.c_char * 64),
                ("name", C.c_char * 128)]


class PoolStats(C.Structure):
    _fields_ = [("reserved_bytes", C.c_uint64), ("allocated_bytes", C.c_uint64),
                ("segments", C.c_uint64), ("allocs", C.c_uint64),
                ("device_mallocs", C.c_uint64)]


_vp, _sz, _i, _d = C.c_void_p, C.c_size_t, C.c_int, C.c_double

# name -> (restype, argtypes); every entry point declared in lmp_hip.h
SIGNATURES = {
    "lmp_rt_init": (_i, [_i]),
    "lmp_rt_device_count": (_i, [C.POINTER(_i)]),
    "lmp_rt_device_info": (_i, [C.POINTER(DeviceInfo)]),
    "lmp_rt_last_error": (C.c_char_p, []),
    "lmp_rt_abi_version": (_i, []),
    "lmp_rt_malloc": (_i, [C.POINTER(_vp), _sz]),
    "lmp_rt_free": (_i, [_vp]),
    "lmp_rt_empty_cache": (_i, []),
    "lmp_rt_pool_stats_get": (_i, [C.POINTER(PoolStats)]),
    "lmp_rt_kernel_launch_count": (_i, [C.POINTER(C.c_uint64)]),
    "lmp_rt_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "lmp_rt_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "lmp_rt_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "lmp_rt_synchronize": (_i, []),
    "lmp_rt_stream": (_vp, []),
    "lmp_rt_event_create": (_i, [C.POINTER(_vp)]),
    "lmp_rt_event_record": (_i, [_vp]),
    "lmp_rt_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(C.c_float)]),
    "lmp_rt_event_destroy": (_i, [_vp]),
    "lmp_rt_graph_begin": (_i, []),
    "lmp_rt_graph_end": (_i, [C.POINTER(_vp)]),
    "lmp_rt_graph_abort": (_i, []),
    "lmp_rt_graph_launch": (_i, [_vp]),
    "lmp_rt_graph_destroy": (_i, [_vp]),
    "lmp_k_binary": (_i, [_i, _i, _vp, _vp, _vp, C.POINTER(Bcast), _d, _d]),
    "lmp_k_unary": (_i, [_i, _i, _vp, _vp, _sz, _d, _d]),
    "lmp_k_fill": (_i, [_i, _vp, _sz, _d]),
    "lmp_k_cast": (_i, [_i, _i, _vp, _vp, _sz]),
    "lmp_k_add_inplace": (_i, [_i, _vp, _vp, _sz]),
    "lmp_k_reduce": (_i, [_i, _i, _vp, _vp, _sz, _sz, _sz]),
    "lmp_k_gemm_f32": (_i, [_i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp,
                            _sz, _i]),
    "lmp_k_gemm_f32_noalloc": (_i, [_i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp,
                                    _sz, _i]),
    "lmp_k_gemm": (_i, [_i, _i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _i]),
    "lmp_k_linear_f32": (_i, [_i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _sz]),
    "lmp_k_linear_relu_f32": (_i, [_i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _sz]),
    "lmp_k_gemm_colsum_f32": (_i, [_i, _i, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _i,
                                   _vp, _i]),
    "lmp_k_gemm_colsum_masked_f32": (_i, [_i, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _sz, _vp, _sz,
                                          _i, _vp, _i]),
    "lmp_k_linear_backward_f32": (_i, [_sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz,
                                       _i, _vp, _sz, _i, _vp, _i]),
    "lmp_k_transpose": (_i, [_i, _vp, _vp, _sz, _sz]),
    "lmp_jit_lookup": (_i, [C.c_uint64, C.POINTER(_vp)]),
    "lmp_jit_compile": (_i, [C.c_uint64, C.c_char_p, C.c_char_p,
                             C.POINTER(_vp)]),
    "lmp_jit_launch": (_i, [_vp, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "lmp_jit_compiled_count": (_i, [C.POINTER(C.c_uint64)]),
    "lmp_jit_disk_loaded_count": (_i, [C.POINTER(C.c_uint64)]),
}

_lib = None


def lib() -> C.CDLL:
    """Load liblmp_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python rushlite_amd/build.py hip`")
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise LmpError(status, lib().lmp_rt_last_error().decode(errors="replace"))


def device_info() -> DeviceInfo:
    info = DeviceInfo()
    check(lib().lmp_rt_device_info(C.byref(info)))
    return info


class DeviceBuffer:
    """A pooled device allocation holding a numpy-typed array."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().lmp_rt_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.shape, arr.dtype)
        if buf.nbytes:
            check(lib().lmp_rt_memcpy_h2d(buf.ptr, arr.ctypes.data, buf.nbytes))
        return buf

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().lmp_rt_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    @property
    def code(self) -> int:
        return CODE_OF[self.dtype]

    def free(self) -> None:
        if self.ptr:
            check(lib().lmp_rt_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.lmp_rt_free(self.ptr)
        except Exception:
            pass


def padded_strides(in_shape, out_shape):
    """Element strides of a contiguous `in_shape` aligned right to
    `out_shape`, 0 where the input broadcasts (cpu/offset_util.cpp:7-28)."""
    in_shape = list(in_shape)
    nd = len(out_shape)
    contig = [0] * len(in_shape)
    s = 1
    for i in range(len(in_shape) - 1, -1, -1):
        contig[i] = s
        s *= in_shape[i]
    out = [0] * nd
    for k in range(len(in_shape)):
        dst, src = nd - 1 - k, len(in_shape) - 1 - k
        if in_shape[src] != 1:
            out[dst] = contig[src]
    return out


def broadcast_shape(a_shape, b_shape):
    nd = max(len(a_shape), len(b_shape))
    out = []
    for i in range(nd):
        av = a_shape[i - (nd - len(a_shape))] if i >= nd - len(a_shape) else 1
        bv = b_shape[i - (nd - len(b_shape))] if i >= nd - len(b_shape) else 1
        if av != 1 and bv != 1 and av != bv:
            raise ValueError("broadcast rule violation")
        out.append(av if av != 1 else bv)
    return out


def make_bcast(a_shape, b_shape) -> tuple[Bcast, list[int]]:
    out_shape = broadcast_shape(a_shape, b_shape)
    d = Bcast()
    d.ndim = len(out_shape)
    sa = padded_strides(a_shape, out_shape)
    sb = padded_strides(b_shape, out_shape)
    for i, n in enumerate(out_shape):
        d.shape[i] = n
        d.stride_a[i] = sa[i]
        d.stride_b[i] = sb[i]
    return d, out_shape


# ---------------------------------------------------------------- wrappers

def binary(op: str, a: DeviceBuffer, b: DeviceBuffer, p0=0.0, p1=0.0) -> DeviceBuffer:
    d, out_shape = make_bcast(a.shape, b.shape)
    out = DeviceBuffer(out_shape, a.dtype)
    check(lib().lmp_k_binary(BIN[op], a.code, out.ptr, a.ptr, b.ptr, C.byref(d),
                             p0, p1))
    return out


def unary(op: str, a: DeviceBuffer, p0=0.0, p1=0.0) -> DeviceBuffer:
    out = DeviceBuffer(a.shape, a.dtype)
    check(lib().lmp_k_unary(UN[op], a.code, out.ptr, a.ptr,
                            int(np.prod(a.shape, dtype=np.int64)), p0, p1))
    return out


def reduce(op: str, a: DeviceBuffer, axis: int) -> DeviceBuffer:
    shape = list(a.shape)
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    length = shape[axis]
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    oshape = shape.copy()
    oshape[axis] = 1
    out = DeviceBuffer(oshape, a.dtype)
    check(lib().lmp_k_reduce(RED[op], a.code, out.ptr, a.ptr, outer, length, inner))
    return out


def gemm(a: DeviceBuffer, b: DeviceBuffer, trans_a=False, trans_b=False,
         out: DeviceBuffer | None = None, accumulate=False) -> DeviceBuffer:
    if trans_a:
        k, m = a.shape
    else:
        m, k = a.shape
    if trans_b:
        n, kb = b.shape
    else:
        kb, n = b.shape
    if kb != k:
        raise ValueError("gemm: inner dimensions differ")
    if a.dtype != b.dtype:
        raise ValueError("gemm: operands must share a dtype")
    if out is None:
        out = DeviceBuffer((m, n), a.dtype)
    if a.dtype == np.float32:
        check(lib().lmp_k_gemm_f32(int(trans_a), int(trans_b), m, n, k, a.ptr,
                                   a.shape[1], b.ptr, b.shape[1], out.ptr, n,
                                   int(accumulate)))
    else:
        check(lib().lmp_k_gemm(a.code, int(trans_a), int(trans_b), m, n, k, a.ptr,
                               a.shape[1], b.ptr, b.shape[1], out.ptr, n, int(accumulate)))
    return out


def synchronize() -> None:
    check(lib().lmp_rt_synchronize())


class Timer:
    """HIP events on the library stream."""

    def __init__(self):
        self.start, self.stop = C.c_void_p(), C.c_void_p()
        check(lib().lmp_rt_event_create(C.byref(self.start)))
        check(lib().lmp_rt_event_create(C.byref(self.stop)))

    def begin(self):
        check(lib().lmp_rt_event_record(self.start))

    def end(self) -> float:
        check(lib().lmp_rt_event_record(self.stop))
        ms = C.c_float()
        check(lib().lmp_rt_event_elapsed_ms(self.start, self.stop, C.byref(ms)))
        return ms.value
