"""Restatement of Lamp3's CPU kernels for every dtype, in numpy.

TEST INFRASTRUCTURE ONLY: the parity checker for the device backend's bool /
int16 / int32 / int64 / float64 paths (and float32 where numpy's IEEE single
operations are the same arithmetic).  Only tests/ may import it; the product
never does.

Semantics restated (file:line in the reference):
  * dtype codes Bool=0 .. Float64=5 and promotion = max code
    (data_type.hpp:25-32, 77-80);
  * binary ops cast both operands to the output dtype, then apply the functor
    in that dtype (cpu/ptr_pack.hpp:9-35, cpu/binary.cpp:30-38,
    cpu/kernels.hpp:22-70): integers wrap modulo 2^bits, integer division
    truncates toward zero, bool arithmetic is C++'s (promote to int, convert
    back: nonzero -> true), comparisons yield 1/0 in the output dtype;
  * pow and the transcendentals run in the input precision for floating types
    and in double for integers, then convert back (math_acc_t,
    cpu/kernels.hpp:20-21, 38-113), float -> integer conversion truncating;
  * clamp converts its bounds to the tensor dtype (cpu/kernels.hpp:115-131);
  * reductions fold from Lamp3's identities (0, lowest(), max(), 1) with the
    functors of cpu/kernels.hpp:155-174 (std::max keeps the accumulator when
    the new value is NaN) in the input dtype (cpu/reduct.cpp:7-19);
  * matmul sums from 0 in the output dtype over static_cast<Out>(a) *
    static_cast<Out>(b) (cpu/matrix.cpp:8-18).

Integer division by zero (undefined in the reference) is defined here as 0,
as the device kernels define it; tests do not rely on either.
"""
from __future__ import annotations

import numpy as np

# DataType codes (data_type.hpp:25-32).
DTYPES = [np.dtype(np.bool_), np.dtype(np.int16), np.dtype(np.int32), np.dtype(np.int64),
          np.dtype(np.float32), np.dtype(np.float64)]
CODE = {dt: i for i, dt in enumerate(DTYPES)}


def upcast(a: np.dtype, b: np.dtype) -> np.dtype:
    """type_upcast (data_type.hpp:77-80)."""
    return DTYPES[max(CODE[np.dtype(a)], CODE[np.dtype(b)])]


def is_int(dt) -> bool:
    return np.dtype(dt).kind == "i"


def is_bool(dt) -> bool:
    return np.dtype(dt) == np.bool_


def cast(x, dt) -> np.ndarray:
    """static_cast<dt>: floats -> ints truncate toward zero; ints wrap;
    anything -> bool is (x != 0)."""
    x = np.asarray(x)
    dt = np.dtype(dt)
    if is_bool(dt):
        return x != 0
    with np.errstate(invalid="ignore", over="ignore"):
        if is_int(dt) and x.dtype.kind == "f":
            return np.trunc(x).astype(dt)
        return x.astype(dt)


def _trunc_div(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C++ integer division (truncation toward zero); b == 0 gives 0."""
    aa, bb = np.broadcast_arrays(a, b)
    out = np.zeros(aa.shape, a.dtype)
    nz = bb != 0
    q = np.abs(aa[nz].astype(np.int64)) // np.abs(bb[nz].astype(np.int64))
    neg = (aa[nz] < 0) != (bb[nz] < 0)
    out[nz] = np.where(neg, -q, q).astype(a.dtype)
    return out


_CMP = {"eq": np.equal, "ne": np.not_equal, "ge": np.greater_equal,
        "le": np.less_equal, "gt": np.greater, "lt": np.less}


def binary(op: str, a, b) -> np.ndarray:
    """Broadcast binary op (cpu/kernels.hpp:22-70, cpu/expand.cpp:7-46)."""
    a, b = np.asarray(a), np.asarray(b)
    out = upcast(a.dtype, b.dtype)
    a, b = cast(a, out), cast(b, out)
    if op in _CMP:
        return _CMP[op](a, b).astype(out)
    if is_bool(out):
        ia, ib = a.astype(np.int64), b.astype(np.int64)
        if op == "add":
            r = ia + ib
        elif op == "sub":
            r = ia - ib
        elif op == "mul":
            r = ia * ib
        elif op == "div":
            r = _trunc_div(ia, ib)
        elif op == "pow":
            r = np.power(ia.astype(np.float64), ib.astype(np.float64))
        else:
            raise ValueError(op)
        return r != 0
    with np.errstate(all="ignore"):
        if op == "add":
            return np.add(a, b, dtype=out)
        if op == "sub":
            return np.subtract(a, b, dtype=out)
        if op == "mul":
            return np.multiply(a, b, dtype=out)
        if op == "div":
            return _trunc_div(a, b) if is_int(out) else np.divide(a, b, dtype=out)
        if op == "pow":
            if is_int(out):
                return cast(np.power(a.astype(np.float64), b.astype(np.float64)), out)
            return np.power(a, b, dtype=out)
    raise ValueError(op)


_UN = {"exp": np.exp, "log": np.log, "sqrt": np.sqrt, "abs": np.abs, "sin": np.sin,
       "cos": np.cos, "tan": np.tan}


def unary(op: str, x, lo=0.0, hi=0.0) -> np.ndarray:
    """Unary functors (cpu/kernels.hpp:71-131); math in double for integers."""
    x = np.asarray(x)
    dt = x.dtype
    with np.errstate(all="ignore"):
        if op == "neg":
            if is_bool(dt):
                return x.copy()  # -(int)b converts back to b
            return np.negative(x)
        if op == "clamp":
            l, h = cast(np.float64(lo), dt), cast(np.float64(hi), dt)
            return np.where(x < l, l, np.where(x > h, h, x)).astype(dt)
        fn = _UN[op]
        if dt.kind == "f":
            return fn(x).astype(dt)
        return cast(fn(x.astype(np.float64)), dt)


def _identity(op: str, dt: np.dtype):
    if op == "sum":
        return dt.type(0)
    if op == "prod":
        return dt.type(1)
    if is_bool(dt):
        return dt.type(op == "min")
    info = np.finfo(dt) if dt.kind == "f" else np.iinfo(dt)
    return dt.type(info.min if op == "max" else info.max)


def reduce(op: str, x, axis: int) -> np.ndarray:
    """Keep-dims reduction folded sequentially from the identity
    (cpu/reduct.cpp:7-19, cpu/kernels.hpp:155-174)."""
    x = np.asarray(x)
    dt = x.dtype
    moved = np.moveaxis(x, axis, 0)
    acc = np.full(moved.shape[1:], _identity(op, dt), dt)
    with np.errstate(all="ignore"):
        for row in moved:
            if op == "sum":
                acc = (acc | row) if is_bool(dt) else np.add(acc, row, dtype=dt)
            elif op == "prod":
                acc = (acc & row) if is_bool(dt) else np.multiply(acc, row, dtype=dt)
            elif op == "max":  # std::max(acc, x) == (acc < x ? x : acc)
                acc = np.where(acc < row, row, acc)
            elif op == "min":  # std::min(acc, x) == (x < acc ? x : acc)
                acc = np.where(row < acc, row, acc)
            else:
                raise ValueError(op)
    return np.expand_dims(acc, axis)


def matmul(a, b) -> np.ndarray:
    """cpu/matrix.cpp:8-18 for integer and bool outputs (exact: modular sums
    and OR of ANDs, independent of order); float64 through numpy's float64
    product (order differs from the serial loop: compare with a tolerance)."""
    a, b = np.asarray(a), np.asarray(b)
    out = upcast(a.dtype, b.dtype)
    a, b = cast(a, out), cast(b, out)
    if is_bool(out):
        return (a.astype(np.int64) @ b.astype(np.int64)) != 0
    if is_int(out):
        # int64 products and sums wrap modulo 2^64, whose residue modulo
        # 2^bits is the narrower type's result.
        with np.errstate(over="ignore"):
            r = a.astype(np.int64) @ b.astype(np.int64)
        return r.astype(out)
    return np.matmul(a, b).astype(out)
