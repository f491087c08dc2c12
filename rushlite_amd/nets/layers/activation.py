"""Activations (src/rushlite/nets/layers/activation.py:8-40)."""
import sys

from ... import _C
from ..Module import Module

# ReLU is clamp(x, 0, DBL_MAX); in fp32 the upper bound becomes +inf, so NaN
# and -0.0 pass through unchanged and the gradient at 0 is 0.
_DBL_MAX = sys.float_info.max


class ReLU(Module):
    def forward(self, x):
        return _C.clamp(x, 0, _DBL_MAX)


class Sigmoid(Module):
    def forward(self, x):
        return 1 / (1 + _C.exp(-x))


class Tanh(Module):
    def forward(self, x):
        e_pos, e_neg = _C.exp(x), _C.exp(-x)
        return (e_pos - e_neg) / (e_pos + e_neg)


class Softmax(Module):
    """exp(x - max_d x) / sum_d exp(x - max_d x) with keep-dims broadcasts;
    the gradient also flows through the max (eq-mask), as in the reference."""

    def __init__(self, dim: int) -> None:
        super().__init__()
        self.dim = dim

    def forward(self, x):
        d = self.dim + x.ndim if self.dim < 0 else self.dim
        if not 0 <= d < x.ndim:
            raise ValueError("Dim not in bounds")
        shifted = x - _C.max(x, d)
        e = _C.exp(shifted)
        return e / _C.sum(e, d)
