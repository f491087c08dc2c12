"""Dropout as Lamp3 defines it: (rand < p) * x, unscaled
(src/rushlite/nets/layers/dropout.py:7-14)."""
from ... import _C
from ..Module import Module


class Dropout(Module):
    def __init__(self, p: float) -> None:
        super().__init__()
        self.p = p

    def forward(self, x):
        keep = _C.rand(x.shape, device=x.device, dtype=x.dtype) < self.p
        return keep * x
