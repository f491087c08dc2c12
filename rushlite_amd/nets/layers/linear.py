"""Linear and Flatten (src/rushlite/nets/layers/linear.py:6-56).

Linear keeps Lamp3's layout: weights are [in, out] and forward is
x @ W + b; both start as randn(0, 1).
"""
from ... import _C
from ..Module import Module


class Linear(Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device=None, dtype=None) -> None:
        super().__init__()
        kw = {}
        if device is not None:
            kw["device"] = device
        if dtype is not None:
            kw["dtype"] = dtype
        self.requires_bias = bias
        self.weights = _C.randn(0, 1, [in_features, out_features], requires_grad=True, **kw)
        if bias:
            self.bias = _C.randn(0, 1, [out_features], requires_grad=True, **kw)

    def forward(self, x):
        # x @ W + b with the bias added in the GEMM's epilogue (one launch,
        # the same values as matmul followed by the broadcast add)
        if self.requires_bias:
            return _C.linear(x, self.weights, self.bias)
        return _C.matmul(x, self.weights)

    def forward_relu(self, x):
        """relu(forward(x)) as one node (Sequential's Linear -> ReLU pairs)."""
        return _C.linear_relu(x, self.weights, self.bias)


class Flatten(Module):
    def __init__(self, start_dim: int = 1, end_dim: int = -1) -> None:
        super().__init__()
        if start_dim < 0:
            raise ValueError("Start dim must be non-negative")
        self.start_dim = start_dim
        self.end_dim = end_dim

    def forward(self, x):
        end = self.end_dim + x.ndim if self.end_dim < 0 else self.end_dim
        if not self.start_dim < end:
            raise ValueError("Start and end dims not valid")
        shape = list(x.shape)
        merged = 1
        for d in shape[self.start_dim:end + 1]:
            merged *= d
        return _C.reshape(x, shape[:self.start_dim] + [merged] + shape[end + 1:])
