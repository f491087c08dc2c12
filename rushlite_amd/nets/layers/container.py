"""Sequential (src/rushlite/nets/layers/container.py:6-19).

A Linear layer (with bias) followed directly by a ReLU runs as one
`linear_relu` node: on the HIP device one GEMM whose epilogue adds the bias
and applies ReLU, with the values and gradients of the two layers run one
after the other.
"""
from ..Module import Module
from .activation import ReLU
from .linear import Linear


def _linear_relu_pair(layer, nxt) -> bool:
    # Exact classes with their own forward, so a subclass or an instance that
    # replaces forward keeps its behaviour.
    return (type(layer) is Linear and type(nxt) is ReLU and layer.requires_bias
            and "forward" not in vars(layer) and "forward" not in vars(nxt))


class Sequential(Module):
    def __init__(self, layers) -> None:
        super().__init__()
        self.layers = list(layers)
        for i, layer in enumerate(self.layers):
            self._params_dict[str(i)] = layer

    def forward(self, *args):
        if not self.layers:
            raise ValueError("Must have at least one layer")
        layers, n = self.layers, len(self.layers)
        i, out = 0, None
        while i < n:
            layer = layers[i]
            if i + 1 < n and (i > 0 or len(args) == 1) and _linear_relu_pair(layer, layers[i + 1]):
                out = layer.forward_relu(args[0] if i == 0 else out)
                i += 2
                continue
            out = layer(*args) if i == 0 else layer(out)
            i += 1
        return out
