"""Lamp3's Python API (the `rushlite` package surface) on the MI355X backend.

`import rushlite_amd as rsl` offers what `import rushlite as rsl` offers
(src/rushlite/__init__.py:1-9): Variable, the op functions, capture_on /
capture, no_grad, Module and nets.layers, with the GPU device being the
HIP backend (rsl.device.hip; rsl.device.cuda is the same device).

The compiled parts are in-tree shared libraries built by
`python rushlite_amd/build.py`; importing fails loudly when they are missing.
"""
from __future__ import annotations

try:
    from . import _C  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "rushlite_amd._C is not built; run `python rushlite_amd/build.py`"
    ) from e

from ._C import *  # noqa: F401,F403
from ._C import Variable
from ._C import _fused_source, _is_deferred, _stats, _storage_ptr  # noqa: F401
from .capture_mode import capture, capture_on
from .grad_mode import no_grad
from .graphs import Graph as _Graph
from .nets.Module import Module

# rsl.hip.Graph (and its rsl.cuda alias): whole-step HIP graphs.
hip.Graph = _Graph  # noqa: F405
cuda.Graph = _Graph  # noqa: F405

__all__ = ["Variable", "Module", "capture_on", "capture", "no_grad"]
