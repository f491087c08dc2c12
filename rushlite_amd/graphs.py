"""Whole-step HIP graphs: record a training (or inference) step once, replay it
with a single launch.

The reference launches every kernel of a step from the host; on the MI355X
the README MLP step (about 54 small kernels) is bound by that host work.  A
`Graph` captures everything the library stream receives inside its `capture()`
block -- eager kernels, fused hipRTC kernels, GEMMs, split-K folds -- and
`replay()` re-issues all of it as one hipGraphLaunch.

    x, y = rsl.Variable(x_np), rsl.Variable(y_np)   # static inputs
    step()                                          # warm-up: compiles kernels
    graph = rsl.hip.Graph()
    with graph.capture(carry=model):
        loss = step()
    for _ in range(100):
        graph.replay()
    print(loss.tolist())

Rules, as for any stream capture:
  * The capture records work without running it; tensors produced inside hold
    their values only after a replay.
  * Buffers made inside the capture come from the graph's own memory pool and
    stay valid while the graph lives; each replay writes the same addresses.
  * Inputs made before the capture (x and y above, the parameters) are read at
    their addresses by every replay: update them in place (`Tensor.copy`,
    `Tensor.fill`) rather than rebinding them.  Realise pending (captured)
    inputs before the capture; the carried parameters are realised for you.
  * Host round trips (building a Variable from host data, `tolist()`,
    `numpy()`, synchronising) raise inside a capture.
  * `carry` handles functional parameter updates (`model.params[name] =
    Variable(p.data - lr * p.grad)`): for every parameter whose Variable the
    step replaced, the new value ends up in the old buffer, so the next replay
    reads the updated parameters.  An update made under `capture_on()` is
    still pending when the capture ends and is computed straight into the old
    buffer (one fused kernel, no extra traffic); an eager update is copied
    there.  `carry` takes a Module, a mapping of Variables, or a callable
    returning one.
"""
from __future__ import annotations

from contextlib import contextmanager

from . import _C


def _snapshot(carry):
    if carry is None:
        return {}
    if callable(getattr(carry, "named_parameters", None)):
        return dict(carry.named_parameters())
    if callable(carry):
        return dict(carry())
    return dict(carry.items())


class Graph:
    """One captured step.  See the module docstring."""

    def __init__(self):
        self._g = _C.hip._Graph()
        self._hold = []

    @property
    def captured(self) -> bool:
        return self._g.captured

    @contextmanager
    def capture(self, carry=None):
        if self._g.captured or self._g.capturing:
            raise RuntimeError("graph: already captured (make a new Graph)")
        before = _snapshot(carry)
        # Pending updates from an earlier eager step belong outside the graph.
        for v in before.values():
            v.realize()
        _C.hip.sync()
        self._g.begin()
        try:
            yield self
            after = _snapshot(carry)
            dsts, srcs = [], []
            for name, old in before.items():
                new = after.get(name)
                if new is None or new is old:
                    continue
                src, dst = new.data, old.data
                if _C._storage_ptr(src) != _C._storage_ptr(dst):
                    dsts.append(dst)
                    srcs.append(src)
            if dsts:
                # Pending fused updates (made under capture_on) are computed
                # straight into the old buffers, together in one kernel where
                # they are independent; anything else is copied there.
                _C._realize_into_many(dsts, srcs)
            self._g.end()
        except BaseException:
            self._g.abort()
            raise
        # The old parameter buffers are the graph's inputs: keep them alive.
        self._hold = [before, _snapshot(carry)]

    def replay(self) -> None:
        """Enqueue one replay on the library stream (asynchronous)."""
        self._g.launch()
