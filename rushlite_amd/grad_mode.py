"""Gradient-recording switch (src/rushlite/grad_mode.py:5-22).

Only op recording is gated: results of ops made inside `no_grad()` have
requires_grad=False and no grad_fn.  Leaves built explicitly with
requires_grad=True still track gradients, and backward() on a graph built
outside the block still runs.  Works as a context manager or a decorator.
"""
from contextlib import contextmanager

from ._C import is_grad_enabled, set_grad_enabled


@contextmanager
def no_grad():
    saved = is_grad_enabled()
    set_grad_enabled(False)
    try:
        yield
    finally:
        set_grad_enabled(saved)
