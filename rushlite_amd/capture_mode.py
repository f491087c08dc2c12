"""Kernel-fusion capture switches (src/rushlite/capture_mode.py:6-30).

Inside `capture_on()` (or a function decorated with `capture()`), elementwise
ops on GPU tensors are recorded lazily instead of launched; the pending graph
is compiled into one fused HIP kernel the first time its values are needed,
wherever that happens.
"""
from contextlib import contextmanager
from functools import wraps

from ._C import is_capture_enabled, set_capture_enabled


@contextmanager
def capture_on(enable: bool = True):
    saved = is_capture_enabled()
    set_capture_enabled(enable)
    try:
        yield
    finally:
        set_capture_enabled(saved)


def capture(enable: bool = True):
    """Decorator form of capture_on."""
    def wrap(fn):
        @wraps(fn)
        def inner(*args, **kwargs):
            with capture_on(enable):
                return fn(*args, **kwargs)
        return inner
    return wrap
