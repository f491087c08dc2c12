"""Module base class with functional parameter updates.

Behaviour follows src/rushlite/nets/Module.py:7-177: Variables and child
Modules assigned as attributes live only in the instance's ``_params_dict``
(never in ``__dict__``), so attribute access, ``parameters()`` and the
``params`` view always agree, and rebinding a parameter through
``model.params["layer.name"] = Variable(...)`` is seen by ``forward`` at once.
Assigning a non-parameter value under a parameter's name removes the
parameter.  ``params`` assignment keeps the value's requires_grad flag, so a
value computed under ``no_grad()`` stays frozen unless re-wrapped with
``Variable(v.data, requires_grad=True)``.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any, Iterator

from .._C import Variable

_STORE = "_params_dict"


class Module(ABC):
    def __init__(self) -> None:
        object.__setattr__(self, _STORE, {})

    @abstractmethod
    def forward(self, *args: Any, **kwargs: Any) -> Any:
        ...

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward(*args, **kwargs)

    # -- attribute routing -------------------------------------------------
    def _store(self, name: str) -> dict:
        store = self.__dict__.get(_STORE)
        if store is None:
            raise AttributeError(
                f"{type(self).__name__!r} object has no attribute {name!r}: "
                "call super().__init__() before assigning/accessing parameters")
        return store

    def __setattr__(self, name: str, value: Any) -> None:
        if isinstance(value, (Module, Variable)):
            self._store(name)[name] = value
            return
        store = self.__dict__.get(_STORE)
        if store is not None:
            store.pop(name, None)  # a plain value shadows (removes) a parameter
        object.__setattr__(self, name, value)

    def __getattr__(self, name: str) -> Any:
        store = self._store(name)
        try:
            return store[name]
        except KeyError:
            raise AttributeError(
                f"{type(self).__name__!r} object has no attribute {name!r}") from None

    def __delattr__(self, name: str) -> None:
        store = self.__dict__.get(_STORE)
        if store is not None and name in store:
            del store[name]
        else:
            object.__delattr__(self, name)

    # -- parameter traversal -----------------------------------------------
    def named_parameters(self, _prefix: str = "") -> Iterator[tuple[str, Variable]]:
        for key, val in self._store("named_parameters").items():
            path = f"{_prefix}{key}"
            if isinstance(val, Variable):
                yield path, val
            elif isinstance(val, Module):
                yield from val.named_parameters(path + ".")
            else:
                raise TypeError(f"unexpected entry {path!r} in parameter store")

    def parameters(self) -> Iterator[Variable]:
        for _, p in self.named_parameters():
            yield p

    @property
    def params(self) -> "ParamsView":
        """Dict-like view keyed by the dotted names of named_parameters()."""
        return ParamsView(self)

    def zero_grad(self) -> None:
        for p in self.parameters():
            if p.requires_grad:
                p.zero_grad()

    def to(self) -> None:
        """Kept for API compatibility; parameters are created on the device."""


class ParamsView:
    """Mapping from dotted parameter paths to Variables of a Module tree."""

    def __init__(self, module: Module) -> None:
        self._root = module

    def _owner(self, key: str) -> tuple[Module, str]:
        *path, leaf = key.split(".")
        mod = self._root
        for part in path:
            nxt = mod.__dict__[_STORE].get(part)
            if not isinstance(nxt, Module):
                raise KeyError(key)
            mod = nxt
        return mod, leaf

    def __getitem__(self, key: str) -> Variable:
        mod, leaf = self._owner(key)
        val = mod.__dict__[_STORE].get(leaf)
        if not isinstance(val, Variable):
            raise KeyError(key)
        return val

    def __setitem__(self, key: str, value: Variable) -> None:
        if not isinstance(value, Variable):
            raise TypeError(f"can only assign a Variable to parameter {key!r}, "
                            f"got {type(value).__name__}")
        mod, leaf = self._owner(key)
        setattr(mod, leaf, value)

    def __contains__(self, key: object) -> bool:
        try:
            self[key]  # type: ignore[index]
            return True
        except (KeyError, TypeError, AttributeError):
            return False

    def __iter__(self) -> Iterator[str]:
        return (name for name, _ in self._root.named_parameters())

    def __len__(self) -> int:
        return sum(1 for _ in self)

    def keys(self) -> Iterator[str]:
        return iter(self)

    def items(self) -> Iterator[tuple[str, Variable]]:
        return self._root.named_parameters()

    def __repr__(self) -> str:
        return f"params({list(self)})"
