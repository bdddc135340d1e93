"""Backend registry: name -> OpExecutor factory.

Same behaviour as the reference's python_runtime/hal/registry.py:13-49:
duplicate names raise ValueError, unknown names raise KeyError.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Any

from python_runtime.hal.interface import OpExecutor

_registry: dict[str, Callable[..., OpExecutor]] = {}


def register(name: str, factory: Callable[..., OpExecutor]) -> None:
    """Registers `factory` under `name`; ValueError if the name is taken."""
    if name in _registry:
        raise ValueError(f"Backend '{name}' already registered")
    _registry[name] = factory


def create(name: str, **kwargs: Any) -> OpExecutor:
    """Calls the factory registered under `name`; KeyError if there is none."""
    factory = _registry.get(name)
    if factory is None:
        raise KeyError(f"Backend '{name}' not found")
    return factory(**kwargs)


def get(name: str) -> Callable[..., OpExecutor]:
    """The factory registered under `name`; KeyError if there is none."""
    if name not in _registry:
        raise KeyError(f"Backend '{name}' not found")
    return _registry[name]


def list_backends() -> list[str]:
    """Sorted names of the registered backends."""
    return sorted(_registry)
