"""HAL abstract interfaces, same contract as the reference's
python_runtime/hal/interface.py:10-72 (Device, Buffer, OpExecutor).

A backend written against the reference's OpExecutor runs unchanged
against these classes and vice versa: `execute(op_name, inputs, **kwargs)`
returns a tensor; the optional extensions raise NotImplementedError unless
a backend supports them.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    import torch


class Device(ABC):
    """A compute device."""

    @abstractmethod
    def synchronize(self) -> None:
        """Blocks until all work submitted to the device has finished."""


class Buffer(ABC):
    """A block of device memory."""

    @property
    @abstractmethod
    def data_ptr(self) -> int:
        """Address of the underlying memory."""

    @abstractmethod
    def copy_from(self, src: torch.Tensor) -> None:
        """Copies src into this buffer."""

    @abstractmethod
    def copy_to(self, dst: torch.Tensor) -> None:
        """Copies this buffer into dst."""

    @abstractmethod
    def create_tensor(self, shape: Any, dtype: Any, device: Any) -> torch.Tensor:
        """A tensor view over this buffer's memory."""


class OpExecutor(ABC):
    """Runs named operators on a device."""

    @abstractmethod
    def execute(self, op_name: str, inputs: list[Any], **kwargs: Any) -> torch.Tensor:
        """Runs op `op_name` on `inputs` and returns the result tensor."""

    def async_copy(self, src: Any, dst: Any, byte_count: int) -> None:  # noqa: B027
        raise NotImplementedError("async_copy not supported")

    def memory_retrieve(self, key: Any, table: Any) -> torch.Tensor:  # noqa: B027
        raise NotImplementedError("memory_retrieve not supported")

    def send_kv_cache(self, blocks: Any, target_device: str) -> None:  # noqa: B027
        raise NotImplementedError("send_kv_cache not supported")
