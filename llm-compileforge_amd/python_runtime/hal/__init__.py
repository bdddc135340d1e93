"""Hardware abstraction layer: OpExecutor contract, backend registry and
the HIP backend for the paged-attention path."""

from python_runtime.hal.interface import Buffer, Device, OpExecutor

__all__ = ["Buffer", "Device", "OpExecutor"]
