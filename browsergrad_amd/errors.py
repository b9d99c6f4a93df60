"""Error types of the HIP realizer.

They mirror the reference's error surface:
  * ``KernelError``          -- packages/browsergrad-kernels/src/types.ts:87-92,
                                raised by the bridge with an op-qualified message;
  * ``RealizationError``     -- packages/browsergrad-jit/src/python/_errors.py,
                                raised by the walker when an op fails
                                (_realize_webgpu.py:415-424);
  * ``JitNotImplementedError`` -- unsupported opcode / no bridge registered
                                (_realize_webgpu.py:407-414, jit index.ts:366-381).
"""
from __future__ import annotations


class KernelError(RuntimeError):
    """Bridge-level failure (bad handle, dtype, shape, HIP runtime error)."""

    def __init__(self, message: str, code: int | None = None) -> None:
        super().__init__(message)
        self.code = code


class RealizationError(RuntimeError):
    """A UOp failed to realize."""


class JitNotImplementedError(NotImplementedError):
    """The realizer does not support this opcode / configuration."""


class ShapeError(ValueError):
    """Shape inference failed while building the graph."""
