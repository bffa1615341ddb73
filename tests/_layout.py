"""Conversions between logical operand planes and the kernels' operand layout.

The oracle works on logical planes ``[R, rows, Kb]``. The HIP kernels store
transformed operands K-slab-major when ``Kb % 32 == 0`` (element (row, k) of a
plane at ``((k // 32) * rows + row) * 32 + k % 32``), else row-major; see
``rdna3_fastmm.runtime.operand_shape``.
"""

from __future__ import annotations

import numpy as np

SLAB = 32


def from_operand(buffer: np.ndarray, rank: int, rows: int, inner: int) -> np.ndarray:
    """Operand buffer (any shape, operand order) -> logical planes [R, rows, inner]."""
    flat = np.ascontiguousarray(buffer).reshape(-1)
    if inner % SLAB == 0:
        return flat.reshape(rank, inner // SLAB, rows, SLAB).transpose(0, 2, 1, 3).reshape(rank, rows, inner)
    return flat.reshape(rank, rows, inner)


def to_operand(planes: np.ndarray) -> np.ndarray:
    """Logical planes [R, rows, inner] -> operand buffer in the kernels' order."""
    rank, rows, inner = planes.shape
    if inner % SLAB == 0:
        return np.ascontiguousarray(planes.reshape(rank, rows, inner // SLAB, SLAB).transpose(0, 2, 1, 3))
    return np.ascontiguousarray(planes)
