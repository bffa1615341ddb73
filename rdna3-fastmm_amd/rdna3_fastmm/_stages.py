"""One function per HIP stage: tensors in, a launch on the current stream out.

Shared by the plans (``runtime``). Each calls the PyTorch-ROCm extension's
operator for one C-ABI entry point (``torch.ops.rdna3_fastmm_hip.*``, see
``csrc/torch_ops.cpp``), which launches on the current HIP stream of the
tensors' device. Callers validate shapes, dtypes and storage; these only pass
tensors through. The element types the library sees are the tensors' own:
transformed planes and leaf operands in the plan's compute dtype, products
likewise (or fp32).
"""

from __future__ import annotations

import torch

from ._torch_ops import stages
from .schemes import Scheme


def left_transform(scheme: Scheme, source: torch.Tensor, output: torch.Tensor, rows: int, inner: int) -> None:
    stages.left_transform(scheme.scheme_id, source, output, rows, inner)


def weight_transform(scheme: Scheme, weight: torch.Tensor, output: torch.Tensor, columns: int, inner: int) -> None:
    stages.weight_transform(scheme.scheme_id, weight, output, columns, inner)


def right_transform(scheme: Scheme, right: torch.Tensor, output: torch.Tensor, inner: int, columns: int) -> None:
    stages.right_transform(scheme.scheme_id, right, output, inner, columns)


def leaf_products(
    rank: int,
    left: torch.Tensor,
    right: torch.Tensor,
    products: torch.Tensor,
    block_rows: int,
    block_inner: int,
    block_columns: int,
    scratch: torch.Tensor | None = None,
) -> None:
    """``scratch`` (bytes on the same device, or None): the split-K tail's fp32 parts."""
    stages.leaf_products(rank, left, right, products, block_rows, block_inner, block_columns, scratch)


def leaf_scratch_bytes(
    rank: int,
    operand_dtype: torch.dtype,
    products_dtype: torch.dtype,
    block_rows: int,
    block_inner: int,
    block_columns: int,
    device: torch.device,
) -> int:
    """Scratch bytes the leaf products can use for this shape on ``device`` (0: none)."""
    return int(stages.leaf_scratch_bytes(rank, operand_dtype, products_dtype, block_rows, block_inner,
                                         block_columns, device))


def reconstruct(
    scheme: Scheme,
    products: torch.Tensor,
    bias: torch.Tensor | None,
    output: torch.Tensor,
    rows: int,
    columns: int,
) -> None:
    stages.reconstruct(scheme.scheme_id, products, bias, output, rows, columns)
