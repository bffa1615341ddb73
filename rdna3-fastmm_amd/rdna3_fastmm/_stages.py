"""One function per HIP stage: tensors in, a launch on the current stream out.

Shared by the plans (``runtime``) and the allocating operators (``linear``).
Callers validate shapes, dtypes and storage; these only marshal pointers. The
element types passed to the library are the tensors' own: transformed planes
and leaf operands in the plan's compute dtype, products likewise (or fp32).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .schemes import Scheme


def left_transform(scheme: Scheme, source: torch.Tensor, output: torch.Tensor, rows: int, inner: int) -> None:
    with torch.cuda.device(source.device):
        _native.call(
            "fastmm_left_transform",
            scheme.scheme_id,
            _native.dtype_code(source.dtype),
            _native.dtype_code(output.dtype),
            source.data_ptr(),
            output.data_ptr(),
            rows,
            inner,
            _native.stream_handle(source.device),
        )


def weight_transform(scheme: Scheme, weight: torch.Tensor, output: torch.Tensor, columns: int, inner: int) -> None:
    with torch.cuda.device(weight.device):
        _native.call(
            "fastmm_weight_transform",
            scheme.scheme_id,
            _native.dtype_code(weight.dtype),
            _native.dtype_code(output.dtype),
            weight.data_ptr(),
            output.data_ptr(),
            columns,
            inner,
            _native.stream_handle(weight.device),
        )


def right_transform(scheme: Scheme, right: torch.Tensor, output: torch.Tensor, inner: int, columns: int) -> None:
    with torch.cuda.device(right.device):
        _native.call(
            "fastmm_right_transform",
            scheme.scheme_id,
            _native.dtype_code(right.dtype),
            _native.dtype_code(output.dtype),
            right.data_ptr(),
            output.data_ptr(),
            inner,
            columns,
            _native.stream_handle(right.device),
        )


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
    with torch.cuda.device(left.device):
        _native.call(
            "fastmm_leaf_products",
            rank,
            _native.dtype_code(left.dtype),
            left.data_ptr(),
            right.data_ptr(),
            products.data_ptr(),
            _native.dtype_code(products.dtype),
            block_rows,
            block_inner,
            block_columns,
            None if scratch is None else scratch.data_ptr(),
            0 if scratch is None else scratch.numel() * scratch.element_size(),
            _native.stream_handle(left.device),
        )


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
    result = ctypes.c_int64(0)
    with torch.cuda.device(device):
        _native.call(
            "fastmm_leaf_scratch_bytes",
            rank,
            _native.dtype_code(operand_dtype),
            _native.dtype_code(products_dtype),
            block_rows,
            block_inner,
            block_columns,
            ctypes.byref(result),
        )
    return int(result.value)


def reconstruct(
    scheme: Scheme,
    products: torch.Tensor,
    bias: torch.Tensor | None,
    output: torch.Tensor,
    rows: int,
    columns: int,
) -> None:
    with torch.cuda.device(products.device):
        _native.call(
            "fastmm_reconstruct",
            scheme.scheme_id,
            _native.dtype_code(products.dtype),
            products.data_ptr(),
            None if bias is None else bias.data_ptr(),
            _native.dtype_code(output.dtype),
            output.data_ptr(),
            rows,
            columns,
            _native.stream_handle(products.device),
        )
