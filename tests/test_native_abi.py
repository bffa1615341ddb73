"""The C ABI library: loads without a GPU, exports every declared symbol, reports
argument errors before any launch, and carries the verified certificates' digests."""

import ctypes
from pathlib import Path
import re

import pytest

from rdna3_fastmm import _native
from rdna3_fastmm.schemes import SCHEME_KEYS, load_scheme

HEADER = Path(__file__).resolve().parent.parent / "include" / "fastmm_amd.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fastmm_\w+)\s*\(", text, re.M)))


def test_header_declares_the_stage_entry_points() -> None:
    names = declared_functions()
    for required in (
        "fastmm_left_transform",
        "fastmm_weight_transform",
        "fastmm_right_transform",
        "fastmm_leaf_products",
        "fastmm_leaf_scratch_bytes",
        "fastmm_leaf_products_noalloc",
        "fastmm_reconstruct",
        "fastmm_abi_version",
        "fastmm_last_error",
    ):
        assert required in names


def test_library_exports_every_declared_symbol() -> None:
    lib = _native.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.fastmm_abi_version() == _native.ABI_VERSION


def test_compiled_scheme_digests_match_verified_certificates() -> None:
    lib = _native.library()
    for key in SCHEME_KEYS:
        scheme = load_scheme(key)
        size, rank = ctypes.c_int(), ctypes.c_int()
        assert lib.fastmm_scheme_info(scheme.scheme_id, ctypes.byref(size), ctypes.byref(rank)) == 0
        assert (size.value, rank.value) == (scheme.size, scheme.rank)
        assert _native.scheme_sha256(scheme.scheme_id) == scheme.certificate_sha256
    assert lib.fastmm_scheme_info(7, None, None) == 1
    assert b"unknown scheme" in lib.fastmm_last_error()


@pytest.mark.parametrize(
    ("call", "message"),
    (
        (lambda lib: lib.fastmm_left_transform(0, 0, 1, None, None, 4, 4, None), b"null pointer"),
        (lambda lib: lib.fastmm_left_transform(0, 2, 1, 16, 16, 4, 4, None), b"dtype"),
        (lambda lib: lib.fastmm_left_transform(0, 0, 2, 16, 16, 4, 4, None), b"planes must be fp16 or bf16"),
        (lambda lib: lib.fastmm_weight_transform(0, 0, 1, 16, 16, 0, 4, None), b"positive"),
        (lambda lib: lib.fastmm_weight_transform(0, 0, 7, 16, 16, 4, 4, None), b"planes must be fp16 or bf16"),
        (lambda lib: lib.fastmm_right_transform(1, 1, 1, 16, 16, 4, -1, None), b"positive"),
        (lambda lib: lib.fastmm_right_transform(1, 1, 2, 16, 16, 4, 4, None), b"planes must be fp16 or bf16"),
        (lambda lib: lib.fastmm_leaf_products(7, 2, 16, 16, 16, 2, 2, 2, 2, None, 0, None),
         b"operands must be fp16 or bf16"),
        (lambda lib: lib.fastmm_leaf_products(7, 1, 16, 16, 16, 0, 2, 2, 2, None, 0, None), b"products must be fp32 or"),
        (lambda lib: lib.fastmm_leaf_products(7, 0, 16, 16, 16, 1, 2, 2, 2, None, 0, None), b"products must be fp32 or"),
        (lambda lib: lib.fastmm_leaf_products(0, 1, 16, 16, 16, 1, 2, 2, 2, None, 0, None), b"positive"),
        (lambda lib: lib.fastmm_leaf_products(7, 1, 16, 16, 16, 1, 1 << 20, 1 << 12, 2, None, 0, None), b"2^31"),
        (lambda lib: lib.fastmm_leaf_products(7, 1, 16, 16, 16, 1, 2, 2, 2, None, 64, None), b"scratch of 64 bytes"),
        (lambda lib: lib.fastmm_leaf_products(7, 1, 16, 16, 16, 1, 2, 2, 2, 16, -1, None), b"scratch of -1 bytes"),
        (lambda lib: lib.fastmm_leaf_scratch_bytes(7, 1, 1, 2, 2, 2, None), b"null result pointer"),
        (lambda lib: lib.fastmm_leaf_products_noalloc(7, 1, None, 16, 16, 1, 2, 2, 2, None), b"null pointer"),
        (lambda lib: lib.fastmm_leaf_products_noalloc(7, 2, 16, 16, 16, 2, 2, 2, 2, None), b"operands must be"),
        (lambda lib: lib.fastmm_leaf_products_noalloc(7, 1, 16, 16, 16, 0, 2, 2, 2, None), b"products must be fp32 or"),
        (lambda lib: lib.fastmm_leaf_products_noalloc(0, 1, 16, 16, 16, 1, 2, 2, 2, None), b"positive"),
        (lambda lib: lib.fastmm_leaf_products_noalloc(7, 1, 16, 16, 16, 1, 1 << 20, 1 << 12, 2, None), b"2^31"),
        (lambda lib: lib.fastmm_leaf_scratch_bytes(7, 2, 2, 2, 2, 2, ctypes.byref(ctypes.c_int64())),
         b"unsupported element types"),
        (lambda lib: lib.fastmm_leaf_scratch_bytes(7, 1, 1, 0, 2, 2, ctypes.byref(ctypes.c_int64())), b"positive"),
        (lambda lib: lib.fastmm_reconstruct(0, 3, 16, None, 0, 16, 4, 4, None), b"fp16, bf16 or fp32"),
        (lambda lib: lib.fastmm_reconstruct(9, 1, 16, None, 0, 16, 4, 4, None), b"unknown scheme"),
    ),
)
def test_argument_errors_are_reported_before_any_launch(call, message) -> None:
    lib = _native.library()
    assert call(lib) != 0
    assert message in lib.fastmm_last_error()


def test_leaf_scratch_query_without_a_device_reports_no_tail() -> None:
    """No GPU here: the query cannot see compute units and asks for no scratch;
    shapes off the 16x16x32 path never need any."""
    lib = _native.library()
    size = ctypes.c_int64(-1)
    assert lib.fastmm_leaf_scratch_bytes(7, 1, 1, 4107, 6144, 2304, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.fastmm_leaf_scratch_bytes(7, 1, 1, 4107, 6150, 2304, ctypes.byref(size)) == 0
    assert size.value == 0


def test_missing_library_fails_loudly(tmp_path: Path) -> None:
    with pytest.raises(_native.NativeLibraryError, match="not built"):
        _native.library(str(tmp_path / "libfastmm_amd.so"))


def test_torch_extension_registers_the_operator_schemas() -> None:
    """The PyTorch-ROCm extension (csrc/torch_ops.cpp) keeps the reference's operator
    schemas (src/rdna3_fastmm/linear.py:50-167) and one stage operator per entry point."""
    import torch

    from rdna3_fastmm import _torch_ops  # noqa: F401  (loads libfastmm_torch.so)

    for name in ("linear", "linear_rank7", "linear_rank48"):
        schema = str(getattr(torch.ops.rdna3_fastmm, name).default._schema)
        assert schema == f"rdna3_fastmm::{name}(Tensor input, Tensor weight, Tensor? bias=None) -> Tensor"
    stages = {
        "left_transform": "(int scheme, Tensor input, Tensor(a!) output, int rows, int inner) -> ()",
        "weight_transform": "(int scheme, Tensor weight, Tensor(a!) output, int columns, int inner) -> ()",
        "right_transform": "(int scheme, Tensor right, Tensor(a!) output, int inner, int columns) -> ()",
        "reconstruct": "(int scheme, Tensor products, Tensor? bias, Tensor(a!) output, int rows, int columns) -> ()",
    }
    for name, signature in stages.items():
        assert str(getattr(torch.ops.rdna3_fastmm_hip, name).default._schema) == f"rdna3_fastmm_hip::{name}{signature}"
    assert "Tensor(a!) products" in str(torch.ops.rdna3_fastmm_hip.leaf_products.default._schema)


@pytest.mark.parametrize(
    ("shapes", "dtypes", "message"),
    (
        (((4, 3), (5, 3)), ("bfloat16", "float16"), "needs bf16 or fp16 input and weight of one dtype"),
        (((4, 3), (5, 3)), ("float32", "float32"), "needs bf16 or fp16 input and weight of one dtype"),
        (((4, 3), (5, 3)), ("bfloat16", "bfloat16"), "needs input and weight on one ROCm device"),
    ),
)
def test_torch_operators_reject_bad_operands_before_any_launch(shapes, dtypes, message) -> None:
    import torch

    from rdna3_fastmm import _torch_ops

    x = torch.zeros(shapes[0], dtype=getattr(torch, dtypes[0]))
    w = torch.zeros(shapes[1], dtype=getattr(torch, dtypes[1]))
    for op in (_torch_ops.linear, _torch_ops.linear_rank7, _torch_ops.linear_rank48):
        with pytest.raises(ValueError, match=message):
            op(x, w)


def test_stage_operators_reject_host_tensors_before_any_launch() -> None:
    """Every stage operator checks its tensors before the C ABI sees a pointer:
    host tensors are refused with a ValueError (no launch, no library status)."""
    import torch

    from rdna3_fastmm import _torch_ops

    stages = _torch_ops.stages
    scheme = load_scheme("rank7").scheme_id
    x = torch.zeros((4, 4), dtype=torch.float16)
    planes = torch.zeros((7, 2, 2), dtype=torch.float16)
    calls = (
        lambda: stages.left_transform(scheme, x, planes, 4, 4),
        lambda: stages.weight_transform(scheme, x, planes, 4, 4),
        lambda: stages.right_transform(scheme, x, planes, 4, 4),
        lambda: stages.leaf_products(7, planes, planes, planes.clone(), 2, 2, 2, None),
        lambda: stages.reconstruct(scheme, planes, None, x, 4, 4),
    )
    for call in calls:
        with pytest.raises(ValueError, match="must be on a ROCm device"):
            call()
