"""ctypes binding of ``libfastmm_amd.so`` (the C ABI in include/fastmm_amd.h).

The library is loaded on first use. If it is missing or does not export the
ABI this package was written against, every entry point raises
``RuntimeError``: there is no fallback path, on a GPU box or anywhere else.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

import torch

from ._build import LIBRARY_PATH

ABI_VERSION = 5

BF16, FP16, FP32 = 0, 1, 2
_DTYPE_CODES = {torch.bfloat16: BF16, torch.float16: FP16, torch.float32: FP32}

_I64 = ctypes.c_int64
_PTR = ctypes.c_void_p
_INT = ctypes.c_int

# name -> argument types (every entry point returns int status).
SIGNATURES: dict[str, list] = {
    "fastmm_left_transform": [_INT, _INT, _INT, _PTR, _PTR, _I64, _I64, _PTR],
    "fastmm_weight_transform": [_INT, _INT, _INT, _PTR, _PTR, _I64, _I64, _PTR],
    "fastmm_right_transform": [_INT, _INT, _INT, _PTR, _PTR, _I64, _I64, _PTR],
    "fastmm_leaf_products": [_INT, _INT, _PTR, _PTR, _PTR, _INT, _I64, _I64, _I64, _PTR, _I64, _PTR],
    "fastmm_leaf_products_noalloc": [_INT, _INT, _PTR, _PTR, _PTR, _INT, _I64, _I64, _I64, _PTR],
    "fastmm_leaf_scratch_bytes": [_INT, _INT, _INT, _I64, _I64, _I64, ctypes.POINTER(_I64)],
    "fastmm_reconstruct": [_INT, _INT, _PTR, _PTR, _INT, _PTR, _I64, _I64, _PTR],
    "fastmm_scheme_info": [_INT, ctypes.POINTER(_INT), ctypes.POINTER(_INT)],
}


class NativeLibraryError(RuntimeError):
    pass


@lru_cache(maxsize=None)
def library(path: str | None = None) -> ctypes.CDLL:
    location = Path(path) if path else LIBRARY_PATH
    if not location.exists():
        raise NativeLibraryError(
            f"{location} is not built; run `python -m rdna3_fastmm._build` "
            "(or __graft_entry__.build()) first"
        )
    lib = ctypes.CDLL(str(location))
    lib.fastmm_abi_version.restype = _INT
    lib.fastmm_abi_version.argtypes = []
    if lib.fastmm_abi_version() != ABI_VERSION:
        raise NativeLibraryError(f"{location} has ABI {lib.fastmm_abi_version()}, expected {ABI_VERSION}")
    lib.fastmm_last_error.restype = ctypes.c_char_p
    lib.fastmm_last_error.argtypes = []
    lib.fastmm_scheme_sha256.restype = ctypes.c_char_p
    lib.fastmm_scheme_sha256.argtypes = [_INT]
    for name, argtypes in SIGNATURES.items():
        function = getattr(lib, name)
        function.restype = _INT
        function.argtypes = argtypes
    return lib


def call(name: str, *args: object) -> None:
    lib = library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.fastmm_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({status}): {message}")


def dtype_code(dtype: torch.dtype) -> int:
    return _DTYPE_CODES[dtype]


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def scheme_sha256(scheme_id: int) -> str:
    raw = library().fastmm_scheme_sha256(scheme_id)
    if raw is None:
        raise NativeLibraryError(f"library does not know scheme {scheme_id}")
    return raw.decode()
