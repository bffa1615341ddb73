"""Load ``libfastmm_torch.so``, the PyTorch-ROCm operator library over the C ABI.

It registers ``torch.ops.rdna3_fastmm.{linear, linear_rank7, linear_rank48}``
(the allocating F.linear operators) and ``torch.ops.rdna3_fastmm_hip.*`` (one
operator per C-ABI stage entry point, used by the plans). Loading it also loads
``libfastmm_amd.so``, and the kernels of the schemes the operators run are
checked against the certificates this package verified, once (the reference
checks its generated modules at import, runtime.py:16-53). If the library is
missing, importing this module raises: there is no fallback path.
"""

from __future__ import annotations

import torch

from . import _native
from ._build import TORCH_OPS_PATH
from .schemes import load_scheme

LINEAR_SCHEMES = ("rank7", "rank48", "rank49")  # the schemes the allocating operators run


def _load() -> None:
    if not TORCH_OPS_PATH.exists():
        raise _native.NativeLibraryError(
            f"{TORCH_OPS_PATH} is not built; run `python -m rdna3_fastmm._build` (or __graft_entry__.build()) first"
        )
    _native.library()  # ABI version check of the kernels' library
    for key in LINEAR_SCHEMES:
        scheme = load_scheme(key)
        if _native.scheme_sha256(scheme.scheme_id) != scheme.certificate_sha256:
            raise RuntimeError("compiled kernel metadata does not match the backend")
    torch.ops.load_library(str(TORCH_OPS_PATH))


_load()

linear = torch.ops.rdna3_fastmm.linear.default
linear_rank7 = torch.ops.rdna3_fastmm.linear_rank7.default
linear_rank48 = torch.ops.rdna3_fastmm.linear_rank48.default
stages = torch.ops.rdna3_fastmm_hip
