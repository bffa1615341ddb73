"""FP16 ``mm`` choice for Inductor's ``external_matmul`` autotuning hook.

reference ``src/rdna3_fastmm/external_mm.py:6-48``. Inductor benchmarks every
callable in ``torch._inductor.config.external_matmul`` as one more candidate
for each ``mm`` it lowers (with ``max_autotune_gemm``) and keeps the fastest.
This candidate runs the rank-49 plan's dynamic ``mm`` path when the call is
eligible -- inference, 2-D contiguous FP16 operands and output on the tested
MI355X runtime, and a shape in ``Rank49Plan.dynamic_shapes`` (measured FP16
``mm`` wins) -- and otherwise ``torch.mm`` into ``out``, so it can never make
a graph wrong, only slower in the autotuner's eyes. A workspace that does not
fit in free device memory also falls back to ``torch.mm``.
"""

from __future__ import annotations

import torch

from .runtime import Rank49Plan, is_tested_runtime


def is_rank49_dynamic_eligible(left: torch.Tensor, right: torch.Tensor, out: torch.Tensor) -> bool:
    if torch.is_grad_enabled():
        return False
    if left.ndim != 2 or right.ndim != 2 or out.ndim != 2:
        return False
    rows, inner = left.shape
    right_inner, columns = right.shape
    if inner != right_inner or tuple(out.shape) != (rows, columns):
        return False
    if (rows, inner, columns) not in Rank49Plan.dynamic_shapes:
        return False
    if not (left.dtype == right.dtype == out.dtype == torch.float16):
        return False
    if not (left.device == right.device == out.device) or left.device.type != "cuda":
        return False
    if not (left.is_contiguous() and right.is_contiguous() and out.is_contiguous()):
        return False
    if left.requires_grad or right.requires_grad or out.requires_grad:
        return False
    return is_tested_runtime(left.device)


def rdna3_rank49_dynamic_v1_out(left: torch.Tensor, right: torch.Tensor, *, out: torch.Tensor) -> None:
    if not is_rank49_dynamic_eligible(left, right, out):
        torch.mm(left, right, out=out)
        return
    rows, inner = left.shape
    plan = Rank49Plan(rows, inner, right.shape[1], left.device, left.dtype)
    free_bytes, _ = torch.cuda.mem_get_info(left.device)
    if plan.workspace_bytes > free_bytes:
        torch.mm(left, right, out=out)
        return
    plan.run(left, right, plan.allocate_workspace(max_free_memory_fraction=1.0), out)
