"""Dynamo backend ``rdna3-fastmm``: FX Linear rewrite and an FP16 ``mm``
autotuning choice, then standard Inductor.

reference ``src/rdna3_fastmm/inductor.py:18-49``. When inference mode is on,
the PyTorch build is ROCm and the current GPU is the tested MI355X: eligible
``F.linear`` nodes become ``rdna3_fastmm`` operators (measured-win shape
families only), ``rdna3_rank49_dynamic_v1_out`` joins Inductor's
``external_matmul`` candidates with ``max_autotune_gemm`` on, and CUDA graphs
are turned off, as in the reference. Otherwise the graph goes to Inductor with
the caller's options untouched.
"""

from __future__ import annotations

from typing import Any, Protocol, Sequence

import torch
import torch._inductor
import torch._inductor.config
from torch.fx import GraphModule

from .external_mm import rdna3_rank49_dynamic_v1_out
from .linear import rewrite_eligible_linears
from .runtime import is_tested_runtime


class CompiledGraph(Protocol):
    def __call__(self, *inputs: torch.Tensor) -> tuple[torch.Tensor, ...]: ...


def _enable_external_matmul() -> bool:
    if torch.is_grad_enabled() or torch.version.hip is None or not torch.cuda.is_available():
        return False
    return is_tested_runtime(torch.device("cuda", torch.cuda.current_device()))


def compile_backend(
    graph_module: GraphModule,
    example_inputs: Sequence[torch.Tensor],
    *,
    mode: str | None = None,
    options: dict[str, Any] | None = None,
) -> CompiledGraph:
    inductor_options = torch._inductor.list_mode_options(mode)
    inductor_options.update(options or {})
    if _enable_external_matmul():
        rewrite_eligible_linears(graph_module, list(example_inputs))
        choices = list(inductor_options.get("external_matmul", torch._inductor.config.external_matmul))
        if rdna3_rank49_dynamic_v1_out not in choices:
            choices.append(rdna3_rank49_dynamic_v1_out)
        inductor_options["external_matmul"] = choices
        inductor_options["max_autotune_gemm"] = True
        inductor_options["triton.cudagraphs"] = False
    return torch._inductor.compile(graph_module, list(example_inputs), options=inductor_options)
