"""Dynamo backend ``rdna3-fastmm``: FX Linear rewrite, then standard Inductor.

reference ``src/rdna3_fastmm/inductor.py:18-49``. When inference mode is on,
the PyTorch build is ROCm and the current GPU is the tested MI355X, eligible
``F.linear`` nodes become ``rdna3_fastmm`` operators before
``torch._inductor.compile``; CUDA graphs are turned off for such graphs, as in
the reference. Otherwise the graph goes to Inductor untouched. The
reference's private ``external_matmul`` FP16 ``mm`` hook is not part of this
backend.
"""

from __future__ import annotations

from typing import Any, Protocol, Sequence

import torch
import torch._inductor
from torch.fx import GraphModule

from .linear import rewrite_eligible_linears
from .runtime import is_tested_runtime


class CompiledGraph(Protocol):
    def __call__(self, *inputs: torch.Tensor) -> tuple[torch.Tensor, ...]: ...


def _enable_rewrite() -> bool:
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
    if _enable_rewrite():
        if rewrite_eligible_linears(graph_module, list(example_inputs)):
            inductor_options["triton.cudagraphs"] = False
    return torch._inductor.compile(graph_module, list(example_inputs), options=inductor_options)
