"""Allocating ``F.linear`` operators and the pre-AOT FX rewrite.

``torch.ops.rdna3_fastmm.linear`` (rank 49) and
``torch.ops.rdna3_fastmm.linear_rank7`` keep the reference's schemas
(``src/rdna3_fastmm/linear.py:50-167``): functional, ``(Tensor input, Tensor
weight, Tensor? bias=None) -> Tensor``, any number of leading dimensions.
The reference builds them as ``triton_op``s so Inductor sees the Triton
kernels; here they are C++ operators of the PyTorch-ROCm extension
``libfastmm_torch.so`` (``csrc/torch_ops.cpp``), which runs the whole call
(planes, products, early release of the planes, output, recombination) as
launches of the HIP library, with a fake (meta) implementation registered here
so Dynamo/Inductor treat them as opaque extern kernels.
``torch.ops.rdna3_fastmm.linear_rank48`` is the rank-48 counterpart.

``rewrite_eligible_linears`` replaces eligible ``aten.linear`` nodes of a
graph before AOT compilation, exactly where the reference does
(linear.py:170-288): BF16 input/weight/bias on one GPU, contiguous, static
shape, a measured-win family, and at most half of the free device memory
for the temporaries (here also the split-K scratch). The reference tries
rank-7 families first, then rank-49 (linear.py:240-252); here every scheme
with measured MI355X families is a candidate (rank 7, rank 48, rank 49) and
the one whose covering family was measured fastest is used, earlier schemes
winning ties.
"""

from typing import Callable, Optional

import torch
from torch.fx import GraphModule, Node
from torch.fx.passes.fake_tensor_prop import FakeTensorProp

from . import _torch_ops
from .runtime import Rank7Plan, Rank48Plan, Rank49Plan, _LinearPlan

LINEAR_TARGETS = frozenset({torch._C._nn.linear, torch.ops.aten.linear.default})
MAX_LINEAR_ALLOCATION_FREE_FRACTION = 0.5
# The most split-K scratch one call allocates: 192 fp32 256 x 256 tile parts, the
# tail planner's maximum on a 256-CU MI355X (FASTMM_STATIC_SCRATCH_BYTES).
MAX_LEAF_SCRATCH_BYTES = 48 << 20


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def _check_operands(name: str, input_tensor: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> None:
    """The operators' argument checks (the C++ operators raise the same ValueErrors)."""
    if input_tensor.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != input_tensor.dtype:
        raise ValueError(f"{name} needs bf16 or fp16 input and weight of one dtype")
    if input_tensor.device.type != "cuda" or weight.device != input_tensor.device:
        raise ValueError(f"{name} needs input and weight on one ROCm device")
    if weight.dim() != 2 or input_tensor.dim() < 1 or input_tensor.shape[-1] != weight.shape[1]:
        raise ValueError(f"{name}: input [..., K] and weight [N, K] do not match")
    if not input_tensor.is_contiguous() or not weight.is_contiguous():
        raise ValueError(f"{name} needs contiguous input and weight")
    if bias is not None and (
        tuple(bias.shape) != (weight.shape[0],)
        or bias.dtype != input_tensor.dtype
        or bias.device != input_tensor.device
        or not bias.is_contiguous()
    ):
        raise ValueError(f"{name}: bias must be a contiguous [N] tensor of the input dtype")


def _fake_linear(input_tensor: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    return input_tensor.new_empty((*input_tensor.shape[:-1], weight.shape[0]))


for _name in ("rdna3_fastmm::linear", "rdna3_fastmm::linear_rank7", "rdna3_fastmm::linear_rank48"):
    torch.library.register_fake(_name)(_fake_linear)

RDNA3_LINEAR_OP = _torch_ops.linear
RDNA3_RANK7_LINEAR_OP = _torch_ops.linear_rank7
RDNA3_RANK48_LINEAR_OP = _torch_ops.linear_rank48


def rdna3_linear(input_tensor: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``torch.ops.rdna3_fastmm.linear``: F.linear through the rank-49 scheme."""
    return RDNA3_LINEAR_OP(input_tensor, weight, bias)


def rdna3_rank7_linear(
    input_tensor: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """``torch.ops.rdna3_fastmm.linear_rank7``: F.linear through the rank-7 scheme."""
    return RDNA3_RANK7_LINEAR_OP(input_tensor, weight, bias)


def rdna3_rank48_linear(
    input_tensor: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """``torch.ops.rdna3_fastmm.linear_rank48``: F.linear through the rank-48 scheme."""
    return RDNA3_RANK48_LINEAR_OP(input_tensor, weight, bias)


def _node_tensor(node: Node) -> Optional[torch.Tensor]:
    value = node.meta.get("val", node.meta.get("example_value"))
    return value if isinstance(value, torch.Tensor) else None


def _has_linear_memory_budget(plan_type: type, shape: tuple, device: torch.device) -> bool:
    """Temporaries of one dynamic call fit in half the free memory (linear.py:175-194):
    the reference's planes, products and output, plus this backend's split-K scratch
    (counted at its maximum; the operator may allocate less)."""
    rows, inner, columns = shape
    s, rank = plan_type.scheme_size, plan_type.rank
    mb, kb, nb = _ceil_div(rows, s), _ceil_div(inner, s), _ceil_div(columns, s)
    allocation = rank * (mb * kb + kb * nb + mb * nb) * 2 + rows * columns * 2 + MAX_LEAF_SCRATCH_BYTES
    free_bytes, _ = torch.cuda.mem_get_info(device)
    return allocation <= free_bytes * MAX_LINEAR_ALLOCATION_FREE_FRACTION


# Candidate plans of the rewrite, in tie-break order: the plan whose covering
# dynamic family was measured fastest is used (if its temporaries fit).
_REWRITE_ORDER: tuple = (
    (Rank7Plan, RDNA3_RANK7_LINEAR_OP),
    (Rank48Plan, RDNA3_RANK48_LINEAR_OP),
    (Rank49Plan, RDNA3_LINEAR_OP),
)


def _rewrite_choice(shape: tuple, has_bias: bool, device: torch.device) -> Optional[Callable]:
    """The operator for the fastest measured dynamic family covering ``shape``, or None."""
    ranked = []
    for order, (plan_type, target) in enumerate(_REWRITE_ORDER):
        plan: type[_LinearPlan] = plan_type
        speedup = plan.measured_linear_speedup(shape, has_bias=has_bias)
        if speedup is not None:
            ranked.append((-speedup, order, plan, target))
    if not ranked:
        return None
    _, _, plan, target = min(ranked, key=lambda item: item[:2])
    return target if _has_linear_memory_budget(plan, shape, device) else None


def _linear_node_target(node: Node) -> Optional[Callable]:
    if node.op != "call_function" or node.target not in LINEAR_TARGETS:
        return None
    if node.kwargs or len(node.args) not in (2, 3):
        return None
    input_node, weight_node = node.args[:2]
    bias_node = node.args[2] if len(node.args) == 3 else None
    if not isinstance(input_node, Node) or not isinstance(weight_node, Node):
        return None
    input_tensor, weight = _node_tensor(input_node), _node_tensor(weight_node)
    if input_tensor is None or weight is None or input_tensor.ndim < 2 or weight.ndim != 2:
        return None
    if input_tensor.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        return None
    if input_tensor.device.type != "cuda" or weight.device != input_tensor.device:
        return None
    if not input_tensor.is_contiguous() or not weight.is_contiguous():
        return None
    inner = input_tensor.shape[-1]
    columns, weight_inner = weight.shape
    if inner != weight_inner:
        return None
    if not all(isinstance(d, int) and d > 0 for d in (*input_tensor.shape[:-1], inner, columns)):
        return None  # symbolic or empty: left to aten
    has_bias = bias_node is not None
    if isinstance(bias_node, Node):
        bias = _node_tensor(bias_node)
        if (
            bias is None
            or tuple(bias.shape) != (columns,)
            or bias.dtype != torch.bfloat16
            or bias.device != input_tensor.device
            or not bias.is_contiguous()
        ):
            return None
    elif bias_node is not None:
        return None
    shape = (input_tensor.numel() // inner, inner, columns)
    return _rewrite_choice(shape, has_bias, input_tensor.device)


def rewrite_eligible_linears(graph_module: GraphModule, example_inputs: list) -> int:
    """Replace eligible Linear nodes in place; returns how many were replaced."""
    linear_nodes = tuple(
        node for node in graph_module.graph.nodes if node.op == "call_function" and node.target in LINEAR_TARGETS
    )
    if any(
        isinstance(argument, Node) and _node_tensor(argument) is None
        for node in linear_nodes
        for argument in node.args
    ):
        FakeTensorProp(graph_module).propagate(*example_inputs)
    rewritten = 0
    for node in linear_nodes:
        target = _linear_node_target(node)
        if target is None:
            continue
        input_node, weight_node = node.args[:2]
        bias_node = node.args[2] if len(node.args) == 3 else None
        with graph_module.graph.inserting_before(node):
            replacement = graph_module.graph.call_function(target, args=(input_node, weight_node, bias_node))
        replacement.meta = node.meta.copy()
        node.replace_all_uses_with(replacement)
        graph_module.graph.erase_node(node)
        rewritten += 1
    if rewritten:
        graph_module.graph.lint()
        graph_module.recompile()
    return rewritten
