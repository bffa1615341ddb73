"""The FX Linear rewrite and the Dynamo backend, on the CPU with fake CUDA tensors.

Mirrors reference tests/test_inductor.py:34-203: eligible BF16 Linears are
replaced by the rdna3_fastmm operators only for measured-win families and
within the memory budget; everything else is left alone; the backend hands
the graph to Inductor with CUDA graphs off only when it rewrote something.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from rdna3_fastmm import external_mm, inductor, linear
from rdna3_fastmm.linear import (
    RDNA3_LINEAR_OP,
    RDNA3_RANK7_LINEAR_OP,
    RDNA3_RANK48_LINEAR_OP,
    _linear_node_target,
    rewrite_eligible_linears,
)
from rdna3_fastmm.runtime import LinearShapeFamily, Rank7Plan, Rank48Plan, Rank49Plan


class Linear(torch.nn.Module):
    def forward(self, input_tensor, weight):
        return torch.nn.functional.linear(input_tensor, weight)


class BiasLinear(torch.nn.Module):
    def forward(self, input_tensor, weight, bias):
        return torch.nn.functional.linear(input_tensor, weight, bias)


def fake(*shapes, dtype=torch.bfloat16, device="cuda"):
    mode = FakeTensorMode(allow_non_fake_inputs=True)
    with mode:
        return [torch.empty(shape, dtype=dtype, device=device) for shape in shapes], mode


def traced(module, *tensors):
    graph_module = torch.fx.symbolic_trace(module)
    placeholders = [n for n in graph_module.graph.nodes if n.op == "placeholder"]
    for node, tensor in zip(placeholders, tensors):
        node.meta["val"] = tensor
    return graph_module


def targets(graph_module):
    return {node.target for node in graph_module.graph.nodes if node.op == "call_function"}


@pytest.fixture
def measured(monkeypatch):
    monkeypatch.setattr(Rank7Plan, "linear_shape_families", (LinearShapeFamily(3_328, 9_216, 4_608, 12_288, False),))
    monkeypatch.setattr(Rank49Plan, "linear_shape_families", (LinearShapeFamily(19_968, 19_968, 4_096, 16_384, True),))
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))


def test_rewrite_replaces_eligible_bfloat16_linear(measured) -> None:
    (x, w), _ = fake((5120, 4608), (12288, 4608))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    assert RDNA3_RANK7_LINEAR_OP in targets(gm)


def test_rewrite_keeps_rank49_for_exact_family(measured) -> None:
    (x, w, b), _ = fake((19_968, 4_096), (16_384, 4_096), (16_384,))
    gm = traced(BiasLinear(), x, w, b)
    assert rewrite_eligible_linears(gm, [x, w, b]) == 1
    assert RDNA3_LINEAR_OP in targets(gm)


def test_rewrite_flattens_leading_dimensions(measured) -> None:
    (x, w), _ = fake((2, 2560, 4608), (12288, 4608))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 1


@pytest.mark.parametrize(
    "shapes, dtype, device",
    (
        (((3072, 4608), (12288, 4608)), torch.bfloat16, "cuda"),  # rows outside the family
        (((5120, 4608), (12288, 4608)), torch.float16, "cuda"),  # not BF16
        (((5120, 4608), (12288, 4608)), torch.bfloat16, "cpu"),  # not on the GPU
        (((5120, 0), (12288, 0)), torch.bfloat16, "cuda"),  # empty inner dimension
        (((0, 4608), (12288, 4608)), torch.bfloat16, "cuda"),  # no rows
    ),
)
def test_rewrite_preserves_ineligible_linear(measured, shapes, dtype, device) -> None:
    (x, w), _ = fake(*shapes, dtype=dtype, device=device)
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 0


def test_rewrite_preserves_linear_without_memory_budget(measured, monkeypatch) -> None:
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (1 << 20, 288 << 30))
    (x, w), _ = fake((5120, 4608), (12288, 4608))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 0


def test_memory_budget_counts_the_split_k_scratch(measured, monkeypatch) -> None:
    """Planes, products and output (the reference's sum) plus the leaf GEMM's split-K
    scratch at its 48 MiB maximum must fit in half the free memory."""
    rows, inner, columns = 5120, 4608, 12288
    mb, kb, nb = rows // 2, inner // 2, columns // 2
    temporaries = 7 * (mb * kb + kb * nb + mb * nb) * 2 + rows * columns * 2
    for free, expected in ((2 * temporaries, 0), (2 * (temporaries + (48 << 20)), 1)):
        monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None, free=free: (free, 288 << 30))
        (x, w), _ = fake((rows, inner), (columns, inner))
        gm = traced(Linear(), x, w)
        assert rewrite_eligible_linears(gm, [x, w]) == expected, free


def test_rewrite_rejects_non_contiguous_weight(measured) -> None:
    (x, w), mode = fake((5120, 4608), (4608, 12288))
    with mode:
        wt = w.t()
    gm = traced(Linear(), x, wt)
    assert _linear_node_target(next(n for n in gm.graph.nodes if n.op == "call_function")) is None


def test_shipped_tables_leave_graphs_untouched(monkeypatch) -> None:
    """An MLP up projection has no measured MI355X win: the rewrite must not fire."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))
    (x, w), _ = fake((5120, 4608), (12288, 4608))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 0


def test_shipped_tables_rewrite_a_measured_down_projection(monkeypatch) -> None:
    """The corpus's 4704-token Ideogram MLP down projection is a measured rank-7 win."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))
    (x, w), _ = fake((4704, 12288), (4608, 12288))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    assert RDNA3_RANK7_LINEAR_OP in targets(gm)


def test_shipped_tables_rewrite_a_rank48_only_family(monkeypatch) -> None:
    """Llama-3-70B's 28672 -> 8192 down projection at 13952 rows: only a rank-48
    dynamic family covers it in the shipped MI355X table."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))
    shape = (13_952, 28_672, 8_192)
    assert Rank48Plan.has_measured_linear_win(shape, has_bias=False)
    assert not Rank7Plan.has_measured_linear_win(shape, has_bias=False)
    (x, w), _ = fake(shape[:2], (shape[2], shape[1]))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    assert RDNA3_RANK48_LINEAR_OP in targets(gm)


def test_shipped_tables_prefer_the_faster_family(monkeypatch) -> None:
    """12288 -> 4096 at 6272 rows is covered by a rank-7 and a rank-48 dynamic
    family; the rank-48 one was measured faster there, so the rewrite picks it."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))
    shape = (6_272, 12_288, 4_096)
    r7 = Rank7Plan.measured_linear_speedup(shape, has_bias=False)
    r48 = Rank48Plan.measured_linear_speedup(shape, has_bias=False)
    assert r7 is not None and r48 is not None and r48 > r7
    (x, w), _ = fake(shape[:2], (shape[2], shape[1]))
    gm = traced(Linear(), x, w)
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    assert RDNA3_RANK48_LINEAR_OP in targets(gm)


def test_rewrite_ranks_plans_by_measured_speedup(monkeypatch) -> None:
    """Overlapping families: the faster one wins; equal speedups keep rank 7 first;
    the chosen plan's memory budget still applies."""
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (200 << 30, 288 << 30))
    (x, w), _ = fake((5120, 4608), (12288, 4608))
    for r7, r48, expected in ((1.10, 1.30, RDNA3_RANK48_LINEAR_OP), (1.30, 1.10, RDNA3_RANK7_LINEAR_OP),
                              (1.20, 1.20, RDNA3_RANK7_LINEAR_OP)):
        monkeypatch.setattr(Rank7Plan, "linear_shape_families",
                            (LinearShapeFamily(4_096, 6_144, 4_608, 12_288, False, r7),))
        monkeypatch.setattr(Rank48Plan, "linear_shape_families",
                            (LinearShapeFamily(5_000, 5_200, 4_608, 12_288, False, r48),))
        gm = traced(Linear(), x, w)
        assert rewrite_eligible_linears(gm, [x, w]) == 1
        assert expected in targets(gm)
    # the speedup takes no part in a family's identity
    assert LinearShapeFamily(1, 2, 3, 4, False, 1.5) == LinearShapeFamily(1, 2, 3, 4, False)


def test_operators_are_registered_with_fake_kernels() -> None:
    for name in ("linear", "linear_rank7", "linear_rank48"):
        assert hasattr(torch.ops.rdna3_fastmm, name)
    (x, w, b), mode = fake((2, 3, 19), (23, 19), (23,))
    with mode:
        out = torch.ops.rdna3_fastmm.linear_rank7(x, w, b)
    assert tuple(out.shape) == (2, 3, 23) and out.dtype == torch.bfloat16


def test_backend_adds_external_choice_and_disables_cudagraphs(monkeypatch) -> None:
    """reference tests/test_inductor.py:34-67."""
    captured = {}
    marker = object()

    def fake_compile(graph, example_inputs, options):
        captured["options"] = options
        return object()

    gm = torch.fx.symbolic_trace(lambda value: value.sin())
    monkeypatch.setattr(torch._inductor, "compile", fake_compile)
    monkeypatch.setattr(inductor, "_enable_external_matmul", lambda: True)
    monkeypatch.setattr(inductor, "rewrite_eligible_linears", lambda graph, inputs: 0)
    inductor.compile_backend(gm, [torch.randn(4)], mode="reduce-overhead", options={"external_matmul": [marker]})
    options = captured["options"]
    assert options["external_matmul"] == [marker, external_mm.rdna3_rank49_dynamic_v1_out]
    assert options["max_autotune_gemm"] is True and options["triton.cudagraphs"] is False
    # the choice is added once
    inductor.compile_backend(gm, [torch.randn(4)], options={"external_matmul": options["external_matmul"]})
    assert captured["options"]["external_matmul"] == [marker, external_mm.rdna3_rank49_dynamic_v1_out]


def test_external_mm_falls_back_for_ineligible_input() -> None:
    """reference tests/test_inductor.py:21-31: CPU input, and a shape outside dynamic_shapes."""
    left = torch.randn((7, 11), dtype=torch.float16)
    right = torch.randn((11, 5), dtype=torch.float16)
    out = torch.empty((7, 5), dtype=torch.float16)
    with torch.inference_mode():
        assert not external_mm.is_rank49_dynamic_eligible(left, right, out)
        external_mm.rdna3_rank49_dynamic_v1_out(left, right, out=out)
    torch.testing.assert_close(out, left @ right, rtol=0, atol=0)


@pytest.mark.parametrize(
    "case",
    ("grad", "dtype", "shape", "out_shape", "device", "noncontiguous", "unmeasured"),
)
def test_external_mm_eligibility(monkeypatch, case) -> None:
    monkeypatch.setattr(Rank49Plan, "dynamic_shapes", frozenset({(64, 32, 48)}))
    monkeypatch.setattr(external_mm, "is_tested_runtime", lambda device: True)
    (left, right, out), mode = fake((64, 32), (32, 48), (64, 48), dtype=torch.float16)
    with torch.inference_mode():
        assert external_mm.is_rank49_dynamic_eligible(left, right, out)
    with mode:
        if case == "dtype":
            left = left.to(torch.bfloat16)
        elif case == "shape":
            right = torch.empty((33, 48), dtype=torch.float16, device="cuda")
        elif case == "out_shape":
            out = torch.empty((64, 47), dtype=torch.float16, device="cuda")
        elif case == "device":
            out = torch.empty((64, 48), dtype=torch.float16)
        elif case == "noncontiguous":
            right = torch.empty((48, 32), dtype=torch.float16, device="cuda").t()
        elif case == "unmeasured":
            left = torch.empty((65, 32), dtype=torch.float16, device="cuda")
            out = torch.empty((65, 48), dtype=torch.float16, device="cuda")
    if case == "grad":
        assert not external_mm.is_rank49_dynamic_eligible(left, right, out)
        return
    with torch.inference_mode():
        assert not external_mm.is_rank49_dynamic_eligible(left, right, out)


def test_backend_preserves_standard_inductor_when_runtime_is_unsupported(monkeypatch) -> None:
    captured = {}
    monkeypatch.setattr(torch._inductor, "compile", lambda g, i, options: captured.update(options=options))
    monkeypatch.setattr(inductor, "_enable_external_matmul", lambda: False)
    inductor.compile_backend(torch.fx.symbolic_trace(lambda v: v.cos()), [torch.randn(4)], mode="reduce-overhead")
    assert captured["options"] == {"triton.cudagraphs": True}


def test_pyproject_registers_named_dynamo_backend() -> None:
    from pathlib import Path

    import tomli

    pyproject = tomli.loads((Path(__file__).resolve().parent.parent / "pyproject.toml").read_text())
    assert pyproject["project"]["entry-points"]["torch_dynamo_backends"] == {
        "rdna3-fastmm": "rdna3_fastmm.inductor:compile_backend"
    }


def test_linear_ops_reject_bad_operands() -> None:
    with pytest.raises(ValueError, match="bf16 or fp16"):
        linear._check_operands("op", torch.empty(2, 3), torch.empty(4, 3), None)
