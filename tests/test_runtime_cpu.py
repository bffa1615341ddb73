"""Plan logic that needs no GPU: shape partition, byte formulas, gates, validation.

Mirrors the reference's CPU-safe tests (tests/test_rdna3.py:32-403), with the
runtime gate retargeted to one MI355X and the device faked by monkeypatch.
"""

from types import SimpleNamespace

import pytest
import torch

from rdna3_fastmm import runtime
from rdna3_fastmm.runtime import (
    LinearShapeFamily,
    MatrixShape,
    Rank7Plan,
    Rank48Plan,
    Rank49Plan,
    unsupported_runtime_reason,
)


def configure_supported_runtime(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(torch.version, "hip", "7.0.51831")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(
        torch.cuda,
        "get_device_properties",
        lambda device: SimpleNamespace(gcnArchName="gfx950:sramecc+:xnack-", multi_processor_count=256),
    )
    monkeypatch.setattr(torch, "__version__", "2.10.0+rocm7.0")


def test_runtime_accepts_tested_stack(monkeypatch) -> None:
    configure_supported_runtime(monkeypatch)
    assert unsupported_runtime_reason() is None


def test_runtime_requires_rocm_build(monkeypatch) -> None:
    monkeypatch.setattr(torch.version, "hip", None)
    assert unsupported_runtime_reason() == "requires a ROCm PyTorch build"


def test_runtime_requires_available_gpu(monkeypatch) -> None:
    configure_supported_runtime(monkeypatch)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert unsupported_runtime_reason() == "requires an available ROCm GPU"


def test_runtime_rejects_cpu_device(monkeypatch) -> None:
    configure_supported_runtime(monkeypatch)
    assert unsupported_runtime_reason(torch.device("cpu")) == "requires a ROCm GPU device"


def test_runtime_describes_wrong_gpu(monkeypatch) -> None:
    configure_supported_runtime(monkeypatch)
    monkeypatch.setattr(
        torch.cuda, "get_device_properties", lambda d: SimpleNamespace(gcnArchName="gfx942", multi_processor_count=304)
    )
    assert unsupported_runtime_reason() == "tested only on gfx950 with 256 compute units; found gfx942 with 304"


@pytest.mark.parametrize(
    ("component", "version", "expected"),
    (
        ("torch", "2.9.1+rocm6.4", "tested only with PyTorch 2.10.0; found 2.9.1+rocm6.4"),
        ("hip", "6.4.1", "tested only with ROCm 7.0; found 6.4.1"),
    ),
)
def test_runtime_describes_version_mismatch(monkeypatch, component, version, expected) -> None:
    configure_supported_runtime(monkeypatch)
    if component == "torch":
        monkeypatch.setattr(torch, "__version__", version)
    else:
        monkeypatch.setattr(torch.version, "hip", version)
    assert unsupported_runtime_reason() == expected


def test_shape_uses_padded_quarters() -> None:
    shape = MatrixShape.from_dimensions(257, 263, 269, 4)
    assert shape.dimensions == (257, 263, 269)
    assert (shape.block_rows, shape.block_inner, shape.block_columns) == (65, 66, 68)
    assert shape.workspace_elements(49) == 49 * (65 * 66 + 66 * 68 + 65 * 68)


def test_shape_rejects_nonpositive_dimensions() -> None:
    with pytest.raises(ValueError, match="positive"):
        MatrixShape.from_dimensions(4, 0, 4, 4)


@pytest.mark.parametrize("plan_type", (Rank7Plan, Rank48Plan, Rank49Plan))
def test_plans_reject_cpu_device(plan_type) -> None:
    with pytest.raises(ValueError, match="ROCm"):
        plan_type(4, 4, 4, torch.device("cpu"))


def test_plan_class_metadata_matches_certificates() -> None:
    from rdna3_fastmm.schemes import load_scheme

    for plan_type in (Rank7Plan, Rank48Plan, Rank49Plan):
        scheme = load_scheme(plan_type.scheme_key)
        assert (plan_type.rank, plan_type.scheme_size) == (scheme.rank, scheme.size)
        assert plan_type.algorithm == scheme.algorithm


def test_byte_formulas_and_precision_pairs(monkeypatch) -> None:
    """reference test_rdna3.py:428-430, 520-522 (no allocation needed)."""
    configure_supported_runtime(monkeypatch)
    plan = Rank48Plan(257, 263, 269, torch.device("cuda", 0), dtype=torch.bfloat16, compute_dtype=torch.float16)
    assert plan.workspace_bytes == 48 * (65 * 66 + 66 * 68 + 65 * 68) * 2
    assert plan.prepacked_workspace_bytes == 48 * (65 * 66 + 65 * 68) * 2
    assert plan.packed_weight_bytes == 48 * 66 * 68 * 2
    rank49 = Rank49Plan(5, 6, 7, torch.device("cuda"))
    assert rank49.workspace_bytes == 3 * 49 * 2 * 2 * 2
    assert rank49.prepacked_workspace_bytes == 2 * 49 * 2 * 2 * 2
    assert rank49.packed_right_bytes == 49 * 2 * 2 * 2
    with pytest.raises(ValueError, match="does not support"):
        Rank48Plan(8, 8, 8, torch.device("cuda"), dtype=torch.float16)
    with pytest.raises(ValueError, match="does not support"):
        Rank7Plan(8, 8, 8, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="does not support"):
        Rank48Plan(8, 8, 8, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.bfloat16)
    # reference test_rdna3.py:713-723: rank 343 is FP16 only
    from rdna3_fastmm.runtime import Rank343Plan

    with pytest.raises(ValueError, match="does not support"):
        Rank343Plan(8, 8, 8, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.float16)
    assert Rank343Plan.rank == 343 and Rank343Plan.scheme_size == 8
    # rank 49 offers BF16 leaves like the reference (runtime.py:852-858); bytes follow compute_dtype
    bf16_leaves = Rank49Plan(5, 6, 7, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.bfloat16)
    assert bf16_leaves.compute_dtype == torch.bfloat16
    assert bf16_leaves.workspace_bytes == rank49.workspace_bytes


def test_memory_budget_is_checked_before_allocation(monkeypatch) -> None:
    configure_supported_runtime(monkeypatch)
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (1 << 28, 1 << 38))
    scratch = {"bytes": 0}
    monkeypatch.setattr(runtime._stages, "leaf_scratch_bytes", lambda *args: scratch["bytes"])
    plan = Rank7Plan(8192, 8192, 8192, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.float16)
    with pytest.raises(MemoryError, match="budget"):
        plan.allocate_workspace()
    # the leaf GEMM's split-K scratch counts against the same budget
    small = Rank7Plan(256, 256, 256, torch.device("cuda"), dtype=torch.bfloat16, compute_dtype=torch.float16)
    scratch["bytes"] = 1 << 28
    assert small.leaf_scratch_bytes == 1 << 28
    with pytest.raises(MemoryError, match="budget"):
        small.allocate_workspace()
    with pytest.raises(ValueError, match="interval"):
        plan.allocate_workspace(max_free_memory_fraction=0)


def test_measured_families_semantics(monkeypatch) -> None:
    """reference test_rdna3.py:152-288: row interval x exact (K, N) x bias; prepacked adds families."""
    monkeypatch.setattr(Rank7Plan, "linear_shape_families", (LinearShapeFamily(3_328, 9_216, 4_608, 12_288, False),))
    monkeypatch.setattr(Rank7Plan, "prepacked_linear_shape_families", (LinearShapeFamily(720, 720, 4_096, 16_384, True),))
    assert Rank7Plan.has_measured_linear_win((3_328, 4_608, 12_288), has_bias=False)
    assert Rank7Plan.has_measured_linear_win((9_216, 4_608, 12_288), has_bias=False)
    assert not Rank7Plan.has_measured_linear_win((9_217, 4_608, 12_288), has_bias=False)
    assert not Rank7Plan.has_measured_linear_win((4_000, 4_608, 12_288), has_bias=True)
    assert not Rank7Plan.has_measured_linear_win((720, 4_096, 16_384), has_bias=True)
    assert Rank7Plan.has_measured_linear_win((720, 4_096, 16_384), has_bias=True, prepacked_weight=True)
    assert not Rank7Plan.has_measured_linear_win((720, 4_096, 16_384), has_bias=False, prepacked_weight=True)


def test_dispatch_tables_hold_only_measured_wins() -> None:
    """Every family in the shipped tables must name a measured MI355X win."""
    for plan_type in (Rank7Plan, Rank48Plan, Rank49Plan):
        for family in plan_type.linear_shape_families + plan_type.prepacked_linear_shape_families:
            assert family in runtime.MEASURED_WINS, (plan_type.__name__, family)


def test_transform_config_reports_launch_geometry() -> None:
    assert Rank7Plan.transform_config(4_096, 12_288).block_elements == 256 * 8
    assert Rank48Plan.transform_config(8_192, 8_192).block_elements == 256 * 4
    assert Rank49Plan.transform_config(263, 269).block_elements == 256


def test_operand_layout_is_k_slab_major_exactly_when_kb_is_a_multiple_of_32() -> None:
    """The documented index: element (row, k) of a plane at ((k // 32) * rows + row) * 32 + k % 32."""
    import numpy as np

    from _layout import from_operand, to_operand
    from rdna3_fastmm.runtime import operand_shape

    assert operand_shape(7, 100, 256) == (7, 8, 100, 32)
    assert operand_shape(7, 100, 250) == (7, 100, 250)
    assert operand_shape(48, 5, 32) == (48, 1, 5, 32)
    rank, rows, inner = 3, 5, 64
    planes = np.arange(rank * rows * inner).reshape(rank, rows, inner)
    buffer = to_operand(planes)
    assert buffer.shape == operand_shape(rank, rows, inner)
    flat = buffer.reshape(rank, -1)
    for r in range(rank):
        for row in range(rows):
            for k in range(inner):
                assert flat[r, ((k // 32) * rows + row) * 32 + k % 32] == planes[r, row, k]
    assert np.array_equal(from_operand(buffer, rank, rows, inner), planes)
    ragged = np.arange(2 * 3 * 40).reshape(2, 3, 40)
    assert np.array_equal(to_operand(ragged), ragged)
    assert np.array_equal(from_operand(to_operand(ragged), 2, 3, 40), ragged)


def test_shipped_dispatch_table_is_consistent() -> None:
    """The MI355X table: measured wins only, above its margin, non-overlapping per pair."""
    import json

    document = json.loads(runtime.DISPATCH_TABLE_PATH.read_text())
    assert document["minimum_speedup"] >= 1.0 and document["error_ratio_bound"] == 1.2
    tables = runtime.load_dispatch_table()
    assert ("rank49", False) not in tables and ("rank49", True) not in tables  # error ratio 1.67 > 1.2
    for (scheme, prepacked), (families, notes) in tables.items():
        plan_type = runtime.PLAN_TYPES[scheme]
        installed = plan_type.prepacked_linear_shape_families if prepacked else plan_type.linear_shape_families
        assert installed == families
        by_pair: dict = {}
        for family in families:
            assert family in runtime.MEASURED_WINS and family in notes
            by_pair.setdefault((family.inner, family.columns, family.has_bias), []).append(family)
        for pair_families in by_pair.values():
            ordered = sorted(pair_families, key=lambda f: f.minimum_rows)
            for before, after in zip(ordered, ordered[1:]):
                assert before.maximum_rows < after.minimum_rows, (scheme, prepacked, before, after)
    # the corpus's Ideogram down projection is a measured rank-7 win; the up projection is not
    assert Rank7Plan.has_measured_linear_win((4704, 12288, 4608), has_bias=False, prepacked_weight=True)
    assert not Rank7Plan.has_measured_linear_win((4704, 4608, 12288), has_bias=False, prepacked_weight=True)
    # the north-star down projection at 8214 rows (between the 8192 and 8320 grid points,
    # measured by the refinement sweep) is a rank-7 and rank-48 win with and without bias
    for bias in (False, True):
        assert Rank7Plan.has_measured_linear_win((8214, 12288, 4608), has_bias=bias, prepacked_weight=True)
        assert Rank7Plan.has_measured_linear_win((8214, 12288, 4608), has_bias=bias)
        assert Rank48Plan.has_measured_linear_win((8214, 12288, 4608), has_bias=bias, prepacked_weight=True)
    assert not Rank7Plan.has_measured_linear_win((8192, 12288, 4608), has_bias=False, prepacked_weight=True)
    # down projections of Qwen3-32B, Gemma-2-27B and Yi-34B inside swept families
    assert Rank7Plan.has_measured_linear_win((8192, 25600, 5120), has_bias=False, prepacked_weight=True)
    assert Rank48Plan.has_measured_linear_win((10240, 25600, 5120), has_bias=False, prepacked_weight=True)
    assert Rank7Plan.has_measured_linear_win((12288, 36864, 4608), has_bias=False, prepacked_weight=True)
    assert Rank48Plan.has_measured_linear_win((5120, 20480, 7168), has_bias=False, prepacked_weight=True)
    # and of DeepSeek-V3's dense layers, Mixtral-8x22B and Gemma-3-12B
    assert Rank48Plan.has_measured_linear_win((5120, 18432, 7168), has_bias=False, prepacked_weight=True)
    assert Rank48Plan.has_measured_linear_win((7168, 16384, 6144), has_bias=False, prepacked_weight=True)
    assert Rank7Plan.has_measured_linear_win((10240, 15360, 3840), has_bias=False, prepacked_weight=True)
    # and of Mistral-Large-2 and Command-R+ (N = 12288)
    assert Rank48Plan.has_measured_linear_win((8192, 28672, 12288), has_bias=False, prepacked_weight=True)
    assert Rank48Plan.has_measured_linear_win((16384, 33792, 12288), has_bias=False, prepacked_weight=True)
    # square attention output projections, in the few row ranges where native is slow
    assert Rank48Plan.has_measured_linear_win((3072, 12288, 12288), has_bias=False, prepacked_weight=True)
    assert Rank48Plan.has_measured_linear_win((4864, 8192, 8192), has_bias=False, prepacked_weight=True)
    # the output projection of Flux's single-stream blocks (attention and MLP halves together)
    assert Rank7Plan.has_measured_linear_win((13312, 15360, 3072), has_bias=True, prepacked_weight=True)
    assert not Rank7Plan.has_measured_linear_win((13312, 15360, 3072), has_bias=False, prepacked_weight=True)
    # and of Mistral-Small-3 and Gemma-3-4B
    assert Rank48Plan.has_measured_linear_win((8192, 32768, 5120), has_bias=False, prepacked_weight=True)
    assert Rank7Plan.has_measured_linear_win((15360, 10240, 2560), has_bias=False, prepacked_weight=True)
    assert Rank7Plan.has_measured_linear_win((12800, 11008, 2048), has_bias=False, prepacked_weight=True)  # Qwen2.5-3B
    assert Rank7Plan.has_measured_linear_win((17024, 8192, 2048), has_bias=False, prepacked_weight=True)  # Llama-3.2-1B


@pytest.mark.parametrize(
    ("mutate", "message"),
    (
        (lambda d: d.update(schema_version=2), "unsupported dispatch schema"),
        (lambda d: d["families"][0].pop("runs"), "has keys"),
        (lambda d: d["families"][0].update(minimum_speedup=0.99), "not a measured win"),
        (lambda d: d["families"][0].update(minimum_rows=0), "not a measured win"),
        (lambda d: d["families"][0].update(maximum_rows=d["families"][0]["minimum_rows"] - 1), "not a measured win"),
    ),
)
def test_dispatch_loader_rejects_bad_tables(tmp_path, mutate, message) -> None:
    import json

    document = json.loads(runtime.DISPATCH_TABLE_PATH.read_text())
    mutate(document)
    path = tmp_path / "table.json"
    path.write_text(json.dumps(document))
    with pytest.raises(ValueError, match=message):
        runtime.load_dispatch_table(path)
