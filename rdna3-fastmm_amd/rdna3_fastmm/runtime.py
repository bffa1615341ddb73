"""Fast-matmul plans for one MI355X: shape partition, workspaces, packing, launches.

The public surface is the reference's (``src/rdna3_fastmm/runtime.py``):
``Rank7Plan``, ``Rank48Plan``, ``Rank49Plan``, ``Workspace``,
``PackedWeight``, ``PackedRight``, ``MatrixShape``, ``LinearShapeFamily``,
``unsupported_runtime_reason``; same constructor, methods, byte formulas,
validation order and error types/messages, so callers and tests written
against the reference run unchanged. Every stage runs as a hand-written HIP
kernel of ``libfastmm_amd.so`` on the caller's current stream, asynchronously;
plans keep no state besides the shape.

Differences that are visible to a caller, all deliberate:

* ``PackedWeight.transformed`` / ``Workspace.right_transformed`` hold B' and
  ``Workspace.left_transformed`` holds A' in the layout the HIP kernels read
  (``operand_shape``): K-slab-major ``[R, Kb/32, Nb, 32]`` when ``Kb % 32 == 0``,
  else ``[R, Nb, Kb]`` -- instead of the reference's ``[R, Kb, Nb]``; the
  element values are the reference's, only their order differs (opaque
  snapshots either way).
* The runtime gate accepts gfx950 with 256 CUs on the torch/ROCm build this
  package was measured with, and the measured-win tables below were derived on
  that GPU against native BF16 ``torch.mm``/``F.linear``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
import json
from pathlib import Path
from typing import ClassVar

import torch

from . import _native, _stages
from .schemes import Scheme, load_scheme


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


SLAB_WIDTH = 32


def operand_shape(rank: int, rows: int, inner: int) -> tuple[int, ...]:
    """Buffer shape of a transformed operand (A': rows = Mb, B': rows = Nb).

    When ``inner`` (Kb) is a multiple of 32 the planes are K-slab-major,
    ``[R, Kb/32, rows, 32]``: the 32-wide K slice of any run of rows is
    contiguous, which is how the leaf-GEMM kernels stream tiles. Otherwise
    they are row-major ``[R, rows, Kb]``. Same element count either way.
    """
    if inner % SLAB_WIDTH == 0:
        return (rank, inner // SLAB_WIDTH, rows, SLAB_WIDTH)
    return (rank, rows, inner)


@dataclass(frozen=True)
class MatrixShape:
    """reference runtime.py:56-89."""

    rows: int
    inner: int
    columns: int
    block_rows: int
    block_inner: int
    block_columns: int

    @classmethod
    def from_dimensions(cls, rows: int, inner: int, columns: int, scheme_size: int) -> "MatrixShape":
        if min(rows, inner, columns) < 1:
            raise ValueError("matrix dimensions must be positive")
        return cls(
            rows=rows,
            inner=inner,
            columns=columns,
            block_rows=_ceil_div(rows, scheme_size),
            block_inner=_ceil_div(inner, scheme_size),
            block_columns=_ceil_div(columns, scheme_size),
        )

    @property
    def dimensions(self) -> tuple[int, int, int]:
        return self.rows, self.inner, self.columns

    def workspace_elements(self, rank: int) -> int:
        return rank * (
            self.block_rows * self.block_inner
            + self.block_inner * self.block_columns
            + self.block_rows * self.block_columns
        )


@dataclass
class Workspace:
    algorithm: str
    output_dtype: torch.dtype
    compute_dtype: torch.dtype
    left_transformed: torch.Tensor
    right_transformed: torch.Tensor | None
    products: torch.Tensor
    # MI355X-specific: bytes for the leaf GEMM's split-K tail (None when the
    # shape has none, or for a workspace built by hand: the tail then runs as
    # whole tiles). Not part of the reference's byte formulas.
    leaf_scratch: torch.Tensor | None = None


@dataclass(frozen=True)
class _PackedTransform:
    algorithm: str
    source_dtype: torch.dtype
    compute_dtype: torch.dtype
    transformed: torch.Tensor
    source_shape: tuple[int, int]


@dataclass(frozen=True)
class PackedRight(_PackedTransform):
    pass


@dataclass(frozen=True)
class PackedWeight(_PackedTransform):
    pass


@dataclass(frozen=True)
class LinearShapeFamily:
    """Rows interval x exact (inner, columns) x bias, where a win was measured.

    ``measured_speedup`` is the smallest speedup over native measured inside the
    family (0.0 when unknown, e.g. a family built by hand); it ranks plans when
    families of several schemes cover one shape. It takes no part in equality.
    """

    minimum_rows: int
    maximum_rows: int
    inner: int
    columns: int
    has_bias: bool
    measured_speedup: float = field(default=0.0, compare=False)

    def matches(self, shape: tuple[int, int, int], has_bias: bool) -> bool:
        rows, inner, columns = shape
        return (
            self.minimum_rows <= rows <= self.maximum_rows
            and inner == self.inner
            and columns == self.columns
            and has_bias == self.has_bias
        )


@dataclass(frozen=True)
class ElementTransformConfig:
    """Launch geometry of the elementwise transforms: elements per workgroup."""

    block_elements: int
    warps: int


@dataclass(frozen=True)
class WeightTransformConfig:
    block_rows: int
    block_columns: int
    warps: int


# --------------------------------------------------------------- runtime gate

TESTED_ARCHITECTURE = "gfx950"
TESTED_COMPUTE_UNITS = 256
TESTED_TORCH_PREFIX = "2.10.0+"
TESTED_HIP_PREFIX = "7.0"


def unsupported_runtime_reason(device: torch.device | None = None) -> str | None:
    """Why the measured dispatch tables do not apply here (None = they do).

    reference runtime.py:970-994, retargeted to one MI355X.
    """
    hip_version = torch.version.hip
    if hip_version is None:
        return "requires a ROCm PyTorch build"
    if not torch.cuda.is_available():
        return "requires an available ROCm GPU"
    resolved = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    if resolved.type != "cuda":
        return "requires a ROCm GPU device"
    properties = torch.cuda.get_device_properties(resolved)
    architecture = getattr(properties, "gcnArchName", "").split(":")[0]
    if architecture != TESTED_ARCHITECTURE or properties.multi_processor_count != TESTED_COMPUTE_UNITS:
        return (
            f"tested only on {TESTED_ARCHITECTURE} with {TESTED_COMPUTE_UNITS} compute units; "
            f"found {architecture or 'unknown'} with {properties.multi_processor_count}"
        )
    if not torch.__version__.startswith(TESTED_TORCH_PREFIX):
        return f"tested only with PyTorch 2.10.0; found {torch.__version__}"
    if not hip_version.startswith(TESTED_HIP_PREFIX):
        return f"tested only with ROCm {TESTED_HIP_PREFIX}; found {hip_version}"
    return None


def is_tested_runtime(device: torch.device) -> bool:
    return unsupported_runtime_reason(device) is None


# ------------------------------------------------------------- dispatch data

# Shape families where a plan beat native BF16 on one MI355X (reference
# runtime.py:793-806, 831-838, 866-871 hold the RDNA3 tables). They are
# measured, not modelled: ``python -m rdna3_fastmm.corpus --sweep`` times each
# plan against native F.linear / torch.mm over a row sweep of a (K, N, bias)
# pair, repeated on separate boxes, and a family is a run of swept rows where
# every measurement beat native by the table's margin within the error bound.
# Native hipBLASLt is fast on the MLP up projections (no family there) but
# picks slow kernels for many row counts of the down projections, where the
# plans' time stays smooth in M. The rewrite and is_linear_recommended only
# ever select a family listed here.
DISPATCH_TABLE_PATH = Path(__file__).resolve().parent / "dispatch" / "mi355x.json"
_FAMILY_KEYS = {"scheme", "prepacked", "minimum_rows", "maximum_rows", "inner", "columns", "bias", "points",
                "runs", "minimum_speedup"}


def load_dispatch_table(path: Path = DISPATCH_TABLE_PATH) -> dict[tuple[str, bool], tuple[tuple[LinearShapeFamily, ...], dict[LinearShapeFamily, str]]]:
    """(scheme, prepacked) -> (families, evidence per family) from a dispatch file."""
    document = json.loads(Path(path).read_text())
    if document.get("schema_version") != 1:
        raise ValueError(f"{path}: unsupported dispatch schema {document.get('schema_version')!r}")
    tables: dict[tuple[str, bool], tuple[list[LinearShapeFamily], dict[LinearShapeFamily, str]]] = {}
    for index, entry in enumerate(document["families"]):
        if set(entry) != _FAMILY_KEYS:
            raise ValueError(f"{path}: families[{index}] has keys {sorted(entry)}")
        if not (0 < entry["minimum_rows"] <= entry["maximum_rows"]) or entry["minimum_speedup"] < document["minimum_speedup"]:
            raise ValueError(f"{path}: families[{index}] is not a measured win")
        family = LinearShapeFamily(entry["minimum_rows"], entry["maximum_rows"], entry["inner"], entry["columns"],
                                   entry["bias"], float(entry["minimum_speedup"]))
        mode = "prepacked" if entry["prepacked"] else "dynamic"
        evidence = (f"{entry['scheme']} {mode}: >= {entry['minimum_speedup']}x native at {entry['points']} swept "
                    f"row counts, {entry['runs']} runs each")
        families, notes = tables.setdefault((entry["scheme"], entry["prepacked"]), ([], {}))
        families.append(family)
        notes[family] = evidence
    return {key: (tuple(families), notes) for key, (families, notes) in tables.items()}


MEASURED_WINS: dict[LinearShapeFamily, str] = {}


# ---------------------------------------------------------------------- plans

_VERIFIED_SCHEMES: set[int] = set()


def _check_library_scheme(scheme: Scheme) -> None:
    """The kernels must be generated from the certificate verified here."""
    if scheme.scheme_id in _VERIFIED_SCHEMES:
        return
    compiled = _native.scheme_sha256(scheme.scheme_id)
    if compiled != scheme.certificate_sha256:
        raise RuntimeError("compiled kernel metadata does not match the backend")
    _VERIFIED_SCHEMES.add(scheme.scheme_id)


class _Plan:
    algorithm: ClassVar[str]
    scheme_key: ClassVar[str]
    rank: ClassVar[int]
    scheme_size: ClassVar[int]
    precision_pairs: ClassVar[frozenset[tuple[torch.dtype, torch.dtype]]]
    dynamic_shapes: ClassVar[frozenset[tuple[int, int, int]]] = frozenset()
    prepacked_shapes: ClassVar[frozenset[tuple[int, int, int]]] = frozenset()

    def __init__(
        self,
        rows: int,
        inner: int,
        columns: int,
        device: torch.device,
        dtype: torch.dtype = torch.float16,
        compute_dtype: torch.dtype | None = None,
    ) -> None:
        device = torch.device(device)
        if device.type != "cuda" or torch.version.hip is None or not torch.cuda.is_available():
            raise ValueError("the MI355X backend requires a ROCm device")
        resolved_compute = dtype if compute_dtype is None else compute_dtype
        if (dtype, resolved_compute) not in self.precision_pairs:
            raise ValueError(
                f"{self.algorithm} does not support {dtype} inputs with "
                f"{resolved_compute} leaf products"
            )
        index = torch.cuda.current_device() if device.index is None else device.index
        self.device = torch.device("cuda", index)
        self.dtype = dtype
        self.compute_dtype = resolved_compute
        self.scheme = load_scheme(self.scheme_key)
        _check_library_scheme(self.scheme)
        self.shape = MatrixShape.from_dimensions(rows, inner, columns, self.scheme_size)

    # ------------------------------------------------------------ byte counts

    @property
    def workspace_bytes(self) -> int:
        return self._workspace_bytes(prepacked_right=False)

    @property
    def prepacked_workspace_bytes(self) -> int:
        return self._workspace_bytes(prepacked_right=True)

    @property
    def packed_right_bytes(self) -> int:
        shape = self.shape
        return self.rank * shape.block_inner * shape.block_columns * self.compute_dtype.itemsize

    @property
    def leaf_scratch_bytes(self) -> int:
        """Device bytes of ``Workspace.leaf_scratch`` (the leaf GEMM's split-K tail)."""
        shape = self.shape
        return _stages.leaf_scratch_bytes(
            self.rank, self.compute_dtype, self.compute_dtype, shape.block_rows, shape.block_inner,
            shape.block_columns, self.device,
        )

    def _workspace_bytes(self, prepacked_right: bool) -> int:
        shape = self.shape
        elements = self.rank * (
            shape.block_rows * shape.block_inner + shape.block_rows * shape.block_columns
        )
        if not prepacked_right:
            elements += self.rank * shape.block_inner * shape.block_columns
        return elements * self.compute_dtype.itemsize

    def is_recommended(self, *, prepacked_right: bool = False) -> bool:
        shapes = self.prepacked_shapes if prepacked_right else self.dynamic_shapes
        return (
            self.dtype == torch.float16
            and self.compute_dtype == torch.float16
            and self.shape.dimensions in shapes
            and is_tested_runtime(self.device)
        )

    # ------------------------------------------------------------- allocation

    def allocate_workspace(
        self, max_free_memory_fraction: float = 0.75, *, prepacked_right: bool = False
    ) -> Workspace:
        scratch_bytes = self.leaf_scratch_bytes
        self._ensure_memory_budget(
            self._workspace_bytes(prepacked_right) + scratch_bytes, max_free_memory_fraction,
            f"{self.algorithm} workspace",
        )
        shape = self.shape
        return Workspace(
            algorithm=self.algorithm,
            output_dtype=self.dtype,
            compute_dtype=self.compute_dtype,
            left_transformed=self._empty(operand_shape(self.rank, shape.block_rows, shape.block_inner)),
            right_transformed=None
            if prepacked_right
            else self._empty(operand_shape(self.rank, shape.block_columns, shape.block_inner)),
            products=self._empty((self.rank, shape.block_rows, shape.block_columns)),
            leaf_scratch=torch.empty(scratch_bytes, device=self.device, dtype=torch.uint8) if scratch_bytes else None,
        )

    def _empty(self, shape: tuple[int, ...]) -> torch.Tensor:
        return torch.empty(shape, device=self.device, dtype=self.compute_dtype)

    def pack_right(self, right: torch.Tensor, max_free_memory_fraction: float = 0.75) -> PackedRight:
        self._validate_right(right)
        self._ensure_memory_budget(
            self.packed_right_bytes, max_free_memory_fraction, f"{self.algorithm} packed right matrix"
        )
        shape = self.shape
        transformed = self._empty(operand_shape(self.rank, shape.block_columns, shape.block_inner))
        self._transform_right(right, transformed)
        return PackedRight(
            algorithm=self.algorithm,
            source_dtype=self.dtype,
            compute_dtype=self.compute_dtype,
            transformed=transformed,
            source_shape=(shape.inner, shape.columns),
        )

    # -------------------------------------------------------------- mm path

    def run(
        self,
        left: torch.Tensor,
        right: torch.Tensor,
        workspace: Workspace,
        output: torch.Tensor | None = None,
    ) -> torch.Tensor:
        self._validate_left(left)
        self._validate_right(right)
        self._validate_workspace(workspace, require_right=True)
        result = self._output(output)
        self._validate_output_storage(
            result, left, right, workspace.left_transformed, workspace.products, workspace.right_transformed,
            workspace.leaf_scratch,
        )
        right_transformed = workspace.right_transformed
        assert right_transformed is not None
        self._transform_left(left, workspace.left_transformed)
        self._transform_right(right, right_transformed)
        self._leaf_products(workspace.left_transformed, right_transformed, workspace.products, workspace.leaf_scratch)
        self._reconstruct(workspace.products, None, result)
        return result

    def run_packed(
        self,
        left: torch.Tensor,
        right: PackedRight,
        workspace: Workspace,
        output: torch.Tensor | None = None,
    ) -> torch.Tensor:
        self._validate_left(left)
        self._validate_packed_right(right)
        self._validate_workspace(workspace, require_right=False)
        result = self._output(output)
        self._validate_separate_storage(right.transformed, workspace.left_transformed, workspace.products)
        self._validate_output_storage(
            result,
            left,
            right.transformed,
            workspace.left_transformed,
            workspace.products,
            workspace.right_transformed,
            workspace.leaf_scratch,
        )
        self._transform_left(left, workspace.left_transformed)
        self._leaf_products(workspace.left_transformed, right.transformed, workspace.products, workspace.leaf_scratch)
        self._reconstruct(workspace.products, None, result)
        return result

    # ---------------------------------------------------------------- stages

    def _transform_left(self, source: torch.Tensor, output: torch.Tensor) -> None:
        _stages.left_transform(self.scheme, source, output, self.shape.rows, self.shape.inner)

    def _transform_right(self, source: torch.Tensor, output: torch.Tensor) -> None:
        _stages.right_transform(self.scheme, source, output, self.shape.inner, self.shape.columns)

    def _transform_weight(self, source: torch.Tensor, output: torch.Tensor) -> None:
        _stages.weight_transform(self.scheme, source, output, self.shape.columns, self.shape.inner)

    def _leaf_products(
        self, left: torch.Tensor, right: torch.Tensor, products: torch.Tensor, scratch: torch.Tensor | None = None
    ) -> None:
        shape = self.shape
        _stages.leaf_products(
            self.rank, left, right, products, shape.block_rows, shape.block_inner, shape.block_columns, scratch
        )

    def _reconstruct(self, products: torch.Tensor, bias: torch.Tensor | None, output: torch.Tensor) -> None:
        _stages.reconstruct(self.scheme, products, bias, output, self.shape.rows, self.shape.columns)

    # ------------------------------------------------------------ validation

    def _validate_left(self, tensor: torch.Tensor) -> None:
        self._validate_tensor(tensor, (self.shape.rows, self.shape.inner), "left")

    def _validate_right(self, tensor: torch.Tensor) -> None:
        self._validate_tensor(tensor, (self.shape.inner, self.shape.columns), "right")

    def _validate_weight(self, tensor: torch.Tensor) -> None:
        self._validate_tensor(tensor, (self.shape.columns, self.shape.inner), "weight")

    def _validate_bias(self, tensor: torch.Tensor) -> None:
        self._validate_tensor(tensor, (self.shape.columns,), "bias")

    def _validate_tensor(self, tensor: torch.Tensor, shape: tuple[int, ...], name: str) -> None:
        if tuple(tensor.shape) != shape:
            raise ValueError(f"{name} matrix has shape {tuple(tensor.shape)}, expected {shape}")
        if tensor.device != self.device or tensor.dtype != self.dtype:
            raise ValueError(f"{name} matrix device or dtype does not match the plan")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} matrix must be contiguous")
        if tensor.requires_grad:
            raise ValueError("the MI355X fast-matmul backend does not support autograd")

    def _validate_workspace(self, workspace: Workspace, *, require_right: bool) -> None:
        if (
            workspace.algorithm != self.algorithm
            or workspace.output_dtype != self.dtype
            or workspace.compute_dtype != self.compute_dtype
        ):
            raise ValueError("workspace does not match the plan")
        shape = self.shape
        expected = [
            (workspace.left_transformed, operand_shape(self.rank, shape.block_rows, shape.block_inner)),
            (workspace.products, (self.rank, shape.block_rows, shape.block_columns)),
        ]
        if require_right:
            if workspace.right_transformed is None:
                raise ValueError("dynamic execution requires a dynamic workspace")
            expected.append(
                (workspace.right_transformed, operand_shape(self.rank, shape.block_columns, shape.block_inner))
            )
        for tensor, tensor_shape in expected:
            if (
                tuple(tensor.shape) != tensor_shape
                or tensor.device != self.device
                or tensor.dtype != self.compute_dtype
                or not tensor.is_contiguous()
                or tensor.requires_grad
            ):
                raise ValueError("workspace does not match the plan")
        scratch = workspace.leaf_scratch
        if scratch is not None and (
            scratch.device != self.device or scratch.dtype != torch.uint8 or scratch.dim() != 1
            or not scratch.is_contiguous()
        ):
            raise ValueError("workspace does not match the plan")
        tensors = [tensor for tensor, _ in expected]
        if scratch is not None and scratch.numel():
            tensors.append(scratch)
        self._validate_separate_storage(*tensors)

    def _validate_packed_right(self, packed: PackedRight) -> None:
        if not isinstance(packed, PackedRight):
            raise ValueError("packed right matrix does not match the plan")
        self._validate_packed_transform(packed, (self.shape.inner, self.shape.columns), "right matrix")

    def _validate_packed_transform(
        self, packed: _PackedTransform, expected_source_shape: tuple[int, int], name: str
    ) -> None:
        if (
            packed.algorithm != self.algorithm
            or packed.source_dtype != self.dtype
            or packed.compute_dtype != self.compute_dtype
        ):
            raise ValueError(f"packed {name} does not match the plan")
        if tuple(packed.source_shape) != expected_source_shape:
            raise ValueError(f"packed {name} shape does not match the plan")
        shape = self.shape
        transformed = packed.transformed
        if (
            tuple(transformed.shape) != operand_shape(self.rank, shape.block_columns, shape.block_inner)
            or transformed.device != self.device
            or transformed.dtype != self.compute_dtype
            or not transformed.is_contiguous()
            or transformed.requires_grad
        ):
            raise ValueError(f"packed {name} does not match the plan")

    def _output(self, output: torch.Tensor | None) -> torch.Tensor:
        shape = (self.shape.rows, self.shape.columns)
        if output is None:
            return torch.empty(shape, device=self.device, dtype=self.dtype)
        self._validate_tensor(output, shape, "output")
        return output

    def _ensure_memory_budget(self, required_bytes: int, max_free_memory_fraction: float, name: str) -> None:
        if not 0 < max_free_memory_fraction <= 1:
            raise ValueError("memory fraction must be in the interval (0, 1]")
        free_bytes, _ = torch.cuda.mem_get_info(self.device)
        budget = free_bytes * max_free_memory_fraction
        if required_bytes > budget:
            raise MemoryError(
                f"{name} needs {required_bytes / 2**30:.2f} GiB, exceeding the {budget / 2**30:.2f} GiB budget"
            )

    def _validate_output_storage(self, output: torch.Tensor, *tensors: torch.Tensor | None) -> None:
        for tensor in tensors:
            if tensor is not None and _storage_overlaps(output, tensor):
                raise ValueError("output storage must not overlap inputs or workspace")

    def _validate_separate_storage(self, *tensors: torch.Tensor) -> None:
        for index, tensor in enumerate(tensors):
            if any(_storage_overlaps(tensor, other) for other in tensors[index + 1:]):
                raise ValueError("work buffers must not overlap")


def _storage_overlaps(first: torch.Tensor, second: torch.Tensor) -> bool:
    first_start = first.data_ptr()
    first_end = first_start + first.numel() * first.element_size()
    second_start = second.data_ptr()
    second_end = second_start + second.numel() * second.element_size()
    return first_start < second_end and second_start < first_end


class _LinearPlan(_Plan):
    linear_shape_families: ClassVar[tuple[LinearShapeFamily, ...]] = ()
    prepacked_linear_shape_families: ClassVar[tuple[LinearShapeFamily, ...]] = ()

    @classmethod
    def has_measured_linear_win(
        cls, shape: tuple[int, int, int], *, has_bias: bool, prepacked_weight: bool = False
    ) -> bool:
        families = cls.linear_shape_families
        if prepacked_weight:
            families += cls.prepacked_linear_shape_families
        return any(family.matches(tuple(shape), has_bias) for family in families)

    @classmethod
    def measured_linear_speedup(
        cls, shape: tuple[int, int, int], *, has_bias: bool, prepacked_weight: bool = False
    ) -> float | None:
        """Largest measured speedup of the families covering ``shape`` (None: no win)."""
        families = cls.linear_shape_families
        if prepacked_weight:
            families += cls.prepacked_linear_shape_families
        speedups = [family.measured_speedup for family in families if family.matches(tuple(shape), has_bias)]
        return max(speedups) if speedups else None

    def is_linear_recommended(self, *, has_bias: bool, prepacked_weight: bool = False) -> bool:
        return (
            self.dtype == torch.bfloat16
            and self.compute_dtype == torch.float16
            and self.has_measured_linear_win(
                self.shape.dimensions, has_bias=has_bias, prepacked_weight=prepacked_weight
            )
            and is_tested_runtime(self.device)
        )

    @classmethod
    def transform_config(cls, inner: int, columns: int) -> ElementTransformConfig:
        """Geometry the elementwise transforms launch with (256 lanes, 4 waves)."""
        per_lane = 8 if cls.rank <= 8 else 4
        if inner % (cls.scheme_size * per_lane) or columns % (cls.scheme_size * per_lane):
            per_lane = 1
        return ElementTransformConfig(256 * per_lane, 4)

    @classmethod
    def weight_transform_config(cls, inner: int, columns: int) -> WeightTransformConfig:
        """The weight transform is the same K-contiguous elementwise pass."""
        config = cls.transform_config(inner, columns)
        return WeightTransformConfig(1, config.block_elements, config.warps)

    @property
    def packed_weight_bytes(self) -> int:
        return self.packed_right_bytes

    def pack_weight(self, weight: torch.Tensor, max_free_memory_fraction: float = 0.75) -> PackedWeight:
        self._validate_weight(weight)
        self._ensure_memory_budget(
            self.packed_weight_bytes, max_free_memory_fraction, f"{self.algorithm} packed Linear weight"
        )
        shape = self.shape
        transformed = self._empty(operand_shape(self.rank, shape.block_columns, shape.block_inner))
        self._transform_weight(weight, transformed)
        return PackedWeight(
            algorithm=self.algorithm,
            source_dtype=self.dtype,
            compute_dtype=self.compute_dtype,
            transformed=transformed,
            source_shape=(shape.columns, shape.inner),
        )

    def _validate_packed_weight(self, packed: PackedWeight) -> None:
        if not isinstance(packed, PackedWeight):
            raise ValueError("packed Linear weight does not match the plan")
        self._validate_packed_transform(packed, (self.shape.columns, self.shape.inner), "Linear weight")

    def run_linear(
        self,
        input_tensor: torch.Tensor,
        weight: torch.Tensor,
        workspace: Workspace,
        bias: torch.Tensor | None = None,
        output: torch.Tensor | None = None,
    ) -> torch.Tensor:
        self._validate_left(input_tensor)
        self._validate_weight(weight)
        if bias is not None:
            self._validate_bias(bias)
        self._validate_workspace(workspace, require_right=True)
        result = self._output(output)
        self._validate_output_storage(
            result,
            input_tensor,
            weight,
            bias,
            workspace.left_transformed,
            workspace.products,
            workspace.right_transformed,
            workspace.leaf_scratch,
        )
        right_transformed = workspace.right_transformed
        assert right_transformed is not None
        self._transform_left(input_tensor, workspace.left_transformed)
        self._transform_weight(weight, right_transformed)
        self._leaf_products(workspace.left_transformed, right_transformed, workspace.products, workspace.leaf_scratch)
        self._reconstruct(workspace.products, bias, result)
        return result

    def run_linear_packed(
        self,
        input_tensor: torch.Tensor,
        weight: PackedWeight,
        workspace: Workspace,
        bias: torch.Tensor | None = None,
        output: torch.Tensor | None = None,
    ) -> torch.Tensor:
        self._validate_left(input_tensor)
        self._validate_packed_weight(weight)
        if bias is not None:
            self._validate_bias(bias)
        self._validate_workspace(workspace, require_right=False)
        self._validate_separate_storage(weight.transformed, workspace.left_transformed, workspace.products)
        result = self._output(output)
        self._validate_output_storage(
            result,
            input_tensor,
            weight.transformed,
            bias,
            workspace.left_transformed,
            workspace.products,
            workspace.right_transformed,
            workspace.leaf_scratch,
        )
        self._transform_left(input_tensor, workspace.left_transformed)
        self._leaf_products(workspace.left_transformed, weight.transformed, workspace.products, workspace.leaf_scratch)
        self._reconstruct(workspace.products, bias, result)
        return result


class Rank7Plan(_LinearPlan):
    """<2,2,2> rank 7 (Strassen-Winograd, 15 additions); reference runtime.py:780-820."""

    algorithm = "rank7-v1"
    scheme_key = "rank7"
    rank = 7
    scheme_size = 2
    precision_pairs = frozenset({(torch.float16, torch.float16), (torch.bfloat16, torch.float16)})


class Rank48Plan(_LinearPlan):
    """<4,4,4> rank 48, dyadic-rational SLP; reference runtime.py:823-844."""

    algorithm = "rank48-accurate-v1"
    scheme_key = "rank48"
    rank = 48
    scheme_size = 4
    precision_pairs = frozenset({(torch.bfloat16, torch.float16)})


class Rank49Plan(_LinearPlan):
    """<4,4,4> rank 49 (159 additions); reference runtime.py:847-880."""

    algorithm = "rank49-v1"
    scheme_key = "rank49"
    rank = 49
    scheme_size = 4
    # (bf16, bf16): BF16 planes, BF16 MFMA leaves and BF16 products, as the reference
    # offers (runtime.py:852-858); far less accurate than the fp16-leaf pairs.
    precision_pairs = frozenset(
        {
            (torch.float16, torch.float16),
            (torch.bfloat16, torch.bfloat16),
            (torch.bfloat16, torch.float16),
        }
    )


class Rank343Plan(_Plan):
    """<8,8,8> rank 343 (1661 additions), FP16 ``mm`` only; reference runtime.py:883-962.

    Only the ``mm`` path (``pack_right``, ``run``, ``run_packed``): the reference
    offers no Linear plan for it. The recombination is the reference's dense
    form (``MFMA_OUTPUT_COEFFICIENTS``: each output block one FP16 MFMA
    contraction of the products with the -1/0/1 output matrix, fp32
    accumulation) when the plan's buffers allow it: fp16 products, columns a
    multiple of 64, products 16-byte and output 8-byte aligned (always so for
    the plan's own workspace and a fresh output). Otherwise the certificate's
    output circuit runs in fp32; the two agree up to fp32 summation order.
    ``prepacked_shapes`` and ``dynamic_shapes`` hold MI355X-measured wins only.
    """

    algorithm = "rank343-mfma-v1"
    scheme_key = "rank343"
    rank = 343
    scheme_size = 8
    precision_pairs = frozenset({(torch.float16, torch.float16)})
    # Prepacked 16384^3 beat FP16 torch.mm on two MI355X boxes (1.09-1.12x with
    # the dense recombination; bench.py --config c6-rank343); the dynamic path
    # (right transform per call) does not (0.89x with the circuit recombination).
    # Smaller squares lose (0.74x at 8192^3).
    prepacked_shapes = frozenset({(16_384, 16_384, 16_384)})


PLAN_TYPES: dict[str, type[_LinearPlan]] = {"rank7": Rank7Plan, "rank48": Rank48Plan, "rank49": Rank49Plan}


def _install_dispatch_table(path: Path = DISPATCH_TABLE_PATH) -> None:
    for (scheme, prepacked), (families, notes) in load_dispatch_table(path).items():
        plan_type = PLAN_TYPES[scheme]
        if prepacked:
            plan_type.prepacked_linear_shape_families = families
        else:
            plan_type.linear_shape_families = families
        for family, note in notes.items():
            MEASURED_WINS[family] = f"{MEASURED_WINS[family]}; {note}" if family in MEASURED_WINS else note


_install_dispatch_table()

Rank7Workspace = Workspace
Rank49Workspace = Workspace
Rank343Workspace = Workspace
