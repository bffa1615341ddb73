"""Write ``association_vectors.npz``: fp32 input/output vectors of the reference's
generated transform kernels, on inputs chosen so that any other summation order
rounds differently.

The reference's generator emits each scheme's programs as straight-line Triton
code (``src/rdna3_fastmm/generated/rank{7,48,49,343}_*.py``; emitters
``tools/generate_triton_scheme.py:133-337`` and
``tools/generate_slp_triton_scheme.py``). Each kernel body loads blocks, combines
them with ``+``, ``-``, unary ``-`` and scalings ``* 2``, ``/ 2`` and ``/ 4``,
and stores planes or C blocks. The values it stores depend on the association
order of those sums (``-signal_1 + signal_7 + signal_6`` is
``((-s1) + s7) + s6``), which the certificates alone do not fix.

This script reads those modules as text with ``ast.parse``. It does not import
them, and needs no Triton. It follows each kernel's statements in order with
numpy float32 arithmetic, one rounding per operation, as the kernel's fp32
values are computed. Block indices come from the address arithmetic:
``k * plane_elements`` names plane ``k``, and
``(r * block_height + ...) ... + c * block_width`` names block ``r * s + c``
(in the weight kernel, ``W`` block ``(c, r)``, which is ``W^T`` block
``(r, c)``). ``bias + c * block_width`` names bias block ``c``.

Inputs are ``N(0, 1)`` samples scaled by ``2**e``, ``e`` uniform in -10..10,
so partial sums span many binades. Rank 343's recombination is a dense
``tl.dot`` (``output_transform_mfma_kernel``), which has no emitted order, so
only its two transforms are recorded.

Run where the reference is present (it is never needed at test time):

    python tests/golden/make_association_vectors.py [/root/reference]
"""

from __future__ import annotations

import ast
import sys
from pathlib import Path

import numpy as np

SCHEMES = {
    # key: (module, block size s, rank)
    "rank7": ("rank7_2x2x2.py", 2, 7),
    "rank48": ("rank48_4x4x4.py", 4, 48),
    "rank49": ("rank49_4x4x4.py", 4, 49),
    "rank343": ("rank343_8x8x8.py", 8, 343),
}
KERNELS = {
    # kernel function: (fixture name, input kind)
    "left_transform_kernel": ("left", "blocks"),
    "right_transform_kernel": ("right", "blocks"),
    "right_transform_weight_kernel": ("weight", "blocks"),
    "output_transform_kernel": ("output", "planes"),
    "output_transform_bias_kernel": ("output_bias", "planes"),
}
SAMPLES = 32
SEED = 20261202
OUTPUT = Path(__file__).resolve().parent / "association_vectors.npz"


def _coefficients(node: ast.AST) -> dict[str, int]:
    """``{name: k}`` for every ``k * name`` product in an address expression."""
    found: dict[str, int] = {}
    for sub in ast.walk(node):
        if (
            isinstance(sub, ast.BinOp)
            and isinstance(sub.op, ast.Mult)
            and isinstance(sub.left, ast.Constant)
            and isinstance(sub.right, ast.Name)
        ):
            assert sub.right.id not in found, ast.dump(node)
            found[sub.right.id] = int(sub.left.value)
    return found


def _root_name(node: ast.AST) -> str:
    """The buffer an address expression starts from (``source``, ``bias``, ``output``)."""
    while isinstance(node, ast.BinOp):
        node = node.left
    assert isinstance(node, ast.Name), ast.dump(node)
    return node.id


def _unwrap_load(node: ast.AST) -> ast.Call | None:
    """The ``tl.load(...)`` call inside ``tl.load(...).to(tl.float32)`` or ``tl.trans(...)``."""
    if isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute):
        if node.func.attr == "load":
            return node
        if node.func.attr == "to":
            return _unwrap_load(node.func.value)
        if node.func.attr == "trans":
            return _unwrap_load(node.args[0])
    return None


def _index(address: ast.AST, s: int) -> tuple[str, int]:
    """(buffer, index) named by an address: a plane, a block or a bias block."""
    buffer = _root_name(address)
    k = _coefficients(address)
    if "plane_elements" in k:
        return buffer, k["plane_elements"]
    if buffer == "bias":
        return buffer, k["block_width"]
    return buffer, k["block_height"] * s + k["block_width"]


def _evaluate(node: ast.AST, values: dict[str, np.ndarray]) -> np.ndarray:
    if isinstance(node, ast.Name):
        return values[node.id]
    if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
        return -_evaluate(node.operand, values)
    assert isinstance(node, ast.BinOp), ast.dump(node)
    left = _evaluate(node.left, values)
    if isinstance(node.right, ast.Constant):
        factor = np.float32(node.right.value)
        assert factor in (2.0, 4.0), ast.dump(node)
        if isinstance(node.op, ast.Mult):
            return (left * factor).astype(np.float32)
        assert isinstance(node.op, ast.Div), ast.dump(node)
        return (left / factor).astype(np.float32)
    right = _evaluate(node.right, values)
    if isinstance(node.op, ast.Add):
        return (left + right).astype(np.float32)
    assert isinstance(node.op, ast.Sub), ast.dump(node)
    return (left - right).astype(np.float32)


def run_kernel(function: ast.FunctionDef, s: int, inputs: np.ndarray, bias: np.ndarray | None) -> dict[int, np.ndarray]:
    """Follow one kernel body: returns ``{output index: fp32 values}``."""
    values: dict[str, np.ndarray] = {}
    stored: dict[int, np.ndarray] = {}
    for statement in function.body:
        if isinstance(statement, ast.Assign):
            (target,) = statement.targets
            if not (isinstance(target, ast.Name) and target.id.startswith(("signal_", "bias_"))):
                continue  # offsets, masks and other index arithmetic
            load = _unwrap_load(statement.value)
            if load is None:
                values[target.id] = _evaluate(statement.value, values)
                continue
            buffer, index = _index(load.args[0], s)
            values[target.id] = inputs[index] if buffer == "source" else bias[index]
        elif isinstance(statement, ast.Expr) and isinstance(statement.value, ast.Call):
            call = statement.value
            if not (isinstance(call.func, ast.Attribute) and call.func.attr == "store"):
                continue
            buffer, index = _index(call.args[0], s)
            assert buffer == "output" and index not in stored, (function.name, index)
            stored[index] = _evaluate(call.args[1], values)
    return stored


def main(reference: Path) -> None:
    rng = np.random.default_rng(SEED)
    arrays: dict[str, np.ndarray] = {}
    for key, (module, s, rank) in SCHEMES.items():
        tree = ast.parse((reference / "src/rdna3_fastmm/generated" / module).read_text())
        functions = {f.name: f for f in tree.body if isinstance(f, ast.FunctionDef)}
        for kernel, (name, kind) in KERNELS.items():
            if kernel not in functions:
                continue
            count = s * s if kind == "blocks" else rank
            inputs = (rng.standard_normal((count, SAMPLES)) * 2.0 ** rng.integers(-10, 11, (count, SAMPLES)))
            inputs = inputs.astype(np.float32)
            bias = None
            if name == "output_bias":
                bias = (rng.standard_normal((s, SAMPLES)) * 2.0 ** rng.integers(-10, 11, (s, SAMPLES)))
                bias = bias.astype(np.float32)
            stored = run_kernel(functions[kernel], s, inputs, bias)
            expected = s * s if kind == "planes" else rank
            assert sorted(stored) == list(range(expected)), (key, kernel, sorted(stored))
            arrays[f"{key}.{name}.inputs"] = inputs
            if bias is not None:
                arrays[f"{key}.{name}.bias"] = bias
            arrays[f"{key}.{name}.outputs"] = np.stack([stored[i] for i in range(expected)])
            print(f"{key} {kernel}: {count} inputs -> {expected} outputs")
    np.savez_compressed(OUTPUT, **arrays)
    print(f"wrote {OUTPUT} ({OUTPUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
