"""Emit gfx950 HIP device code for a scheme's three straight-line programs.

The reference emits one Triton kernel per program (``tools/
generate_triton_scheme.py:133-337``, ``tools/generate_slp_triton_scheme.py:
65-132``). Here the emitter produces only the *program*: a ``__device__``
template that evaluates the straight-line program on an abstract value type
``V`` and hands every output to a ``store`` callback as soon as it is final.
The memory side (which blocks to read, coalesced 128-bit vectors, zero
padding, where outputs go) lives once in the hand-written kernels of
``csrc/transforms.hip``, which instantiate these programs for every scheme.

Rounding order: every expression node becomes one fp32 operation in tree
order (left operand first), which is the order the reference's kernels
evaluate in; ``/2^j`` is emitted as ``* 2^-j`` (the same correctly rounded
value). The kernels are built with ``-ffp-contract=off`` so nothing fuses.

Usage: ``python -m rdna3_fastmm.hipgen [output_dir]`` rewrites
``csrc/generated/*.h``; ``tests/test_hipgen.py`` checks the checked-in files
are current.
"""

from __future__ import annotations

import argparse
from fractions import Fraction
from pathlib import Path
import sys

from .program import Add, Expr, LinearProgram, Neg, Scale, Sig, Sub, expression_signals
from .schemes import SCHEME_KEYS, Scheme, load_scheme

GENERATED_DIR = Path(__file__).resolve().parent.parent / "csrc" / "generated"


def _literal(factor: Fraction) -> str:
    value = float(factor)
    if Fraction(value) != factor or value == 0:
        raise ValueError(f"scaling {factor} is not exact in fp32")
    text = repr(value)
    return f"{text}f"


def _expression(expr: Expr) -> str:
    if isinstance(expr, Sig):
        return f"s{expr.index}"
    if isinstance(expr, Add):
        return f"({_expression(expr.left)} + {_expression(expr.right)})"
    if isinstance(expr, Sub):
        return f"({_expression(expr.left)} - {_expression(expr.right)})"
    if isinstance(expr, Neg):
        return f"(-{_expression(expr.operand)})"
    return f"({_expression(expr.operand)} * {_literal(expr.factor)})"


def emit_program(function: str, program: LinearProgram, comment: str) -> str:
    """One ``__device__`` template evaluating ``program`` in step order.

    ``load(i)`` returns input ``i`` as ``V``; ``store(k, v)`` receives output
    ``k``. Inputs are loaded at first use; each output is stored right after
    the step that defines it (outputs that are plain inputs right after the
    load).
    """
    output_of: dict[int, list[int]] = {}
    for index, signal in enumerate(program.outputs):
        output_of.setdefault(signal, []).append(index)
    lines = [
        f"// {comment}",
        f"// {program.input_count} inputs, {len(program.steps)} steps, "
        f"{program.additions} additions, {program.scalings} scalings, "
        f"{program.output_count} outputs.",
        "template <class V, class Load, class Store>",
        f"static __device__ __forceinline__ void {function}(const Load& load, const Store& store) {{",
    ]
    loaded: set[int] = set()

    def ensure_loaded(index: int) -> None:
        if index < program.input_count and index not in loaded:
            loaded.add(index)
            lines.append(f"  const V s{index} = load({index});")
            for output in output_of.get(index, []):
                lines.append(f"  store({output}, s{index});")

    for step in program.steps:
        for index in expression_signals(step.expr):
            ensure_loaded(index)
        lines.append(f"  const V s{step.signal} = {_expression(step.expr)};  // {step.name}")
        for output in output_of.get(step.signal, []):
            lines.append(f"  store({output}, s{step.signal});")
    for signal in program.outputs:
        ensure_loaded(signal)
    lines.append("}")
    return "\n".join(lines)


def emit_output_matrix(program: LinearProgram) -> str:
    """The C-side map as a dense int8 matrix, ``kOutputMatrix[c][r]``.

    Emitted for the 8x8-block scheme, whose recombination runs as one dense
    MFMA contraction over the products, as in the reference
    (``generated/rank343_8x8x8.py`` ``MFMA_OUTPUT_COEFFICIENTS``, written
    rank-major there; here output-major, the layout the kernel stages). Every
    coefficient must be an integer in [-128, 127].
    """
    rows = program.coefficients()
    for row in rows:
        for value in row:
            if value.denominator != 1 or not -128 <= value.numerator <= 127:
                raise ValueError("the dense output matrix needs int8 coefficients")
    lines = [
        f"// Output c = sum over r of kOutputMatrix[c][r] * P[r] ({program.output_count} x {program.input_count}).",
        f"static constexpr signed char kOutputMatrix[{program.output_count}][{program.input_count}] = {{",
    ]
    for row in rows:
        lines.append("    {" + ",".join(str(value.numerator) for value in row) + "},")
    lines.append("};")
    return "\n".join(lines)


def _guard(scheme: Scheme) -> str:
    return f"FASTMM_GENERATED_{scheme.name.upper()}_H"


def emit_scheme_header(scheme: Scheme) -> str:
    relative = scheme.certificate.relative_to(scheme.certificate.parents[2])
    parts = [
        "// Generated by `python -m rdna3_fastmm.hipgen`; do not edit.",
        f"// Source: {relative.as_posix()}",
        f"// Certificate SHA-256: {scheme.certificate_sha256}",
        "// Licence: that of the certificate (see rdna3_fastmm/certificates/NOTICE.md).",
        f"#ifndef {_guard(scheme)}",
        f"#define {_guard(scheme)}",
        "",
        "namespace fastmm {",
        "",
        f"struct {_struct_name(scheme)} {{",
        f"  static constexpr int kSize = {scheme.size};",
        f"  static constexpr int kRank = {scheme.rank};",
        f"  static constexpr int kSchemeId = {scheme.scheme_id};",
        f'  static constexpr const char* kCertificateSha256 = "{scheme.certificate_sha256}";',
        "",
        _indent(emit_program(
            "left", scheme.left,
            "A side: input i = block (i / kSize, i % kSize) of x; output r = plane r of A'.",
        )),
        "",
        _indent(emit_program(
            "right", scheme.right,
            "B side: input j = block (j / kSize, j % kSize) of B = W^T; output r = plane r of B'.",
        )),
        "",
        _indent(emit_program(
            "output", scheme.output,
            "Recombination: input r = product P[r]; output c = block (c / kSize, c % kSize) of C.",
        )),
        *([ "", _indent(emit_output_matrix(scheme.output))] if scheme.size == 8 else []),
        "};",
        "",
        "}  // namespace fastmm",
        "",
        f"#endif  // {_guard(scheme)}",
        "",
    ]
    return "\n".join(parts)


def _indent(text: str) -> str:
    return "\n".join(("  " + line) if line else line for line in text.splitlines())


def _struct_name(scheme: Scheme) -> str:
    # rank7_2x2x2 -> SchemeRank7
    return "Scheme" + scheme.name.split("_")[0].capitalize()


def header_filename(scheme: Scheme) -> str:
    return f"{scheme.name}.h"


def generate_all() -> dict[str, str]:
    result = {}
    for key in SCHEME_KEYS:
        scheme = load_scheme(key)
        result[header_filename(scheme)] = emit_scheme_header(scheme)
    return result


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("output_dir", nargs="?", type=Path, default=GENERATED_DIR)
    args = parser.parse_args(argv)
    args.output_dir.mkdir(parents=True, exist_ok=True)
    for name, text in generate_all().items():
        (args.output_dir / name).write_text(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
