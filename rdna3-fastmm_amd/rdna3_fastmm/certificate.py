"""Reduced-circuit certificates (rank-7 and rank-49 schemes).

A reduced certificate is a JSON object with dimensions ``n = [m, p, q]``, the
rank ``m`` and, for each side (``u`` = A, ``v`` = B, ``w`` = output), a list
of fresh gates and a list of outputs. Every gate or output is a signed sum of
earlier signals written as ``[{"index": i, "value": +-1}, ...]``. The format,
field names and the column-major numbering of the ``w`` outputs are the
upstream format the reference consumes (``src/rdna3_fastmm/certificate.py``);
the checks below are this package's own, lowered onto ``LinearProgram``.

Public names mirror the reference: ``load_reduced_scheme`` (certificate.py:
258-266), ``verify_reduced_scheme`` (201-255), ``load_expanded_scheme``
(269-292), ``expand_linear_map`` (58-78) and ``ExpandedScheme`` (49-55).
"""

from __future__ import annotations

from dataclasses import dataclass
from fractions import Fraction
import json
from pathlib import Path
from typing import Any, Mapping, Sequence

from .program import Add, Expr, LinearProgram, Neg, Sig, Step, Sub, brent_mismatches

LinearTerm = Mapping[str, int]
ReducedSchemeData = dict[str, Any]

_REQUIRED_FIELDS = ("n", "m", "u_fresh", "v_fresh", "w_fresh", "u", "v", "w")


@dataclass(frozen=True)
class VerificationSummary:
    dimensions: tuple[int, int, int]
    rank: int
    additions: int
    side_additions: tuple[int, int, int]
    naive_additions: int
    tensor_entries: int


@dataclass(frozen=True)
class ExpandedScheme:
    """Integer coefficient matrices of a verified scheme.

    ``left_coefficients[r]`` is over row-major A blocks, ``right_coefficients[r]``
    over row-major B blocks and ``output_coefficients[c]`` (one row per
    row-major C block) over the ``rank`` products.
    """

    dimensions: tuple[int, int, int]
    rank: int
    left_coefficients: tuple[tuple[int, ...], ...]
    right_coefficients: tuple[tuple[int, ...], ...]
    output_coefficients: tuple[tuple[int, ...], ...]


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _term_expression(name: str, position: int, terms: object, available: int) -> Expr:
    """Lower one signed sum to a left-to-right expression tree."""
    if not isinstance(terms, list):
        raise ValueError(f"{name} expression {position} must be a list")
    if not terms:
        raise ValueError(f"{name} expression {position} is empty")
    expr: Expr | None = None
    for term in terms:
        if not isinstance(term, dict):
            raise ValueError(f"{name} expression {position} has invalid term")
        index, value = term.get("index"), term.get("value")
        if not _is_int(index):
            raise ValueError(f"{name} expression {position} has invalid index")
        if not 0 <= index < available:
            raise ValueError(
                f"{name} expression {position} references unavailable signal {index}"
            )
        if not _is_int(value) or value not in (-1, 1):
            raise ValueError(f"{name} expression {position} has non-signed value")
        signal = Sig(index)
        if expr is None:
            expr = signal if value == 1 else Neg(signal)
        else:
            expr = Add(expr, signal) if value == 1 else Sub(expr, signal)
    assert expr is not None
    return expr


def circuit_program(
    name: str, input_count: int, gates: object, outputs: object
) -> LinearProgram:
    """Lower ``gates`` + ``outputs`` of one side to a program.

    Gates may read the inputs and earlier gates; outputs may read the inputs
    and every gate (the reference's ``validate_expressions``,
    certificate.py:96-128). Each output becomes one step, in order.
    """
    if not isinstance(gates, list) or not isinstance(outputs, list):
        raise ValueError(f"{name} expressions must be a list")
    steps: list[Step] = []
    for position, terms in enumerate(gates):
        available = input_count + position
        steps.append(
            Step(available, _term_expression(name, position, terms, available), f"g{position}")
        )
    gate_signals = input_count + len(gates)
    output_signals: list[int] = []
    for offset, terms in enumerate(outputs):
        position = len(gates) + offset
        signal = gate_signals + offset
        steps.append(
            Step(signal, _term_expression(name, position, terms, gate_signals), f"o{offset}")
        )
        output_signals.append(signal)
    if not output_signals:
        raise ValueError(f"{name} circuit has no outputs")
    return LinearProgram(input_count, tuple(steps), tuple(output_signals))


def _header(source: Mapping[str, Any]) -> tuple[int, int, int, int]:
    dimensions = source["n"]
    if (
        not isinstance(dimensions, list)
        or len(dimensions) != 3
        or any(not _is_int(d) or d < 1 for d in dimensions)
    ):
        raise ValueError("scheme dimensions must be three positive integers")
    rank = source["m"]
    if not _is_int(rank) or rank < 1:
        raise ValueError("scheme rank must be a positive integer")
    if source.get("z2") is not False:
        raise ValueError("certificate must explicitly define an integer, non-Z2 circuit")
    return dimensions[0], dimensions[1], dimensions[2], rank


def _integer_rows(rows: Sequence[Sequence[Fraction]]) -> tuple[tuple[int, ...], ...]:
    result = []
    for row in rows:
        if any(value.denominator != 1 for value in row):
            raise ValueError("reduced circuit expanded to non-integer coefficients")
        result.append(tuple(int(value) for value in row))
    return tuple(result)


@dataclass(frozen=True)
class ReducedCircuit:
    """A verified reduced certificate lowered to three programs.

    ``output`` has its outputs renumbered to row-major C blocks
    (``row * q + column``); the file numbers them column-major
    (``column * m + row``, reference certificate.py:186-198, 281-285).
    """

    dimensions: tuple[int, int, int]
    rank: int
    left: LinearProgram
    right: LinearProgram
    output: LinearProgram
    summary: VerificationSummary


def lower_reduced_scheme(source: ReducedSchemeData) -> ReducedCircuit:
    first, shared, second, rank = _header(source)
    left = circuit_program("u", first * shared, source["u_fresh"], source["u"])
    right = circuit_program("v", shared * second, source["v_fresh"], source["v"])
    output_file_order = circuit_program("w", rank, source["w_fresh"], source["w"])
    if left.output_count != rank or right.output_count != rank:
        raise ValueError("input factor row count does not match rank")
    if output_file_order.output_count != first * second:
        raise ValueError("output circuit row count does not match output size")
    output = output_file_order.with_outputs(
        [
            output_file_order.outputs[column * first + row]
            for row in range(first)
            for column in range(second)
        ]
    )
    u = left.coefficients()
    v = right.coefficients()
    w = output.coefficients()
    mismatches, entries = brent_mismatches((first, shared, second), u, v, w)
    if mismatches:
        raise ValueError(f"Brent tensor has {mismatches} mismatched entries")
    side_costs = (left.additions, right.additions, output.additions)
    nonzero = sum(1 for rows in (u, v, w) for row in rows for value in row if value)
    naive = nonzero - 2 * rank - first * second
    declared = source.get("complexity")
    if declared is not None:
        if not isinstance(declared, dict):
            raise ValueError("declared complexity must be an object")
        if declared.get("reduced") != sum(side_costs):
            raise ValueError("declared reduced complexity is incorrect")
        if declared.get("naive") != naive:
            raise ValueError("declared naive complexity is incorrect")
    summary = VerificationSummary(
        dimensions=(first, shared, second),
        rank=rank,
        additions=sum(side_costs),
        side_additions=side_costs,
        naive_additions=naive,
        tensor_entries=entries,
    )
    return ReducedCircuit((first, shared, second), rank, left, right, output, summary)


def verify_reduced_scheme(source: ReducedSchemeData) -> VerificationSummary:
    """Check a reduced certificate exactly and recount its additions."""
    return lower_reduced_scheme(source).summary


def load_reduced_scheme(path: Path) -> ReducedSchemeData:
    raw = json.loads(Path(path).read_text())
    if not isinstance(raw, dict):
        raise ValueError("certificate must be a JSON object")
    if any(field not in raw for field in _REQUIRED_FIELDS):
        raise ValueError("input is not a reduced scheme")
    return raw


def expand_linear_map(
    input_count: int, gates: list[list[LinearTerm]], outputs: list[list[LinearTerm]]
) -> list[list[int]]:
    """Integer matrix of one side, outputs in file order."""
    program = circuit_program("expression", input_count, gates, outputs)
    return [list(row) for row in _integer_rows(program.coefficients())]


def load_expanded_scheme(path: Path) -> ExpandedScheme:
    circuit = lower_reduced_scheme(load_reduced_scheme(path))
    return ExpandedScheme(
        dimensions=circuit.dimensions,
        rank=circuit.rank,
        left_coefficients=_integer_rows(circuit.left.coefficients()),
        right_coefficients=_integer_rows(circuit.right.coefficients()),
        output_coefficients=_integer_rows(circuit.output.coefficients()),
    )
