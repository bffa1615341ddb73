"""Straight-line linear programs: the one form every scheme side is lowered to.

A scheme side (the A-side transform, the B-side transform, the output
recombination) is a linear map evaluated by a straight-line program. Signals
``0 .. input_count-1`` are the inputs; every step defines one new signal as an
expression tree over earlier signals; ``outputs[k]`` names the signal that
holds output ``k``.

Expression nodes are ``Sig``, ``Add``, ``Sub``, ``Neg`` and ``Scale``. The tree
fixes the floating-point evaluation order: the left operand is evaluated
first and every node rounds once. That is the order the reference's generated
kernels use in fp32 (reduced circuits: ``generate_triton_scheme.py:70-80``,
left-to-right term sums; SLP files: ``slp.py:134-193``, the parsed tree), so a
program evaluated in fp32 here, in the numpy oracle and in the generated HIP
gives identical bits.
"""

from __future__ import annotations

from dataclasses import dataclass
from fractions import Fraction
from typing import Callable, Sequence, TypeVar, Union

T = TypeVar("T")


@dataclass(frozen=True)
class Sig:
    index: int


@dataclass(frozen=True)
class Add:
    left: "Expr"
    right: "Expr"


@dataclass(frozen=True)
class Sub:
    left: "Expr"
    right: "Expr"


@dataclass(frozen=True)
class Neg:
    operand: "Expr"


@dataclass(frozen=True)
class Scale:
    operand: "Expr"
    factor: Fraction


Expr = Union[Sig, Add, Sub, Neg, Scale]


@dataclass(frozen=True)
class Step:
    """One assignment ``signal := expr``; ``name`` is the source label."""

    signal: int
    expr: Expr
    name: str


def expression_signals(expr: Expr) -> tuple[int, ...]:
    """Signals read by ``expr`` in first-use order, without repeats."""
    seen: dict[int, None] = {}

    def walk(node: Expr) -> None:
        if isinstance(node, Sig):
            seen.setdefault(node.index, None)
        elif isinstance(node, (Add, Sub)):
            walk(node.left)
            walk(node.right)
        else:
            walk(node.operand)

    walk(expr)
    return tuple(seen)


def count_operations(expr: Expr) -> tuple[int, int]:
    """(additions, scalings) in ``expr``; a scaling by +-1 is free."""
    if isinstance(expr, Sig):
        return 0, 0
    if isinstance(expr, (Add, Sub)):
        la, ls = count_operations(expr.left)
        ra, rs = count_operations(expr.right)
        return la + ra + 1, ls + rs
    if isinstance(expr, Neg):
        return count_operations(expr.operand)
    additions, scalings = count_operations(expr.operand)
    return additions, scalings + int(abs(expr.factor) != 1)


def evaluate_expression(
    expr: Expr,
    values: Sequence[T] | dict[int, T],
    scale: Callable[[T, Fraction], T],
) -> T:
    """Evaluate one tree, left operand first (the rounding order)."""
    if isinstance(expr, Sig):
        return values[expr.index]
    if isinstance(expr, Add):
        left = evaluate_expression(expr.left, values, scale)
        return left + evaluate_expression(expr.right, values, scale)  # type: ignore[operator]
    if isinstance(expr, Sub):
        left = evaluate_expression(expr.left, values, scale)
        return left - evaluate_expression(expr.right, values, scale)  # type: ignore[operator]
    if isinstance(expr, Neg):
        return -evaluate_expression(expr.operand, values, scale)  # type: ignore[operator]
    return scale(evaluate_expression(expr.operand, values, scale), expr.factor)


@dataclass(frozen=True)
class LinearProgram:
    input_count: int
    steps: tuple[Step, ...]
    outputs: tuple[int, ...]

    def __post_init__(self) -> None:
        if self.input_count < 1 or not self.outputs:
            raise ValueError("a program needs inputs and outputs")
        for offset, step in enumerate(self.steps):
            if step.signal != self.input_count + offset:
                raise ValueError("program signals must be numbered in step order")
            for index in expression_signals(step.expr):
                if not 0 <= index < step.signal:
                    raise ValueError(f"step {step.name} reads unavailable signal {index}")
        signal_count = self.input_count + len(self.steps)
        if any(not 0 <= signal < signal_count for signal in self.outputs):
            raise ValueError("program output names an unknown signal")

    @property
    def signal_count(self) -> int:
        return self.input_count + len(self.steps)

    @property
    def output_count(self) -> int:
        return len(self.outputs)

    @property
    def additions(self) -> int:
        return sum(count_operations(step.expr)[0] for step in self.steps)

    @property
    def scalings(self) -> int:
        return sum(count_operations(step.expr)[1] for step in self.steps)

    @property
    def operations(self) -> int:
        return self.additions + self.scalings

    @property
    def assignments(self) -> tuple[Step, ...]:
        return self.steps

    @property
    def output_signals(self) -> tuple[int, ...]:
        return self.outputs

    @property
    def output_coefficients(self) -> tuple[tuple[Fraction, ...], ...]:
        return self.coefficients()

    def evaluate(
        self, inputs: Sequence[T], scale: Callable[[T, Fraction], T]
    ) -> list[T]:
        if len(inputs) != self.input_count:
            raise ValueError("wrong number of program inputs")
        values: list[T] = list(inputs)
        for step in self.steps:
            values.append(evaluate_expression(step.expr, values, scale))
        return [values[signal] for signal in self.outputs]

    def signal_coefficients(self) -> list[tuple[Fraction, ...]]:
        """Exact coefficient vector of every signal over the inputs."""
        vectors = [
            _Vector(tuple(Fraction(int(row == column)) for column in range(self.input_count)))
            for row in range(self.input_count)
        ]
        for step in self.steps:
            vectors.append(
                evaluate_expression(step.expr, vectors, lambda v, f: v.scaled(f))
            )
        return [vector.values for vector in vectors]

    def coefficients(self) -> tuple[tuple[Fraction, ...], ...]:
        """Exact ``output_count x input_count`` matrix of the program."""
        signals = self.signal_coefficients()
        return tuple(signals[signal] for signal in self.outputs)

    def with_outputs(self, outputs: Sequence[int]) -> "LinearProgram":
        return LinearProgram(self.input_count, self.steps, tuple(outputs))


@dataclass(frozen=True)
class _Vector:
    """Exact linear form used to expand a program symbolically."""

    values: tuple[Fraction, ...]

    def __add__(self, other: "_Vector") -> "_Vector":
        return _Vector(tuple(a + b for a, b in zip(self.values, other.values)))

    def __sub__(self, other: "_Vector") -> "_Vector":
        return _Vector(tuple(a - b for a, b in zip(self.values, other.values)))

    def __neg__(self) -> "_Vector":
        return _Vector(tuple(-a for a in self.values))

    def scaled(self, factor: Fraction) -> "_Vector":
        return _Vector(tuple(factor * a for a in self.values))


def brent_mismatches(
    dimensions: tuple[int, int, int],
    left: Sequence[Sequence[Fraction]],
    right: Sequence[Sequence[Fraction]],
    output: Sequence[Sequence[Fraction]],
) -> tuple[int, int]:
    """Check the Brent equations of a bilinear scheme exactly.

    For ``dimensions = (m, p, q)``: ``left[r]`` is over A blocks (row-major
    ``i*p + k``), ``right[r]`` over B blocks (``k*q + j``) and ``output[c][r]``
    over C blocks (``i*q + j``). The scheme multiplies an ``m x p`` block
    matrix by a ``p x q`` one exactly iff
    ``sum_r left[r][a] * right[r][b] * output[c][r]`` is 1 when
    ``a=(i,k), b=(k,j), c=(i,j)`` and 0 otherwise. Returns
    ``(mismatched entries, nonzero entries)``.
    """
    first, shared, second = dimensions
    rank = len(left)
    entries: dict[tuple[int, int, int], Fraction] = {}
    for term in range(rank):
        a_terms = [(a, value) for a, value in enumerate(left[term]) if value]
        b_terms = [(b, value) for b, value in enumerate(right[term]) if value]
        c_terms = [(c, row[term]) for c, row in enumerate(output) if row[term]]
        for a, a_value in a_terms:
            for b, b_value in b_terms:
                product = a_value * b_value
                for c, c_value in c_terms:
                    key = (a, b, c)
                    entries[key] = entries.get(key, Fraction(0)) + product * c_value
    nonzero = {key: value for key, value in entries.items() if value}
    expected = {
        (i * shared + k, k * second + j, i * second + j)
        for i in range(first)
        for k in range(shared)
        for j in range(second)
    }
    mismatches = sum(1 for key, value in nonzero.items() if key not in expected or value != 1)
    mismatches += sum(1 for key in expected if key not in nonzero)
    return mismatches, len(nonzero)
