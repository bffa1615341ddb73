"""Dyadic-rational straight-line-program certificates (the rank-48 scheme).

An SLP file holds one assignment per line, ``target:=expression;``. Inputs are
``i0 .. i{n-1}``; a target ``o<k>`` is output ``k`` and, like every other
target, may be read by later lines. Expressions use ``+ - * /``, parentheses
and integer constants; a product or quotient must scale a linear expression
by a dyadic rational. The manifest (``certificate.json``) names the three
files, their operation counts and the dimension/rank.

The file format, the manifest fields, the operation counting (one addition
per binary ``+``/``-``, one scaling per ``*``/``/`` by a factor other than
+-1) and the composite SHA-256 are those of the reference
(``src/rdna3_fastmm/slp.py:105-283``), because they identify the same
certificate; the tokenizer/parser and the verification are this package's
own, lowered onto ``LinearProgram``.
"""

from __future__ import annotations

from dataclasses import dataclass
from fractions import Fraction
import hashlib
import json
from pathlib import Path
import re
from typing import Any

from .program import Add, Expr, LinearProgram, Scale, Sig, Step, Sub, brent_mismatches

_TARGET = re.compile(r"[A-Za-z][A-Za-z0-9_]*")
_TOKEN = re.compile(r"\s*(?:(?P<name>[A-Za-z][A-Za-z0-9_]*)|(?P<number>[0-9]+)|(?P<op>[-+*/()]))")

SlpProgram = LinearProgram


@dataclass(frozen=True)
class SlpCertificate:
    dimensions: tuple[int, int, int]
    rank: int
    left: LinearProgram
    right: LinearProgram
    output: LinearProgram
    sha256: str


@dataclass(frozen=True)
class SlpVerificationSummary:
    dimensions: tuple[int, int, int]
    rank: int
    additions: tuple[int, int, int]
    scalings: tuple[int, int, int]
    operations: tuple[int, int, int]
    tensor_entries: int
    sha256: str


def _is_dyadic(value: Fraction) -> bool:
    return value.denominator & (value.denominator - 1) == 0


class _Parser:
    """Recursive descent over ``expr := term (('+'|'-') term)*`` etc.

    A parsed value is either a constant (``Fraction``) or a linear
    expression (``Expr``); binary ``+``/``-`` need two linear operands,
    ``*`` exactly one constant, ``/`` a constant divisor.
    """

    def __init__(self, text: str, signals: dict[str, int]) -> None:
        self.tokens: list[tuple[str, str]] = []
        position = 0
        text = text.rstrip()
        while position < len(text):
            match = _TOKEN.match(text, position)
            if match is None or match.end() == position:
                raise SyntaxError("unexpected character")
            kind = match.lastgroup
            assert kind is not None
            self.tokens.append((kind, match.group(kind)))
            position = match.end()
        self.position = 0
        self.signals = signals

    def _peek(self) -> tuple[str, str] | None:
        return self.tokens[self.position] if self.position < len(self.tokens) else None

    def _take(self) -> tuple[str, str]:
        token = self._peek()
        if token is None:
            raise SyntaxError("unexpected end of expression")
        self.position += 1
        return token

    def parse(self) -> Expr | Fraction:
        value = self._sum()
        if self._peek() is not None:
            raise SyntaxError("trailing tokens")
        return value

    def _sum(self) -> Expr | Fraction:
        value = self._product()
        while (token := self._peek()) is not None and token[1] in "+-":
            self._take()
            right = self._product()
            if isinstance(value, Fraction) or isinstance(right, Fraction):
                raise ValueError("SLP additions require two linear expressions")
            value = Add(value, right) if token[1] == "+" else Sub(value, right)
        return value

    def _product(self) -> Expr | Fraction:
        value = self._atom()
        while (token := self._peek()) is not None and token[1] in "*/":
            self._take()
            right = self._atom()
            if token[1] == "*":
                if isinstance(value, Fraction) and not isinstance(right, Fraction):
                    factor, operand = value, right
                elif isinstance(right, Fraction) and not isinstance(value, Fraction):
                    factor, operand = right, value
                else:
                    raise ValueError("SLP multiplication requires one scalar")
            else:
                if isinstance(value, Fraction) or not isinstance(right, Fraction) or right == 0:
                    raise ValueError("SLP division requires a linear expression and scalar")
                factor, operand = 1 / right, value
            if not _is_dyadic(factor):
                raise ValueError("SLP scaling must be dyadic")
            value = Scale(operand, factor)
        return value

    def _atom(self) -> Expr | Fraction:
        kind, text = self._take()
        if kind == "number":
            return Fraction(int(text))
        if kind == "name":
            signal = self.signals.get(text)
            if signal is None:
                raise ValueError(f"SLP references unavailable signal {text}")
            return Sig(signal)
        if text == "(":
            value = self._sum()
            if self._take()[1] != ")":
                raise SyntaxError("unbalanced parenthesis")
            return value
        raise ValueError(f"unsupported SLP expression starting with {text!r}")


def parse_slp_text(text: str, input_count: int, output_count: int, origin: str) -> LinearProgram:
    if input_count < 1 or output_count < 1:
        raise ValueError("SLP input and output counts must be positive")
    signals = {f"i{index}": index for index in range(input_count)}
    steps: list[Step] = []
    outputs: dict[int, int] = {}
    for line_number, raw in enumerate(text.splitlines(), 1):
        line = raw.strip()
        if not line:
            continue
        where = f"{origin}:{line_number}"
        if not line.endswith(";") or line.count(":=") != 1:
            raise ValueError(f"{where}: invalid SLP assignment")
        target, source = line[:-1].split(":=", 1)
        if _TARGET.fullmatch(target) is None:
            raise ValueError(f"{where}: invalid SLP target")
        if target in signals:
            raise ValueError(f"{where}: duplicate SLP target {target}")
        try:
            value = _Parser(source, signals).parse()
        except SyntaxError as error:
            raise ValueError(f"{where}: invalid SLP expression") from error
        if isinstance(value, Fraction):
            raise ValueError(f"{where}: SLP result must be linear")
        signal = input_count + len(steps)
        steps.append(Step(signal, value, target))
        signals[target] = signal
        if target[0] == "o" and target[1:].isdigit():
            index = int(target[1:])
            if not 0 <= index < output_count:
                raise ValueError(f"{where}: output index {index} is out of range")
            outputs[index] = signal
    missing = sorted(set(range(output_count)) - set(outputs))
    if missing:
        raise ValueError(f"{origin}: missing SLP outputs {missing}")
    return LinearProgram(input_count, tuple(steps), tuple(outputs[k] for k in range(output_count)))


def load_slp_program(path: Path, input_count: int, output_count: int) -> LinearProgram:
    path = Path(path)
    return parse_slp_text(path.read_text(), input_count, output_count, str(path))


def _nonempty_string(source: dict[str, Any], name: str) -> str:
    value = source.get(name)
    if not isinstance(value, str) or not value:
        raise ValueError(f"certificate {name} must be a nonempty string")
    return value


def certificate_sha256(manifest: Path, programs: tuple[tuple[str, Path], ...]) -> str:
    """Composite digest: manifest bytes, then ``\\0 name \\0 bytes`` per program."""
    digest = hashlib.sha256(manifest.read_bytes())
    for name, path in programs:
        digest.update(b"\0" + name.encode() + b"\0")
        digest.update(path.read_bytes())
    return digest.hexdigest()


def load_slp_certificate(manifest_path: Path) -> SlpCertificate:
    manifest_path = Path(manifest_path)
    source = json.loads(manifest_path.read_text())
    if not isinstance(source, dict):
        raise ValueError("SLP certificate must be an object")
    if source.get("schema_version") != 1:
        raise ValueError("unsupported SLP certificate schema")
    dims, rank = source.get("n"), source.get("m")
    if (
        not isinstance(dims, list)
        or len(dims) != 3
        or any(not isinstance(d, int) or isinstance(d, bool) or d < 1 for d in dims)
        or not isinstance(rank, int)
        or isinstance(rank, bool)
        or rank < 1
    ):
        raise ValueError("invalid SLP dimensions or rank")
    if source.get("domain") != "dyadic-rational":
        raise ValueError("SLP certificate must use the dyadic-rational domain")
    if source.get("input_order") != "row-major":
        raise ValueError("SLP certificate inputs must be row-major")
    if source.get("output_order") != "row-major":
        raise ValueError("SLP certificate outputs must be row-major")
    programs, complexity = source.get("programs"), source.get("complexity")
    if not isinstance(programs, dict) or not isinstance(complexity, dict):
        raise ValueError("SLP certificate programs and complexity must be objects")
    directory = manifest_path.parent.resolve()
    paths: list[tuple[str, Path]] = []
    for name in ("u", "v", "w"):
        path = (directory / _nonempty_string(programs, name)).resolve()
        if path.parent != directory:
            raise ValueError("SLP program paths must stay inside the certificate")
        paths.append((name, path))
    first, shared, second = dims
    left = load_slp_program(paths[0][1], first * shared, rank)
    right = load_slp_program(paths[1][1], shared * second, rank)
    output = load_slp_program(paths[2][1], rank, first * second)
    for name, program in zip(("u", "v", "w"), (left, right, output)):
        declared = complexity.get(name)
        if isinstance(declared, bool) or declared != program.operations:
            raise ValueError(f"SLP {name} complexity does not match the manifest")
    return SlpCertificate(
        dimensions=(first, shared, second),
        rank=rank,
        left=left,
        right=right,
        output=output,
        sha256=certificate_sha256(manifest_path, tuple(paths)),
    )


def verify_slp_certificate(certificate: SlpCertificate) -> SlpVerificationSummary:
    mismatches, entries = brent_mismatches(
        certificate.dimensions,
        certificate.left.coefficients(),
        certificate.right.coefficients(),
        certificate.output.coefficients(),
    )
    if mismatches:
        raise ValueError(f"SLP Brent tensor has {mismatches} mismatches")
    sides = (certificate.left, certificate.right, certificate.output)
    return SlpVerificationSummary(
        dimensions=certificate.dimensions,
        rank=certificate.rank,
        additions=tuple(p.additions for p in sides),  # type: ignore[arg-type]
        scalings=tuple(p.scalings for p in sides),  # type: ignore[arg-type]
        operations=tuple(p.operations for p in sides),  # type: ignore[arg-type]
        tensor_entries=entries,
        sha256=certificate.sha256,
    )


def load_and_verify_slp_certificate(
    manifest_path: Path,
) -> tuple[SlpCertificate, SlpVerificationSummary]:
    certificate = load_slp_certificate(manifest_path)
    return certificate, verify_slp_certificate(certificate)
