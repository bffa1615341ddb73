"""The generated HIP programs: checked-in files are current, and the emitted
expressions evaluate to the certificate's linear maps (reference
tests/test_generate_triton_scheme.py:169-248 keep the generated Triton in sync
the same way)."""

from fractions import Fraction
import re

from rdna3_fastmm import hipgen
from rdna3_fastmm.schemes import SCHEME_KEYS, load_scheme


def test_checked_in_headers_match_generator() -> None:
    for name, text in hipgen.generate_all().items():
        assert (hipgen.GENERATED_DIR / name).read_text() == text, name


def _run_emitted(function_text: str, inputs: list[Fraction]) -> dict[int, Fraction]:
    """Interpret one emitted C++ program with exact arithmetic."""
    values: dict[str, Fraction] = {}
    outputs: dict[int, Fraction] = {}
    for line in function_text.splitlines():
        line = line.strip()
        if m := re.fullmatch(r"const V (s\d+) = load\((\d+)\);", line):
            values[m.group(1)] = inputs[int(m.group(2))]
        elif m := re.fullmatch(r"const V (s\d+) = (.*);  // \w+", line):
            expression = re.sub(r"(\d+\.\d+(?:e-?\d+)?)f", r"Fraction('\1')", m.group(2))
            values[m.group(1)] = eval(expression, {"Fraction": Fraction}, dict(values))
        elif m := re.fullmatch(r"store\((\d+), (s\d+)\);", line):
            outputs[int(m.group(1))] = values[m.group(2)]
    return outputs


def test_emitted_programs_compute_the_certificate_maps() -> None:
    for key in SCHEME_KEYS:
        scheme = load_scheme(key)
        header = hipgen.emit_scheme_header(scheme)
        for side, program in (("left", scheme.left), ("right", scheme.right), ("output", scheme.output)):
            start = header.index(f"void {side}(")
            body = header[start:header.index("\n  }\n", start)]
            matrix = program.coefficients()
            for column in range(program.input_count):
                unit = [Fraction(int(i == column)) for i in range(program.input_count)]
                got = _run_emitted(body, unit)
                assert sorted(got) == list(range(program.output_count))
                assert [got[k] for k in range(program.output_count)] == [row[column] for row in matrix]


def test_dense_output_matrix_is_the_certificate_map() -> None:
    """The 8x8-block scheme's kOutputMatrix (the dense recombination's operand)
    equals the output program's exact coefficient matrix; only that scheme
    carries one."""
    for key in SCHEME_KEYS:
        scheme = load_scheme(key)
        header = hipgen.emit_scheme_header(scheme)
        if scheme.size != 8:
            assert "kOutputMatrix" not in header
            continue
        body = header[header.index("kOutputMatrix["):]
        body = body[body.index("= {") + 3:body.index("};")]
        rows = [[int(v) for v in row.split(",")] for row in re.findall(r"\{([-0-9,]+)\}", body)]
        expected = scheme.output.coefficients()
        assert len(rows) == scheme.size**2 == len(expected)
        assert rows == [[int(v) for v in row] for row in expected]
        assert all(v.denominator == 1 for row in expected for v in row)
