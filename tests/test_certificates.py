"""Certificate loaders: the reference's own known answers and rejection cases.

Expected values are copied from the reference's tests (paths relative to the
reference repository): tests/test_slp.py:17-83,
tests/test_fastmm_certificate.py:10-44, tests/test_verify_reduced_scheme.py:9-64.
"""

from copy import deepcopy
import hashlib
import json
from pathlib import Path

import pytest

from rdna3_fastmm import ExpandedScheme, load_expanded_scheme
from rdna3_fastmm.certificate import (
    expand_linear_map,
    load_reduced_scheme,
    verify_reduced_scheme,
)
from rdna3_fastmm.schemes import CERTIFICATE_ROOT, SCHEME_KEYS, load_scheme
from rdna3_fastmm.slp import load_and_verify_slp_certificate, load_slp_program

RANK48 = CERTIFICATE_ROOT / "4x4x4_rank48_accurate" / "certificate.json"
RANK49 = CERTIFICATE_ROOT / "4x4x4_rank49_159add" / "certificate.json"
RANK7 = CERTIFICATE_ROOT / "2x2x2_rank7_15add" / "certificate.json"


def test_vendored_files_match_pinned_digests() -> None:
    lines = (CERTIFICATE_ROOT / "SHA256SUMS").read_text().split("\n")
    checked = 0
    for line in filter(None, lines):
        digest, name = line.split()
        assert hashlib.sha256((CERTIFICATE_ROOT / name).read_bytes()).hexdigest() == digest
        checked += 1
    assert checked == 11


@pytest.mark.parametrize(
    ("name", "sha256"),
    (
        ("left.slp", "af7719f288b346ae0dde8b8bf4a4a7bcf8d160ec8387c4a72d560a4bdb65f19b"),
        ("right.slp", "c09dda6d06633b9b438683819be49151c2ff24d26bca1097c8023ad534d390fa"),
        ("output.slp", "d441067f8e8d5d9c374ab2f290763ecc5f4738f989e1e3570d844d8207ed042f"),
    ),
)
def test_rank48_vendored_slp_matches_upstream(name: str, sha256: str) -> None:
    assert hashlib.sha256((RANK48.parent / name).read_bytes()).hexdigest() == sha256


def test_rank48_slp_certificate_is_exact() -> None:
    certificate, summary = load_and_verify_slp_certificate(RANK48)
    assert summary.dimensions == (4, 4, 4)
    assert summary.rank == 48
    assert summary.additions == (80, 68, 108)
    assert summary.scalings == (4, 8, 16)
    assert summary.operations == (84, 76, 124)
    assert summary.tensor_entries == 64
    assert summary.sha256 == "c7103a1165af22d4e1a417607e9618b0bbae1b69e0c48ed7fa2a5aba26a3bcb7"
    assert tuple(
        len(program.assignments) for program in (certificate.left, certificate.right, certificate.output)
    ) == (82, 60, 72)


def test_rank49_certificate_is_exact() -> None:
    summary = verify_reduced_scheme(load_reduced_scheme(RANK49))
    assert summary.dimensions == (4, 4, 4)
    assert summary.rank == 49
    assert summary.side_additions == (42, 42, 75)
    assert summary.additions == 159
    assert summary.tensor_entries == 64


def test_rank343_certificate_is_exact() -> None:
    """Counts stated in the certificate's README (8x8x8_rank343_1661add): 343
    multiplications, 1661 additions, directional costs 462, 456 and 743, every
    edge +-1; the upstream file's SHA-256."""
    path = RANK49.parent.parent / "8x8x8_rank343_1661add" / "certificate.json"
    assert hashlib.sha256(path.read_bytes()).hexdigest() == (
        "c7afccb09f8491e484af1696c25c809757c4af649ee7220e79f25d1c7afe3955"
    )
    source = load_reduced_scheme(path)
    summary = verify_reduced_scheme(source)
    assert summary.dimensions == (8, 8, 8)
    assert summary.rank == 343
    assert summary.side_additions == (462, 456, 743)
    assert summary.additions == 1661
    assert {term["value"] for key in ("u_fresh", "u", "v_fresh", "v", "w_fresh", "w")
            for expression in source[key] for term in expression} == {-1, 1}
    # the reference's MFMA recombination table: 343 rows of 64 coefficients in {-1, 0, 1}
    # (tests/test_generate_triton_scheme.py:262-281)
    expanded = load_expanded_scheme(path)
    assert len(expanded.output_coefficients) == 64
    assert all(len(row) == 343 for row in expanded.output_coefficients)
    assert {value for row in expanded.output_coefficients for value in row} == {-1, 0, 1}


def test_rank7_certificate_is_exact() -> None:
    summary = verify_reduced_scheme(load_reduced_scheme(RANK7))
    assert summary.side_additions == (4, 4, 7)
    assert summary.additions == 15
    assert summary.naive_additions == 24
    assert summary.tensor_entries == 8


def test_load_expanded_rank49_scheme() -> None:
    scheme = load_expanded_scheme(RANK49)
    assert isinstance(scheme, ExpandedScheme)
    assert scheme.dimensions == (4, 4, 4)
    assert scheme.rank == 49
    assert len(scheme.left_coefficients) == 49 and all(len(r) == 16 for r in scheme.left_coefficients)
    assert len(scheme.right_coefficients) == 49 and all(len(r) == 16 for r in scheme.right_coefficients)
    assert len(scheme.output_coefficients) == 16 and all(len(r) == 49 for r in scheme.output_coefficients)
    # rank 49 is the Kronecker square of the 2x2x2 rank-7 scheme, whose factor matrices
    # hold 14 nonzeros each: 14^2 = 196 per factor matrix here.
    for matrix in (scheme.left_coefficients, scheme.right_coefficients, scheme.output_coefficients):
        assert sum(1 for row in matrix for value in row if value) == 196
        assert {value for row in matrix for value in row} <= {-1, 0, 1}


def test_expanded_loader_rejects_invalid_brent_tensor(tmp_path: Path) -> None:
    source = json.loads(RANK49.read_text())
    source["u"][0][0]["value"] *= -1
    invalid = tmp_path / "invalid-certificate.json"
    invalid.write_text(json.dumps(source))
    with pytest.raises(ValueError, match="Brent tensor"):
        load_expanded_scheme(invalid)


def test_output_circuit_semantics_on_integer_products() -> None:
    """reference tests/test_generate_triton_scheme.py:47-98 for the W side.

    Evaluating the w circuit (column-major outputs) on the integer products
    -24..24 must equal the row-major output coefficient matrix times the
    products, after reordering column-major to row-major.
    """
    source = load_reduced_scheme(RANK49)
    products = list(range(-24, 25))
    signals = list(products)
    for expression in source["w_fresh"]:
        signals.append(sum(term["value"] * signals[term["index"]] for term in expression))
    circuit = [sum(term["value"] * signals[term["index"]] for term in expression) for expression in source["w"]]
    row_major = [circuit[column * 4 + row] for row in range(4) for column in range(4)]
    coefficients = load_expanded_scheme(RANK49).output_coefficients
    assert [sum(c[r] * products[r] for r in range(49)) for c in coefficients] == row_major
    columns = expand_linear_map(49, source["w_fresh"], source["w"])
    assert tuple(tuple(columns[col * 4 + row]) for row in range(4) for col in range(4)) == coefficients


def test_every_scheme_loads_with_pinned_digest() -> None:
    for key in SCHEME_KEYS:
        scheme = load_scheme(key)
        assert scheme.left.output_count == scheme.rank
        assert scheme.right.output_count == scheme.rank
        assert scheme.output.output_count == scheme.size**2


def test_slp_rejects_unavailable_signal(tmp_path: Path) -> None:
    path = tmp_path / "invalid.slp"
    path.write_text("o0:=i0+missing;\n")
    with pytest.raises(ValueError, match="unavailable signal missing"):
        load_slp_program(path, 1, 1)


def test_slp_rejects_nondyadic_scale(tmp_path: Path) -> None:
    path = tmp_path / "invalid.slp"
    path.write_text("o0:=i0/3;\n")
    with pytest.raises(ValueError, match="dyadic"):
        load_slp_program(path, 1, 1)


def test_slp_rejects_missing_output(tmp_path: Path) -> None:
    path = tmp_path / "invalid.slp"
    path.write_text("x0:=i0+i0;\n")
    with pytest.raises(ValueError, match=r"missing SLP outputs \[0\]"):
        load_slp_program(path, 1, 1)


def test_slp_rejects_duplicate_and_unary(tmp_path: Path) -> None:
    path = tmp_path / "invalid.slp"
    path.write_text("o0:=i0+i0;\no0:=i0;\n")
    with pytest.raises(ValueError, match="duplicate"):
        load_slp_program(path, 1, 1)
    path.write_text("o0:=-i0;\n")
    with pytest.raises(ValueError, match="unsupported"):
        load_slp_program(path, 1, 1)


def test_slp_counts_scalings_and_parses_precedence(tmp_path: Path) -> None:
    path = tmp_path / "ok.slp"
    path.write_text("x:=(i0-i1)/2;\no0:=x*4+i1-i0/4;\no1:=x*1;\n")
    program = load_slp_program(path, 2, 2)
    assert program.additions == 3
    assert program.scalings == 3  # /2, *4, /4; *1 is free
    from fractions import Fraction

    assert program.coefficients() == (
        (Fraction(2) - Fraction(1, 4), Fraction(-2) + 1),
        (Fraction(1, 2), Fraction(-1, 2)),
    )


def identity_panel_scheme() -> dict:
    return {
        "n": [1, 1, 2],
        "m": 2,
        "z2": False,
        "complexity": {"naive": 0, "reduced": 0},
        "u_fresh": [],
        "v_fresh": [],
        "w_fresh": [],
        "u": [[{"index": 0, "value": 1}], [{"index": 0, "value": 1}]],
        "v": [[{"index": 0, "value": 1}], [{"index": 1, "value": 1}]],
        "w": [[{"index": 0, "value": 1}], [{"index": 1, "value": 1}]],
    }


def test_verify_reduced_scheme_accepts_exact_tensor() -> None:
    summary = verify_reduced_scheme(identity_panel_scheme())
    assert summary.dimensions == (1, 1, 2)
    assert summary.rank == 2
    assert summary.additions == 0
    assert summary.tensor_entries == 2


@pytest.mark.parametrize(
    ("mutate", "message"),
    (
        (lambda s: s["w"].__setitem__(1, [{"index": 0, "value": 1}]), "Brent tensor"),
        (lambda s: s["complexity"].__setitem__("reduced", 1), "declared reduced"),
        (lambda s: s["u"].__setitem__(0, [{"index": 0, "value": 2}]), "non-signed"),
        (lambda s: s.__setitem__("z2", True), "non-Z2"),
        (lambda s: s.__setitem__("n", [0, 1, 2]), "positive integers"),
        (lambda s: s["u"].__setitem__(0, [{"index": 5, "value": 1}]), "unavailable signal"),
    ),
)
def test_verify_reduced_scheme_rejects(mutate, message: str) -> None:
    scheme = deepcopy(identity_panel_scheme())
    mutate(scheme)
    with pytest.raises(ValueError, match=message):
        verify_reduced_scheme(scheme)
