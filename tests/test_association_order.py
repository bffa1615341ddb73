"""fp32 summation order of every scheme program against the reference's generated
kernels (CPU only).

``golden/association_vectors.npz`` holds fp32 input/output vectors of the
reference's generated Triton transforms, written by
``golden/make_association_vectors.py`` from the text of
``src/rdna3_fastmm/generated/rank{7,48,49,343}_*.py``. The inputs span 21
binades, so evaluating any sum in another order rounds differently on some
sample. This test checks two things against those vectors, bit for bit: the
oracle's programs, which the GPU parity tests compare the HIP kernels with, and
the HIP programs this package emits (``csrc/generated/*.h``), interpreted here
in fp32 in the order their parentheses fix (the library is built with
``-ffp-contract=off`` and no fast-math). A planted regrouping of one oracle sum
must fail.
"""

from __future__ import annotations

from pathlib import Path
import re

import numpy as np
import pytest

from oracle import fastmm_oracle as O
from rdna3_fastmm import _build, hipgen
from rdna3_fastmm.schemes import load_scheme

VECTORS = np.load(Path(__file__).parent / "golden" / "association_vectors.npz")
# fixture kernel -> the program that computes it (the weight path runs the right
# program on W^T blocks; the bias path adds the bias after the whole output sum)
PROGRAMS = {"left": "left", "right": "right", "weight": "right", "output": "output", "output_bias": "output"}
CASES = sorted({tuple(name.split(".")[:2]) for name in VECTORS.files})


def _bits(values) -> np.ndarray:
    return np.stack([np.asarray(v, dtype=np.float32) for v in values]).view(np.uint32)


def _oracle_outputs(program: O.OracleProgram, key: str, kernel: str) -> list:
    inputs = VECTORS[f"{key}.{kernel}.inputs"]
    outputs = O.evaluate_program(program, list(inputs))
    if kernel == "output_bias":
        s = O.load_oracle_scheme(key).size
        bias = VECTORS[f"{key}.{kernel}.bias"]
        outputs = [np.float32(1) * value + bias[i % s] for i, value in enumerate(outputs)]
    return outputs


def test_every_reference_transform_is_covered() -> None:
    assert set(CASES) == {
        (key, kernel)
        for key in ("rank7", "rank48", "rank49")
        for kernel in ("left", "right", "weight", "output", "output_bias")
    } | {("rank343", "left"), ("rank343", "right")}


@pytest.mark.parametrize("key, kernel", CASES, ids=[f"{k}-{n}" for k, n in CASES])
def test_oracle_sums_in_the_reference_order(key: str, kernel: str) -> None:
    program = getattr(O.load_oracle_scheme(key), PROGRAMS[kernel])
    got = _bits(_oracle_outputs(program, key, kernel))
    assert np.array_equal(got, VECTORS[f"{key}.{kernel}.outputs"].view(np.uint32))


def _run_emitted_f32(body: str, inputs: np.ndarray) -> dict[int, np.ndarray]:
    """Interpret one emitted C++ program in fp32, one rounding per operation."""
    values: dict[str, np.ndarray] = {}
    outputs: dict[int, np.ndarray] = {}
    for line in body.splitlines():
        line = line.strip()
        if m := re.fullmatch(r"const V (s\d+) = load\((\d+)\);", line):
            values[m.group(1)] = inputs[int(m.group(2))]
        elif m := re.fullmatch(r"const V (s\d+) = (.*);  // \w+", line):
            expression = re.sub(r"(\d+\.\d+(?:e-?\d+)?)f", r"f32(\1)", m.group(2))
            values[m.group(1)] = np.asarray(eval(expression, {"f32": np.float32}, dict(values)), dtype=np.float32)
        elif m := re.fullmatch(r"store\((\d+), (s\d+)\);", line):
            outputs[int(m.group(1))] = values[m.group(2)]
    return outputs


@pytest.mark.parametrize("key, kernel", CASES, ids=[f"{k}-{n}" for k, n in CASES])
def test_emitted_hip_programs_sum_in_the_reference_order(key: str, kernel: str) -> None:
    header = hipgen.emit_scheme_header(load_scheme(key))
    side = PROGRAMS[kernel]
    start = header.index(f"void {side}(")
    body = header[start:header.index("\n  }\n", start)]
    # the compiler keeps the emitted order: no reassociation, no contraction
    assert all("fast-math" not in f and "reassoc" not in f for f in _build.COMMON_FLAGS)
    assert "-ffp-contract=off" in _build.COMMON_FLAGS
    stored = _run_emitted_f32(body, VECTORS[f"{key}.{kernel}.inputs"])
    values = [stored[i] for i in range(len(stored))]
    if kernel == "output_bias":
        s = load_scheme(key).size
        bias = VECTORS[f"{key}.{kernel}.bias"]
        values = [v + bias[i % s] for i, v in enumerate(values)]
    assert np.array_equal(_bits(values), VECTORS[f"{key}.{kernel}.outputs"].view(np.uint32))


def _regroup_first_chain(program: O.OracleProgram) -> O.OracleProgram:
    """The program with its first three-term sum ``(a ± b) ± c`` evaluated as
    ``a ± (b ± c)``: the same value in exact arithmetic, another fp32 rounding."""
    inner_sign = {("add", "add"): "add", ("add", "sub"): "sub", ("sub", "add"): "sub", ("sub", "sub"): "add"}

    def regroup(node):
        if node[0] in ("add", "sub") and node[1][0] in ("add", "sub"):
            (outer, (inner, a, b), c) = node
            # (a + b) ± c = a + (b ± c); (a - b) + c = a - (b - c); (a - b) - c = a - (b + c)
            return (inner, a, (inner_sign[(inner, outer)], b, c))
        for position, child in enumerate(node[1:], start=1):
            if isinstance(child, tuple) and child[0] != "sig" and (changed := regroup(child)) is not None:
                return node[:position] + (changed,) + node[position + 1:]
        return None

    assignments = list(program.assignments)
    for i, (signal, node) in enumerate(assignments):
        if (changed := regroup(node)) is not None:
            assignments[i] = (signal, changed)
            return O.OracleProgram(program.input_count, assignments, list(program.outputs))
    raise AssertionError("no three-term sum in the program")


@pytest.mark.parametrize("key, kernel", [("rank7", "output_bias"), ("rank48", "left"), ("rank48", "weight"),
                                         ("rank49", "output"), ("rank343", "left")])
def test_a_regrouped_oracle_sum_is_caught(key: str, kernel: str) -> None:
    program = _regroup_first_chain(getattr(O.load_oracle_scheme(key), PROGRAMS[kernel]))
    got = _bits(_oracle_outputs(program, key, kernel))
    assert not np.array_equal(got, VECTORS[f"{key}.{kernel}.outputs"].view(np.uint32))
