"""Corpus loader and runner (reference tests of benchmarks/corpus.py and run_corpus.py).

The loader must accept the shipped corpus and reject the same malformed files
the reference's loader rejects; the runner's arithmetic (quartiles, break-even,
win selection) is checked on hand-computed values. One GPU test runs a small
case through every plan.
"""

from __future__ import annotations

import copy
import json

import pytest

from rdna3_fastmm import corpus as C


def _raw() -> dict:
    return json.loads(C.DEFAULT_CORPUS_PATH.read_text())


def _write(tmp_path, document) -> object:
    path = tmp_path / "corpus.json"
    path.write_text(json.dumps(document))
    return path


def test_shipped_corpus_lists_the_reference_shapes() -> None:
    corpus = C.load_corpus()
    assert corpus.schema_version == 1 and corpus.operator == "torch.nn.functional.linear"
    assert len(corpus.cases) == 15
    shapes = {case.shape for case in corpus.cases}
    # the north-star workloads are in the corpus
    assert {(4096, 4096, 12288), (8214, 12288, 4608), (19968, 4096, 16384)} <= shapes
    case = corpus.case("ltx-2.3-blueprint-4992-mlp-up")
    assert (case.rows, case.inner, case.columns, case.bias, case.priority) == (4992, 4096, 16384, True, 1)
    assert all(c.input_output_dtype == "bfloat16" and c.weight_layout == "out_in" for c in corpus.cases)
    with pytest.raises(KeyError):
        corpus.case("missing")


@pytest.mark.parametrize(
    ("mutate", "message"),
    (
        (lambda d: d.update(schema_version=2), "unsupported corpus schema version 2"),
        (lambda d: d.update(operator="torch.mm"), "unsupported corpus operator"),
        (lambda d: d.update(cases=[]), "cases must be a non-empty array"),
        (lambda d: d.update(extra=1), "corpus has invalid keys"),
        (lambda d: d["cases"][0].pop("bias"), r"cases\[0\] has invalid keys; missing=\['bias'\]"),
        (lambda d: d["cases"][0].update(shape=[1, 2]), "must contain three dimensions"),
        (lambda d: d["cases"][0].update(shape=[1, 0, 2]), "dimensions must be positive"),
        (lambda d: d["cases"][0].update(shape=[1, True, 2]), "must be an integer"),
        (lambda d: d["cases"][0].update(priority=4), "priority must be 1, 2, or 3"),
        (lambda d: d["cases"][0].update(bias=1), "bias must be a boolean"),
        (lambda d: d["cases"][0].update(compute_dtype="float32"), "compute_dtype must be one of"),
        (lambda d: d["cases"][0].update(weight_layout="in_out"), "weight_layout must be one of"),
        (lambda d: d["cases"][0]["evidence"].update(kind="guess"), "evidence.kind must be one of"),
        (lambda d: d["cases"][0]["evidence"].update(references=[]), "references must not be empty"),
        (lambda d: d["cases"][0].update(id=""), "id must be a non-empty string"),
        (lambda d: d["cases"].append(copy.deepcopy(d["cases"][0])), "case ids must be unique"),
    ),
)
def test_loader_rejects_malformed_corpus(tmp_path, mutate, message) -> None:
    document = _raw()
    mutate(document)
    with pytest.raises(ValueError, match=message):
        C.load_corpus(_write(tmp_path, document))


def test_quartiles_interpolate_between_order_statistics() -> None:
    values = [4.0, 1.0, 3.0, 2.0]
    assert C.quartile(values, 2) == pytest.approx(2.5)
    assert C.quartile(values, 1) == pytest.approx(1.75)
    assert C.quartile(values, 3) == pytest.approx(3.25)
    t = C.timing([5.0, 1.0, 3.0])
    assert (t.median_ms, t.first_quartile_ms, t.third_quartile_ms) == (3.0, 2.0, 4.0)


def test_break_even_reuses() -> None:
    assert C.break_even_reuses(1.0, 1.0, 0.75) == 4
    assert C.break_even_reuses(1.1, 1.0, 0.75) == 5
    assert C.break_even_reuses(1.0, 0.8, 0.8) is None
    assert C.break_even_reuses(1.0, 0.7, 0.8) is None


def _report(case_id, shape, bias, dynamic, prepacked, ratio) -> dict:
    timing = {"median_ms": 1.0, "first_quartile_ms": 1.0, "third_quartile_ms": 1.0, "raw_ms": [1.0]}
    return {
        "case": {"id": case_id, "shape": list(shape), "bias": bias},
        "schemes": {
            "rank7": {
                "timings": {name: timing for name in ("native_linear", "native_into", "dynamic", "prepacked")},
                "dynamic": {"speedup_vs_native": dynamic, "error_ratio": ratio},
                "prepacked": {"speedup_vs_native": prepacked, "error_ratio": ratio},
            },
            "rank48": {"skipped": "no pair"},
        },
    }


def test_wins_need_speed_and_the_error_bound() -> None:
    reports = [
        _report("a", (8214, 12288, 4608), True, 0.9, 1.05, 1.08),
        _report("b", (4096, 4096, 12288), False, 1.1, 1.2, 1.5),  # too inaccurate
        _report("c", (720, 4096, 16384), True, 0.5, 0.8, 1.0),
    ]
    wins = C.winning_families(reports)
    assert wins == [{"scheme": "rank7", "prepacked": True, "rows": 8214, "inner": 12288, "columns": 4608,
                     "bias": True, "speedup": 1.05, "case": "a"}]
    assert C.winning_families(reports, minimum_speedup=1.1) == []
    table = C.summary_table(reports)
    assert table.count("\n") == 2 + 3 - 1 and "8214×12288×4608" in table


def test_cli_lists_cases_and_validates_arguments(capsys) -> None:
    assert C.main(["--list"]) == 0
    lines = capsys.readouterr().out.strip().splitlines()
    assert len(lines) == 15 and lines[0].startswith("hidream-o1-4mp-mlp-up\tpriority=1\t4096x4096x12288")
    with pytest.raises(SystemExit):
        C.main(["--all"])  # no output directory
    with pytest.raises(SystemExit):
        C.main(["--case", "x", "--case", "x", "--output-directory", "o"])
    with pytest.raises(SystemExit):
        C.main(["--all", "--output-directory", "o", "--rounds", "2"])


@pytest.mark.gpu
def test_runner_measures_a_small_case(tmp_path) -> None:
    document = _raw()
    case = document["cases"][0]
    case.update(id="small", shape=[200, 512, 520], bias=True)
    document["cases"] = [case]
    path = _write(tmp_path, document)
    print("\n[case] corpus runner, 200x512x520 with bias, rank7/48/49", flush=True)
    assert C.main(["--corpus", str(path), "--all", "--output-directory", str(tmp_path / "out"),
                   "--warmups", "1", "--rounds", "3"]) == 0
    report = json.loads((tmp_path / "out" / "small.json").read_text())
    assert set(report["schemes"]) == {"rank7", "rank48", "rank49"}
    for result in report["schemes"].values():
        assert len(result["timings"]["prepacked"]["raw_ms"]) == 3
        for mode in ("dynamic", "prepacked"):
            assert result[mode]["error"]["nonfinite_count"] == 0
            assert result[mode]["error_ratio"] <= 2.0


def test_row_intervals_are_maximal_winning_runs() -> None:
    points = [(480, 0.9, 1.08), (864, 1.1, 1.08), (1248, 1.2, 1.08), (1632, 0.99, 1.08),
              (2016, 1.3, 1.08), (2400, 1.3, 1.5), (2784, 1.04, 1.08)]
    assert C.row_intervals(points, 1.0) == [(864, 1248), (2016, 2016), (2784, 2784)]
    assert C.row_intervals(list(reversed(points)), 1.05) == [(864, 1248), (2016, 2016)]
    assert C.row_intervals([], 1.0) == []


def test_sweep_families_group_by_scheme_mode_and_pair() -> None:
    reports = [_report(f"s{rows}", (rows, 12288, 4608), False, d, p, 1.08)
               for rows, d, p in ((480, 0.9, 1.1), (864, 1.05, 1.2), (1248, 0.8, 1.06))]
    families = C.sweep_families(reports, 1.0)
    assert families == [
        {"scheme": "rank7", "prepacked": False, "minimum_rows": 864, "maximum_rows": 864, "inner": 12288,
         "columns": 4608, "bias": False, "points": 1, "runs": 1, "minimum_speedup": 1.05},
        {"scheme": "rank7", "prepacked": True, "minimum_rows": 480, "maximum_rows": 1248, "inner": 12288,
         "columns": 4608, "bias": False, "points": 3, "runs": 1, "minimum_speedup": 1.06},
    ]
    # a second run that is slower at 864 rows splits the prepacked family and drops the dynamic one
    second = [_report(f"t{rows}", (rows, 12288, 4608), False, d, p, 1.08)
              for rows, d, p in ((480, 0.9, 1.2), (864, 0.99, 0.98), (1248, 0.8, 1.2))]
    combined = C.sweep_families(reports + second, 1.0)
    assert [(f["prepacked"], f["minimum_rows"], f["maximum_rows"], f["runs"], f["minimum_speedup"])
            for f in combined] == [(True, 480, 480, 2, 1.1), (True, 1248, 1248, 2, 1.06)]
    document = C.dispatch_document(reports + second, 1.0, "test")
    assert document["families"] == combined and document["minimum_speedup"] == 1.0
    # with two runs required, a row measured once never wins: 1248 rows of the second
    # run missing leaves only 480 rows as a prepacked family
    partial = C.sweep_families(reports + second[:2], 1.0, minimum_runs=2)
    assert [(f["prepacked"], f["minimum_rows"], f["maximum_rows"], f["runs"]) for f in partial] == [(True, 480, 480, 2)]
    assert C.dispatch_document(reports + second[:2], 1.0, "test", minimum_runs=2)["families"] == partial
    case = C.sweep_case(12288, 4608, True, 480)
    assert case.shape == (480, 12288, 4608) and case.bias and case.compute_dtype == "float16"


def test_llm_corpus_loads() -> None:
    corpus = C.load_corpus(C.DEFAULT_CORPUS_PATH.parent / "llm-mlp-2025.json")
    assert len(corpus.cases) == 24 and all(not case.bias for case in corpus.cases)
    down = corpus.case("llama-3-8b-4096-down")
    assert down.shape == (4096, 14336, 4096) and down.projection == "MLP down projection"
