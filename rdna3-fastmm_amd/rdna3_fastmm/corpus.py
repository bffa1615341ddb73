"""Real-model GEMM corpus: loader and MI355X runner.

The corpus format is the reference's (benchmarks/corpus.py:1-200, schema
version 1): a JSON object with ``schema_version``, ``name``, ``operator``
(``torch.nn.functional.linear``) and ``cases``, each case naming a model
projection's ``[rows, inner, columns]`` shape, dtypes, weight layout
(``out_in``: ``weight[N, K]``), bias and priority 1-3, plus its evidence. The
loader accepts exactly those keys and raises ``ValueError`` on anything else,
as the reference's does, so a corpus file written for the reference loads
here unchanged. The shipped corpus lists the reference corpus's 15 shapes.

The runner (the reference's benchmarks/run_corpus.py:1-134, which starts
benchmarks/benchmark.py once per case) measures every selected case in ONE
process: a GPU box allows few processes on its card, and the plans hold no
state between cases. Per case and scheme it times native BF16 (``F.linear``
for the dynamic path; ``torch.mm``/``torch.addmm`` into a preallocated output
for the prepacked path), the dynamic plan (``run_linear``, output allocated
per call) and the prepacked plan (``run_linear_packed``, output reused) with
the reference's protocol (benchmark.py:109-157): warmups and rounds in
rotated order, one HIP-event pair per call, median and quartiles. It also
records packing time and its break-even reuse count (benchmark.py:268-296),
and the full-output relative L2 error against an fp64 product next to native
BF16's.

``python -m rdna3_fastmm.corpus --list`` prints the cases;
``python -m rdna3_fastmm.corpus --case ID [--case ID ...] | --all
--output-directory DIR`` measures them (one JSON file per case);
``--sweep INNER,COLUMNS[,bias] --rows START:STOP:STEP --output-directory DIR``
measures one (K, N) pair over a range of row counts; ``--summarize DIR`` prints
a table, the exact shapes where a plan beat native, and the row intervals of a
sweep on which it beat native at every measured point (the runtime's dispatch
families).
"""

from __future__ import annotations

import argparse
from dataclasses import asdict, dataclass
import json
import math
from pathlib import Path
import sys
import time
from typing import Callable, Literal

DTypeName = Literal["float16", "bfloat16"]
DEFAULT_CORPUS_PATH = Path(__file__).resolve().parent / "corpora" / "comfyui-sota-2026.json"
SCHEMA_VERSION = 1
OPERATOR = "torch.nn.functional.linear"
CASE_KEYS = {
    "id", "model", "workload", "projection", "shape", "input_output_dtype", "compute_dtype",
    "weight_layout", "bias", "priority", "evidence",
}
EVIDENCE_KINDS = ("architecture-derived", "locally-profiled")
DTYPE_NAMES = ("float16", "bfloat16")


@dataclass(frozen=True)
class Evidence:
    kind: str
    note: str
    references: tuple[str, ...]


@dataclass(frozen=True)
class GemmCase:
    id: str
    model: str
    workload: str
    projection: str
    shape: tuple[int, int, int]
    input_output_dtype: DTypeName
    compute_dtype: DTypeName
    weight_layout: str
    bias: bool
    priority: int
    evidence: Evidence

    @property
    def rows(self) -> int:
        return self.shape[0]

    @property
    def inner(self) -> int:
        return self.shape[1]

    @property
    def columns(self) -> int:
        return self.shape[2]


@dataclass(frozen=True)
class GemmCorpus:
    schema_version: int
    name: str
    operator: str
    cases: tuple[GemmCase, ...]

    def case(self, case_id: str) -> GemmCase:
        for case in self.cases:
            if case.id == case_id:
                return case
        raise KeyError(f"corpus {self.name!r} has no case {case_id!r}")


# ------------------------------------------------------------------- loading

def _object(value: object, where: str, keys: set[str]) -> dict:
    if not isinstance(value, dict) or not all(isinstance(key, str) for key in value):
        raise ValueError(f"{where} must be an object with string keys")
    if value.keys() != keys:
        missing, unexpected = sorted(keys - value.keys()), sorted(value.keys() - keys)
        raise ValueError(f"{where} has invalid keys; missing={missing}, unexpected={unexpected}")
    return value


def _text(value: object, where: str) -> str:
    if not isinstance(value, str) or not value:
        raise ValueError(f"{where} must be a non-empty string")
    return value


def _int(value: object, where: str) -> int:
    # bool is an int subclass; JSON true/false are not integers here
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError(f"{where} must be an integer")
    return value


def _choice(value: object, allowed: tuple[str, ...], where: str) -> str:
    text = _text(value, where)
    if text not in allowed:
        raise ValueError(f"{where} must be one of {sorted(allowed)}")
    return text


def _case(raw: object, index: int) -> GemmCase:
    where = f"cases[{index}]"
    fields = _object(raw, where, CASE_KEYS)
    shape = fields["shape"]
    if not isinstance(shape, list) or len(shape) != 3:
        raise ValueError(f"{where}.shape must contain three dimensions")
    dims = tuple(_int(d, f"{where}.shape[]") for d in shape)
    if min(dims) < 1:
        raise ValueError(f"{where}.shape dimensions must be positive")
    priority = _int(fields["priority"], f"{where}.priority")
    if priority not in (1, 2, 3):
        raise ValueError(f"{where}.priority must be 1, 2, or 3")
    if not isinstance(fields["bias"], bool):
        raise ValueError(f"{where}.bias must be a boolean")
    evidence = _object(fields["evidence"], f"{where}.evidence", {"kind", "note", "references"})
    references = evidence["references"]
    if not isinstance(references, list):
        raise ValueError(f"{where}.evidence.references must be an array")
    if not references:
        raise ValueError(f"{where}.evidence.references must not be empty")
    return GemmCase(
        id=_text(fields["id"], f"{where}.id"),
        model=_text(fields["model"], f"{where}.model"),
        workload=_text(fields["workload"], f"{where}.workload"),
        projection=_text(fields["projection"], f"{where}.projection"),
        shape=dims,  # type: ignore[arg-type]
        input_output_dtype=_choice(fields["input_output_dtype"], DTYPE_NAMES, f"{where}.input_output_dtype"),  # type: ignore[arg-type]
        compute_dtype=_choice(fields["compute_dtype"], DTYPE_NAMES, f"{where}.compute_dtype"),  # type: ignore[arg-type]
        weight_layout=_choice(fields["weight_layout"], ("out_in",), f"{where}.weight_layout"),
        bias=fields["bias"],
        priority=priority,
        evidence=Evidence(
            kind=_choice(evidence["kind"], EVIDENCE_KINDS, f"{where}.evidence.kind"),
            note=_text(evidence["note"], f"{where}.evidence.note"),
            references=tuple(_text(r, f"{where}.evidence.references[]") for r in references),
        ),
    )


def load_corpus(path: Path = DEFAULT_CORPUS_PATH) -> GemmCorpus:
    """Parse and validate a corpus file (reference benchmarks/corpus.py:177-200)."""
    raw = _object(json.loads(Path(path).read_text()), "corpus", {"schema_version", "name", "operator", "cases"})
    version = _int(raw["schema_version"], "schema_version")
    if version != SCHEMA_VERSION:
        raise ValueError(f"unsupported corpus schema version {version}")
    operator = _text(raw["operator"], "operator")
    if operator != OPERATOR:
        raise ValueError(f"unsupported corpus operator {operator}")
    if not isinstance(raw["cases"], list) or not raw["cases"]:
        raise ValueError("cases must be a non-empty array")
    cases = tuple(_case(case, index) for index, case in enumerate(raw["cases"]))
    ids = [case.id for case in cases]
    if len(ids) != len(set(ids)):
        raise ValueError("case ids must be unique")
    return GemmCorpus(version, _text(raw["name"], "name"), operator, cases)


# ----------------------------------------------------------------- measuring

@dataclass(frozen=True)
class Timing:
    median_ms: float
    first_quartile_ms: float
    third_quartile_ms: float
    raw_ms: tuple[float, ...]


def quartile(values: list[float], quarter: int) -> float:
    """Linear interpolation between order statistics (reference benchmark.py:109-115)."""
    ordered = sorted(values)
    position = (len(ordered) - 1) * quarter / 4
    low = int(position)
    high = min(low + 1, len(ordered) - 1)
    fraction = position - low
    return ordered[low] * (1 - fraction) + ordered[high] * fraction


def timing(values: list[float]) -> Timing:
    return Timing(quartile(values, 2), quartile(values, 1), quartile(values, 3), tuple(values))


def measure(operations: dict[str, Callable[[], object]], warmups: int, rounds: int) -> dict[str, Timing]:
    """Warmups then rounds, each in an order rotated by one, one HIP-event pair
    per call on the current stream (reference benchmark.py:127-157)."""
    import torch

    names = list(operations)
    for index in range(warmups):
        shift = index % len(names)
        for name in names[shift:] + names[:shift]:
            operations[name]()
    torch.cuda.synchronize()
    samples: dict[str, list[float]] = {name: [] for name in names}
    for index in range(rounds):
        shift = index % len(names)
        for name in names[shift:] + names[:shift]:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            operations[name]()
            end.record()
            end.synchronize()
            samples[name].append(float(start.elapsed_time(end)))
    return {name: timing(values) for name, values in samples.items()}


def break_even_reuses(packing_ms: float, native_ms: float, prepacked_ms: float) -> int | None:
    """Calls after which packing has paid for itself (reference benchmark.py:290-296)."""
    saved = native_ms - prepacked_ms
    return math.ceil(packing_ms / saved) if saved > 0 else None


def _inputs(case: GemmCase, seed: int):
    """Synthetic inputs of the case's shape, drawn on the CPU (seeded) and copied."""
    import torch

    g = torch.Generator().manual_seed(seed)
    m, k, n = case.shape
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16)
    b = (torch.randn((n,), generator=g) * 0.02).to(torch.bfloat16) if case.bias else None
    return x, w, b


def run_case(case: GemmCase, schemes: tuple[str, ...], warmups: int, rounds: int, seed: int = 0) -> dict:
    """Measure one case on the current GPU; every tensor is freed before returning."""
    import torch

    from .runtime import PLAN_TYPES

    if case.input_output_dtype != "bfloat16":
        raise ValueError(f"{case.id}: the Linear plans take bfloat16 inputs, not {case.input_output_dtype}")
    device = torch.device("cuda", torch.cuda.current_device())
    compute = torch.float16 if case.compute_dtype == "float16" else torch.bfloat16
    x_cpu, w_cpu, b_cpu = _inputs(case, seed)
    x, w = x_cpu.to(device), w_cpu.to(device)
    b = None if b_cpu is None else b_cpu.to(device)
    m, k, n = case.shape
    flops = 2.0 * m * k * n
    exact = x.double() @ w.double().T
    if b is not None:
        exact += b.double()
    norm = float(torch.linalg.vector_norm(exact))

    def rel_l2(result) -> dict:
        finite = torch.isfinite(result)
        difference = torch.where(finite, result.double() - exact, torch.zeros_like(exact))
        return {"relative_l2_error": float(torch.linalg.vector_norm(difference)) / norm,
                "nonfinite_count": int((~finite).sum())}

    native_out = torch.empty((m, n), device=device, dtype=torch.bfloat16)

    def native_linear():
        return torch.nn.functional.linear(x, w, b)

    def native_into():
        if b is None:
            torch.mm(x, w.T, out=native_out)
        else:
            torch.addmm(b, x, w.T, out=native_out)

    native_into()
    native_error = rel_l2(native_out)
    report: dict = {
        "case": asdict(case),
        "device": torch.cuda.get_device_properties(device).gcnArchName,
        "torch": torch.__version__,
        "blas": str(torch.backends.cuda.preferred_blas_library()),
        "warmups": warmups,
        "rounds": rounds,
        "seed": seed,
        "native": {"error": native_error},
        "schemes": {},
    }
    for scheme in schemes:
        plan_type = PLAN_TYPES[scheme]
        if (torch.bfloat16, compute) not in plan_type.precision_pairs:
            report["schemes"][scheme] = {"skipped": f"no (bfloat16, {case.compute_dtype}) precision pair"}
            continue
        plan = plan_type(m, k, n, device, dtype=torch.bfloat16, compute_dtype=compute)
        workspace = plan.allocate_workspace()
        out = torch.empty((m, n), device=device, dtype=torch.bfloat16)
        plan.pack_weight(w)  # warm the packing kernels
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        packed = plan.pack_weight(w)
        end.record()
        end.synchronize()
        packing_ms = float(start.elapsed_time(end))
        dynamic_error = rel_l2(plan.run_linear(x, w, workspace, b))
        prepacked_error = rel_l2(plan.run_linear_packed(x, packed, workspace, b, out))
        timings = measure(
            {
                "native_linear": native_linear,
                "native_into": native_into,
                "dynamic": lambda: plan.run_linear(x, w, workspace, b),
                "prepacked": lambda: plan.run_linear_packed(x, packed, workspace, b, out),
            },
            warmups,
            rounds,
        )
        native_dynamic = timings["native_linear"].median_ms
        native_prepacked = timings["native_into"].median_ms
        report["schemes"][scheme] = {
            "compute_dtype": case.compute_dtype,
            "timings": {name: asdict(t) for name, t in timings.items()},
            "dynamic": {
                "speedup_vs_native": native_dynamic / timings["dynamic"].median_ms,
                "effective_tflops": flops / (timings["dynamic"].median_ms * 1e9),
                "error": dynamic_error,
                "error_ratio": dynamic_error["relative_l2_error"] / native_error["relative_l2_error"],
            },
            "prepacked": {
                "speedup_vs_native": native_prepacked / timings["prepacked"].median_ms,
                "effective_tflops": flops / (timings["prepacked"].median_ms * 1e9),
                "error": prepacked_error,
                "error_ratio": prepacked_error["relative_l2_error"] / native_error["relative_l2_error"],
                "packing_ms": packing_ms,
                "break_even_reuses": break_even_reuses(packing_ms, native_prepacked,
                                                       timings["prepacked"].median_ms),
            },
        }
        del plan, workspace, out, packed
        torch.cuda.empty_cache()
    del x, w, b, exact, native_out
    torch.cuda.empty_cache()
    return report


# ---------------------------------------------------------------- summarizing

ERROR_RATIO_BOUND = 1.2


def winning_families(reports: list[dict], minimum_speedup: float = 1.0) -> list[dict]:
    """Exact-shape families where a plan beat native within the error bound."""
    wins = []
    for report in reports:
        case = report["case"]
        rows, inner, columns = case["shape"]
        for scheme, result in report["schemes"].items():
            if "skipped" in result:
                continue
            for mode in ("dynamic", "prepacked"):
                entry = result[mode]
                if entry["speedup_vs_native"] >= minimum_speedup and entry["error_ratio"] <= ERROR_RATIO_BOUND:
                    wins.append({"scheme": scheme, "prepacked": mode == "prepacked", "rows": rows,
                                 "inner": inner, "columns": columns, "bias": case["bias"],
                                 "speedup": round(entry["speedup_vs_native"], 4), "case": case["id"]})
    return wins


def sweep_case(inner: int, columns: int, bias: bool, rows: int) -> GemmCase:
    """A synthetic corpus case for one point of a row sweep."""
    return GemmCase(
        id=f"sweep-{rows}x{inner}x{columns}{'-bias' if bias else ''}",
        model="row sweep", workload="synthetic", projection="linear", shape=(rows, inner, columns),
        input_output_dtype="bfloat16", compute_dtype="float16", weight_layout="out_in", bias=bias,
        priority=3, evidence=Evidence("locally-profiled", "row sweep point", ("rdna3_fastmm.corpus",)),
    )


def row_intervals(points: list[tuple[int, float, float]], minimum_speedup: float) -> list[tuple[int, int]]:
    """Maximal runs of consecutive sweep points (rows, speedup, error ratio),
    sorted by rows, on which every point beat native by ``minimum_speedup``
    within the error bound; each run is a measured row interval."""
    runs: list[tuple[int, int]] = []
    start = last = None
    for rows, speedup, ratio in sorted(points):
        if speedup >= minimum_speedup and ratio <= ERROR_RATIO_BOUND:
            start = rows if start is None else start
            last = rows
        elif start is not None:
            runs.append((start, last))
            start = None
    if start is not None:
        runs.append((start, last))
    return runs


def sweep_families(reports: list[dict], minimum_speedup: float, minimum_runs: int = 1) -> list[dict]:
    """Row-interval families per (scheme, mode, inner, columns, bias) of a sweep.

    Reports of repeated sweeps (other boxes, other days) combine point by
    point: a row counts with its slowest speedup and worst error ratio, so a
    family is a run of rows that beat native in every measurement. A row
    measured fewer than ``minimum_runs`` times counts as no win."""
    measured: dict[tuple, dict[int, list[tuple[float, float]]]] = {}
    for report in reports:
        rows, inner, columns = report["case"]["shape"]
        for scheme, result in report["schemes"].items():
            if "skipped" in result:
                continue
            for mode in ("dynamic", "prepacked"):
                key = (scheme, mode == "prepacked", inner, columns, report["case"]["bias"])
                entry = result[mode]
                measured.setdefault(key, {}).setdefault(rows, []).append(
                    (entry["speedup_vs_native"], entry["error_ratio"]))
    families = []
    for (scheme, prepacked, inner, columns, bias), by_rows in sorted(measured.items()):
        points = [(rows, min(s for s, _ in runs) if len(runs) >= minimum_runs else 0.0, max(r for _, r in runs))
                  for rows, runs in by_rows.items()]
        for low, high in row_intervals(points, minimum_speedup):
            inside = [speedup for rows, speedup, _ in points if low <= rows <= high]
            runs = min(len(runs) for rows, runs in by_rows.items() if low <= rows <= high)
            families.append({"scheme": scheme, "prepacked": prepacked, "minimum_rows": low, "maximum_rows": high,
                             "inner": inner, "columns": columns, "bias": bias, "points": len(inside),
                             "runs": runs, "minimum_speedup": round(min(inside), 4)})
    return families


DISPATCH_SCHEMA_VERSION = 1


def dispatch_document(reports: list[dict], minimum_speedup: float, measurement: str,
                      minimum_runs: int = 1) -> dict:
    """The runtime's dispatch table (``rdna3_fastmm/dispatch/mi355x.json``) from sweep reports."""
    devices = sorted({report.get("device", "?") for report in reports})
    torch_versions = sorted({report.get("torch", "?") for report in reports})
    return {
        "schema_version": DISPATCH_SCHEMA_VERSION,
        "devices": devices,
        "torch": torch_versions,
        "baseline": "native BF16: torch.nn.functional.linear (dynamic), torch.mm/addmm into a preallocated "
                    "output (prepacked)",
        "minimum_speedup": minimum_speedup,
        "error_ratio_bound": ERROR_RATIO_BOUND,
        "measurement": measurement,
        "families": sweep_families(reports, minimum_speedup, minimum_runs),
    }


def summary_table(reports: list[dict]) -> str:
    lines = ["| case | M×K×N | bias | scheme | native ms | dynamic ms (×) | prepacked ms (×) | err ratio |",
             "|---|---|---|---|---:|---:|---:|---:|"]
    for report in reports:
        case = report["case"]
        shape = "×".join(str(d) for d in case["shape"])
        for scheme, result in report["schemes"].items():
            if "skipped" in result:
                continue
            t = result["timings"]
            lines.append(
                f"| {case['id']} | {shape} | {'yes' if case['bias'] else 'no'} | {scheme} | "
                f"{t['native_into']['median_ms']:.3f} | "
                f"{t['dynamic']['median_ms']:.3f} ({result['dynamic']['speedup_vs_native']:.2f}) | "
                f"{t['prepacked']['median_ms']:.3f} ({result['prepacked']['speedup_vs_native']:.2f}) | "
                f"{result['prepacked']['error_ratio']:.3f} |"
            )
    return "\n".join(lines)


def _arguments(argv: list[str] | None) -> argparse.Namespace:
    parser = argparse.ArgumentParser(prog="python -m rdna3_fastmm.corpus")
    parser.add_argument("--corpus", type=Path, default=DEFAULT_CORPUS_PATH)
    selection = parser.add_mutually_exclusive_group(required=True)
    selection.add_argument("--list", action="store_true")
    selection.add_argument("--case", action="append")
    selection.add_argument("--all", action="store_true")
    selection.add_argument("--summarize", type=Path, metavar="DIR", action="append",
                           help="report directories to summarize (repeat to combine runs)")
    parser.add_argument("--dispatch-output", type=Path, metavar="FILE",
                        help="with --summarize: write the sweep families as a dispatch table")
    parser.add_argument("--measurement", default="",
                        help="with --dispatch-output: how the reports were measured (recorded in the table)")
    selection.add_argument("--sweep", action="append", metavar="INNER,COLUMNS[,bias]",
                           help="measure a row sweep of this (K, N) pair instead of corpus cases")
    parser.add_argument("--rows", default="480:20480:384", metavar="START:STOP:STEP",
                        help="row counts of a sweep (Python range)")
    parser.add_argument("--scheme", action="append", choices=("rank7", "rank48", "rank49"))
    parser.add_argument("--output-directory", type=Path)
    parser.add_argument("--warmups", type=int, default=3)
    parser.add_argument("--rounds", type=int, default=9)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--minimum-speedup", type=float, default=1.0)
    parser.add_argument("--minimum-runs", type=int, default=1,
                        help="with --summarize: rows measured fewer times than this never win")
    arguments = parser.parse_args(argv)
    running = arguments.case is not None or arguments.all or arguments.sweep is not None
    if running and arguments.output_directory is None:
        parser.error("--output-directory is required when running cases")
    if arguments.warmups < 1 or arguments.rounds < 3:
        parser.error("warmups must be positive and rounds must be at least three")
    if arguments.case is not None and len(arguments.case) != len(set(arguments.case)):
        parser.error("case ids must not be repeated")
    return arguments


def main(argv: list[str] | None = None) -> int:
    arguments = _arguments(argv)
    if arguments.summarize is not None:
        reports = [json.loads(p.read_text()) for d in arguments.summarize for p in sorted(d.glob("*.json"))]
        if arguments.dispatch_output is not None:
            document = dispatch_document(reports, arguments.minimum_speedup, arguments.measurement,
                                         arguments.minimum_runs)
            arguments.dispatch_output.write_text(json.dumps(document, indent=1) + "\n")
            print(f"{len(document['families'])} families -> {arguments.dispatch_output}")
            return 0
        print(summary_table(reports))
        print(json.dumps(winning_families(reports, arguments.minimum_speedup), indent=1))
        print(json.dumps(sweep_families(reports, arguments.minimum_speedup, arguments.minimum_runs), indent=1))
        return 0
    if arguments.sweep is not None:
        start, stop, step = (int(v) for v in arguments.rows.split(":"))
        selected = []
        for pair in arguments.sweep:
            fields = pair.split(",")
            if len(fields) not in (2, 3) or (len(fields) == 3 and fields[2] != "bias"):
                raise SystemExit(f"--sweep takes INNER,COLUMNS or INNER,COLUMNS,bias, not {pair!r}")
            selected += [sweep_case(int(fields[0]), int(fields[1]), len(fields) == 3, rows)
                         for rows in range(start, stop, step)]
    else:
        corpus = load_corpus(arguments.corpus)
        if arguments.list:
            for case in corpus.cases:
                bias = "bias" if case.bias else "no-bias"
                print(f"{case.id}\tpriority={case.priority}\t{'x'.join(map(str, case.shape))}\t{bias}")
            return 0
        selected = corpus.cases if arguments.all else tuple(corpus.case(i) for i in arguments.case)
    schemes = tuple(arguments.scheme or ("rank7", "rank48", "rank49"))
    arguments.output_directory.mkdir(parents=True, exist_ok=True)
    for index, case in enumerate(selected, start=1):
        print(f"[{index}/{len(selected)}] {case.id} {'x'.join(map(str, case.shape))} {','.join(schemes)}", flush=True)
        began = time.perf_counter()
        report = run_case(case, schemes, arguments.warmups, arguments.rounds, arguments.seed)
        (arguments.output_directory / f"{case.id}.json").write_text(json.dumps(report, indent=1) + "\n")
        for scheme, result in report["schemes"].items():
            if "skipped" in result:
                print(f"    {scheme}: skipped ({result['skipped']})", flush=True)
                continue
            print(f"    {scheme}: dynamic {result['dynamic']['speedup_vs_native']:.3f}x, prepacked "
                  f"{result['prepacked']['speedup_vs_native']:.3f}x, error ratio "
                  f"{result['prepacked']['error_ratio']:.3f} ({time.perf_counter() - began:.1f} s)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
