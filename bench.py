"""Benchmark: fast-matmul Linears on one MI355X against native BF16, one JSON line.

Headline workload (the largest single-GPU BASELINE configuration, C4): the
rank-49 prepacked plan on the biased MLP-up linear M x K x N = 19968 x 4096 x
16384, x ~ N(0,1) BF16, weight[N, K] ~ N(0, 1/K) BF16, bias ~ N(0, 0.02),
FP16 leaves, workspace and output reused. ``--steps`` K back-to-back calls
of ``run_linear_packed`` are timed between two synchronizations; ``value``
is the effective TFLOP/s 2*M*N*K / t of those K calls.

In the same run, and in the same line under ``points``, every other GPU
configuration is measured the same way: C2 (rank-7 dynamic), C3 (rank-7
prepacked + bias), C5 (rank-48 prepacked 8192^3) with its rank-7 and rank-49
controls, and the north star's rank-48 point at 8214 x 12288 x 4608. For each
(headline included): sustained back-to-back ms against native BF16; the
reference's protocol (benchmarks/benchmark.py:109-157: warmups, then rounds
in rotated order, one HIP-event pair per operation, median and quartiles);
the per-stage HIP-event times recorded inside the timed calls; the
full-output error ratio against native; packing time and break-even uses;
memory estimate, free and peak bytes (benchmark.py:299-319, 631-707).

``roofline`` is the headline's leaf-product stage (the dominant kernel:
mfma16::persistent_kernel plus its split-K tail), with HIP events recorded
on the launch stream around that stage in each timed call. ``cpu_baseline``
times the CPU oracle (the reference's scheme evaluation restated in numpy)
on a row sample of the headline workload; ``cpu_c1`` runs the BASELINE's C1
CPU protocol (rank 7, 1024^3, 3 warmups, 9 rounds).

``--config NAME`` makes another configuration the headline; ``--only``
skips the other points.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
from pathlib import Path
import platform
import subprocess
import sys
import time

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT / "rdna3-fastmm_amd"))

import torch  # noqa: E402

METRIC = "ms and effective TFLOP/s per linear vs native BF16 GEMM (speedup), 1 MI355X"
MFMA_16BIT_PEAK_TFLOPS = 2500.0  # dense FP16 and BF16 MFMA peak of MI355X
HBM_PEAK_GBPS = 8000.0
ERROR_RATIO_BOUND = 1.2
HEADLINE = "c4"
POINTS = ("c2", "c3", "c3-rank48", "c5", "c5-rank7", "c5-rank49")
ENVIRONMENT_KEYS = (
    "TORCH_BLAS_PREFER_HIPBLASLT",
    "PYTORCH_TUNABLEOP_ENABLED",
    "PYTORCH_TUNABLEOP_TUNING",
    "PYTORCH_TUNABLEOP_FILENAME",
    "HIP_VISIBLE_DEVICES",
    "HSA_XNACK",
    "OMP_NUM_THREADS",
)

CONFIGS = {
    "c1": dict(scheme="rank7", rows=1024, inner=1024, columns=1024, bias=False, prepacked=False,
               name="C1 rank7-cpu-1024x1024x1024"),
    "c2": dict(scheme="rank7", rows=4096, inner=4096, columns=12288, bias=False, prepacked=False,
               name="C2 rank7-dynamic-mlp-up-4096x4096x12288"),
    "c3": dict(scheme="rank7", rows=8214, inner=12288, columns=4608, bias=True, prepacked=True,
               name="C3 rank7-prepacked-mlp-down-8214x12288x4608-bias"),
    "c3-rank48": dict(scheme="rank48", rows=8214, inner=12288, columns=4608, bias=False, prepacked=True,
                      name="north-star rank48-prepacked-8214x12288x4608"),
    "c4": dict(scheme="rank49", rows=19968, inner=4096, columns=16384, bias=True, prepacked=True,
               name="C4 rank49-prepacked-mlp-up-19968x4096x16384-bias"),
    "c4-bf16": dict(scheme="rank49", rows=19968, inner=4096, columns=16384, bias=True, prepacked=True,
                    compute="bf16", name="C4 rank49-bf16-leaves-prepacked-mlp-up-19968x4096x16384-bias"),
    "c5": dict(scheme="rank48", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
               name="C5 rank48-prepacked-square-8192"),
    "c5-rank7": dict(scheme="rank7", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
                     name="C5 control rank7-prepacked-square-8192"),
    "c5-rank49": dict(scheme="rank49", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
                      name="C5 control rank49-prepacked-square-8192"),
    # FP16 mm (not Linear): the reference's rank-343 prepacked shape
    "c6-rank343": dict(scheme="rank343", rows=16384, inner=16384, columns=16384, bias=False, prepacked=True,
                       mm=True, name="rank343-prepacked-fp16-mm-16384"),
}


def _inputs(cfg: dict, seed: int = 0):
    """BASELINE inputs on the CPU: seeded torch.Generator, x ~ N(0,1), W ~ N(0,1/K), bias std 0.02."""
    g = torch.Generator().manual_seed(seed)
    m, k, n = cfg["rows"], cfg["inner"], cfg["columns"]
    if cfg.get("mm"):
        # FP16 left[M, K] @ right[K, N]; "w" is the right operand
        return (torch.randn((m, k), generator=g).to(torch.float16),
                (torch.randn((k, n), generator=g) / k**0.5).to(torch.float16), None)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16)
    b = (torch.randn((n,), generator=g) * 0.02).to(torch.bfloat16) if cfg["bias"] else None
    return x, w, b


def _quartile(values: list[float], numerator: int) -> float:
    """Linear-interpolated quartile (reference benchmark.py:109-115)."""
    ordered = sorted(values)
    position = (len(ordered) - 1) * numerator / 4
    lower = int(position)
    upper = min(lower + 1, len(ordered) - 1)
    weight = position - lower
    return ordered[lower] * (1 - weight) + ordered[upper] * weight


def _summary(values: list[float]) -> dict:
    return {"median_ms": round(_quartile(values, 2), 4), "q1_ms": round(_quartile(values, 1), 4),
            "q3_ms": round(_quartile(values, 3), 4), "rounds": len(values)}


def _sustained_ms(fn, steps: int) -> float:
    """ms per call over `steps` back-to-back calls, synchronized on both sides."""
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - start) * 1e3 / steps


def _event_ms(fn) -> float:
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end)


def rotated_rounds(operations: dict, warmups: int, rounds: int) -> dict:
    """reference benchmark.py:137-157: warmups and rounds in rotated order, one event pair per op."""
    names = list(operations)
    for warmup in range(warmups):
        offset = warmup % len(names)
        for name in names[offset:] + names[:offset]:
            operations[name]()
    torch.cuda.synchronize()
    raw: dict[str, list[float]] = {name: [] for name in names}
    for index in range(rounds):
        offset = index % len(names)
        for name in names[offset:] + names[:offset]:
            raw[name].append(_event_ms(operations[name]))
    return {name: _summary(values) for name, values in raw.items()}


class StageClock:
    """HIP events around each stage of the plan's own calls (on the launch stream).

    Installed on a plan instance by wrapping its stage methods, so the timed
    calls are the public API calls themselves; while ``armed`` every stage
    call records a start and an end event on torch's current stream, which is
    the stream the library launches on."""

    STAGES = ("_transform_left", "_transform_weight", "_transform_right", "_leaf_products", "_reconstruct")

    def __init__(self, plan) -> None:
        self.armed: frozenset = frozenset()  # stage names that record events
        self.events: dict[str, list] = {}
        for name in self.STAGES:
            original = getattr(plan, name)
            setattr(plan, name, self._wrap(name, original))

    def _wrap(self, name: str, original):
        def timed(*args, **kwargs):
            if name not in self.armed:
                return original(*args, **kwargs)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            result = original(*args, **kwargs)
            end.record()
            self.events.setdefault(name.lstrip("_"), []).append((start, end))
            return result
        return timed

    def averages_ms(self) -> dict[str, float]:
        torch.cuda.synchronize()
        averages = {name: sum(s.elapsed_time(e) for s, e in pairs) / len(pairs) for name, pairs in self.events.items()}
        self.events = {}
        return averages


def leaf_kernel_name(rank: int, mb: int, kb: int, nb: int, compute: str, cus: int, split_tail: bool) -> str:
    """The main leaf-GEMM kernel fastmm_leaf_products runs for the bench shapes (aligned
    16-bit products), by the library's launch rule: on the 16x16x32 path (Kb % 128 == 0)
    the persistent kernel when the tiles left after the split-K tail exceed one round
    (CUs rounded down to a multiple of 8), Kb >= 256 and a leaf's products fit 32-bit
    offsets; else one workgroup per tile; the 32x32x16 kernel for other Kb. A last tile
    row of at most 16 rows is left out of the 256x256 tiles when that takes them down a
    round: fused into the persistent kernel (its strip form) when those tiles have no
    split-K tail and the last group of 8 tile rows holds at least 4, else run by
    fastmm::thin::thin_rows_kernel when R * Nb <= 32768."""
    if kb % 128:
        return f"fastmm::fast::leaf_gemm_kernel<{compute}, {compute}> (fastmm_leaf_products)"
    tiles_n = -(-nb // 256)
    with_row = rank * -(-mb // 256) * tiles_n
    without = with_row - rank * tiles_n

    def split_of(tiles: int) -> tuple[int, int]:
        tail = tiles % cus
        split = min(8, kb // 128, 3 * cus // (4 * tail)) if tail else 0
        return tail, split

    drop = mb > 256 and 0 < mb % 256 <= 16 and -(-without // cus) < -(-with_row // cus)
    full = mb // 256
    strip = drop and full - 8 * ((full - 1) // 8) >= 4 and split_of(without)[1] < 2
    thin = drop and not strip and rank * nb <= 32768
    tiles = without if strip or thin else with_row
    tail, split = split_of(tiles)
    main = tiles - tail if split_tail and split >= 2 else tiles
    extra = " + thin_rows_kernel for the last tile row" if thin else ""
    if main > cus // 8 * 8 and kb >= 256 and mb * nb * 2 <= 2**31 - 1:
        stream = "true" if rank * mb * nb * 2 > 2**30 else "false"  # products stored non-temporally
        fused = "true" if strip else "false"  # the last tile row fused as a strip
        return (f"fastmm::mfma16::persistent_kernel<{compute}, {compute}, {stream}, {fused}> "
                f"(fastmm_leaf_products){extra}")
    if strip:
        extra = " + thin_rows_kernel for the last tile row"
    return f"fastmm::mfma16::leaf_gemm_kernel<{compute}, {compute}> (fastmm_leaf_products){extra}"


def measured_traffic(config: str) -> float | None:
    """HBM-side bytes per leaf-GEMM launch from the committed rocprofv3 summary, if any.

    profiles/leaf_gemm_traffic_<config>.md holds FETCH_SIZE + WRITE_SIZE of the
    same workload, scaled by a 1 GiB copy (see that file for the commands).
    """
    path = REPO_ROOT / "profiles" / f"leaf_gemm_traffic_{config}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split(":")[1])
    return None


def _sha256(path: Path) -> str | None:
    return hashlib.sha256(path.read_bytes()).hexdigest() if path.exists() else None


def provenance() -> dict:
    """What produced the numbers: commit (when .git is present), digests of the library,
    its sources, the generated scheme programs and the certificates, and the runtime."""
    package = REPO_ROOT / "rdna3-fastmm_amd"
    commit, dirty = None, None
    try:
        commit = subprocess.run(["git", "rev-parse", "HEAD"], cwd=REPO_ROOT, capture_output=True, text=True,
                                check=True, timeout=10).stdout.strip()
        dirty = bool(subprocess.run(["git", "status", "--porcelain"], cwd=REPO_ROOT, capture_output=True,
                                    text=True, check=True, timeout=10).stdout.strip())
    except (OSError, subprocess.SubprocessError):
        pass  # the GPU box's snapshot carries no .git
    sources = hashlib.sha256()
    for path in sorted((package / "csrc").rglob("*")) + sorted((package / "rdna3_fastmm").glob("*.py")):
        if path.is_file():
            sources.update(path.relative_to(package).as_posix().encode())
            sources.update(path.read_bytes())
    from rdna3_fastmm import _native
    from rdna3_fastmm.schemes import load_scheme

    schemes = {}
    for key in ("rank7", "rank48", "rank49"):
        scheme = load_scheme(key)
        header = package / "csrc" / "generated" / f"{key}_{scheme.size}x{scheme.size}x{scheme.size}.h"
        schemes[key] = {"certificate_sha256": scheme.certificate_sha256,
                        "library_sha256": _native.scheme_sha256(scheme.scheme_id),
                        "generated_header_sha256": _sha256(header)}
    return {
        "git_commit": commit,
        "git_dirty": dirty,
        "source_tree_sha256": sources.hexdigest(),
        "library_sha256": _sha256(package / "rdna3_fastmm" / "libfastmm_amd.so"),
        "abi_version": _native.ABI_VERSION,
        "schemes": schemes,
        "bench_sha256": _sha256(Path(__file__)),
        "python": platform.python_version(),
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "blas": str(torch.backends.cuda.preferred_blas_library()),
        "tunableop_enabled": bool(torch.cuda.tunable.is_enabled()),
        "environment": {key: os.environ.get(key) for key in ENVIRONMENT_KEYS},
    }


def _cpu_threads() -> int:
    # a GPU box's CPU share is 16 threads whatever os.cpu_count() reports
    return max(1, min(16, os.cpu_count() or 1))


def _oracle_call(cfg: dict, scheme, x, w, b, packed):
    from oracle import fastmm_oracle as O

    mm = bool(cfg.get("mm"))
    transform = O.right_transform if mm else O.weight_transform  # mm: w is right[K, N]
    columns = w.shape[1] if mm else w.shape[0]

    def one() -> None:
        a = O.left_transform(scheme, x)
        bt = packed if packed is not None else transform(scheme, w)
        p = O.leaf_products(a, bt, product_dtype="fp16", accumulate="f32")
        O.reconstruct(scheme, p, x.shape[0], columns, b, "fp16" if mm else "bf16")

    return one, transform


def cpu_baseline(cfg: dict, x, w, b, budget_s: float) -> dict:
    """The CPU oracle on a 256-row sample of the workload: TFLOP/s of that sample."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import fastmm_oracle as O

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    scheme = O.load_oracle_scheme(cfg["scheme"])
    rows = 256
    xs = x[:rows].float().numpy()
    wn = w.float().numpy()
    bn = None if b is None else b.float().numpy()
    with threadpool_limits(limits=cores):
        blas_threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
        _, transform = _oracle_call(cfg, scheme, xs, wn, bn, None)
        packed = transform(scheme, wn) if cfg["prepacked"] else None
        one, _ = _oracle_call(cfg, scheme, xs, wn, bn, packed)
        one()  # warm
        times = []
        deadline = time.perf_counter() + budget_s
        while True:
            t0 = time.perf_counter()
            one()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > deadline or len(times) >= 20:
                break
    seconds = float(np.median(times))
    flops = 2.0 * rows * cfg["inner"] * cfg["columns"]
    return {
        "value": flops / seconds / 1e12,
        "unit": "TFLOP/s",
        "cores": int(min(cores, blas_threads)),
        "kind": "port",
        "sample": (
            f"{rows} of {cfg['rows']} rows of {cfg['name']} "
            f"({'prepacked weight' if cfg['prepacked'] else 'weight transformed per call'}), "
            f"fp32 BLAS leaf sums, median of {len(times)} runs, {seconds * 1e3:.0f} ms each"
        ),
        "os_cpu_count": os.cpu_count(),
        "torch_num_threads": torch.get_num_threads(),
    }


def cpu_c1() -> dict:
    """BASELINE C1: rank 7 at 1024^3 through the CPU oracle, 3 warmups + 9 rounds, rel-L2 vs fp64."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import fastmm_oracle as O

    cfg = CONFIGS["c1"]
    cores = _cpu_threads()
    torch.set_num_threads(cores)
    x, w, _ = _inputs(cfg)
    xn, wn = x.float().numpy(), w.float().numpy()
    scheme = O.load_oracle_scheme("rank7")
    with threadpool_limits(limits=cores):
        blas_threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
        times = []
        for index in range(12):
            t0 = time.perf_counter()
            out = O.linear(scheme, xn, wn, accumulate="f32")
            if index >= 3:
                times.append((time.perf_counter() - t0) * 1e3)
    exact = xn.astype(np.float64) @ wn.astype(np.float64).T
    native = O.bf16_bits_to_f32(O.round_to_bf16((xn @ wn.T).astype(np.float32)))
    error = float(np.linalg.norm(O.bf16_bits_to_f32(out) - exact) / np.linalg.norm(exact))
    native_error = float(np.linalg.norm(native - exact) / np.linalg.norm(exact))
    flops = 2.0 * cfg["rows"] * cfg["inner"] * cfg["columns"]
    summary = _summary(times)
    return {
        "workload": cfg["name"],
        "ms": summary,
        "tflops": round(flops / (summary["median_ms"] * 1e-3) / 1e12, 4),
        "protocol": "3 warmups, 9 rounds, wall clock per call",
        "rel_l2": error,
        "native_bf16_rel_l2": native_error,
        "error_ratio": round(error / native_error, 4),
        "native_emulation": "fp32 BLAS x @ W.T rounded once to bf16",
        "cores": int(min(cores, blas_threads)),
        "os_cpu_count": os.cpu_count(),
        "torch_num_threads": torch.get_num_threads(),
    }


def measure(config: str, steps: int, warmup: int, rounds: int, device: torch.device) -> tuple[dict, tuple]:
    """Every figure for one configuration; returns the record and its CPU inputs."""
    from rdna3_fastmm.runtime import PLAN_TYPES, Rank343Plan, operand_shape

    cfg = CONFIGS[config]
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(device)
    free_before, total = torch.cuda.mem_get_info(device)
    x_cpu, w_cpu, b_cpu = _inputs(cfg)
    x, w = x_cpu.to(device), w_cpu.to(device)
    b = None if b_cpu is None else b_cpu.to(device)
    m, k, n = cfg["rows"], cfg["inner"], cfg["columns"]
    flops = 2.0 * m * n * k

    compute = torch.bfloat16 if cfg.get("compute") == "bf16" else torch.float16
    mm = bool(cfg.get("mm"))
    io_dtype = torch.float16 if mm else torch.bfloat16
    plan_type = Rank343Plan if cfg["scheme"] == "rank343" else PLAN_TYPES[cfg["scheme"]]
    plan = plan_type(m, k, n, device, dtype=io_dtype, compute_dtype=compute)
    clock = StageClock(plan)
    workspace = plan.allocate_workspace(prepacked_right=cfg["prepacked"])
    pack = (lambda: plan.pack_right(w)) if mm else (lambda: plan.pack_weight(w))
    warm = pack()  # reference benchmark.py:268-287: one warmup packing, then one timed
    torch.cuda.synchronize()
    del warm
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    packed = pack()
    end.record()
    end.synchronize()
    pack_ms, pack_wall_ms = start.elapsed_time(end), (time.perf_counter() - t0) * 1e3
    if not cfg["prepacked"] and not mm:
        packed = None
    out = torch.empty((m, n), device=device, dtype=io_dtype) if cfg["prepacked"] else None
    native_out = torch.empty((m, n), device=device, dtype=io_dtype)

    if mm:
        def step():
            plan.run_packed(x, packed, workspace, out)

        def native():
            torch.mm(x, w, out=native_out)
        native_op = "torch.mm(left, right, out=) fp16"
    elif cfg["prepacked"]:
        def step():
            plan.run_linear_packed(x, packed, workspace, b, out)

        def native():
            if b is None:
                torch.mm(x, w.T, out=native_out)
            else:
                torch.addmm(b, x, w.T, out=native_out)
        native_op = "torch.addmm(bias, x, W.T, out=)" if b is not None else "torch.mm(x, W.T, out=)"
    else:
        def step():
            plan.run_linear(x, w, workspace, b)

        def native():
            torch.nn.functional.linear(x, w, b)
        native_op = "torch.nn.functional.linear"

    for _ in range(warmup):
        step()
        native()
    # The K timed calls, with one HIP-event pair around the leaf stage inside each
    # (events at every stage boundary would drain the queue there and slow the calls).
    clock.armed = frozenset({"_leaf_products"})
    ms = _sustained_ms(step, steps)
    leaf_live_ms = clock.averages_ms()["leaf_products"]
    # then the same K calls with events around every stage, for the breakdown
    clock.armed = frozenset(StageClock.STAGES)
    staged_ms = _sustained_ms(step, steps)
    stages = clock.averages_ms()
    clock.armed = frozenset()
    native_ms = _sustained_ms(native, steps)
    protocol = rotated_rounds({"fastmm": step, "native": native}, warmups=2, rounds=rounds)

    shape = plan.shape
    leaf_flops = 2.0 * plan.rank * shape.block_rows * shape.block_inner * shape.block_columns
    leaf_tflops = leaf_flops / (leaf_live_ms * 1e-3) / 1e12

    # accuracy on this workload (outside the timed region)
    if mm:
        result = plan.run_packed(x, packed, workspace, out).clone()
    elif cfg["prepacked"]:
        result = plan.run_linear_packed(x, packed, workspace, b, out).clone()
    else:
        result = plan.run_linear(x, w, workspace, b)
    exact = x.double() @ (w.double() if mm else w.double().T)
    if b is not None:
        exact += b.double()
    norm = torch.linalg.vector_norm(exact)
    reference = torch.mm(x, w) if mm else torch.nn.functional.linear(x, w, b)
    native_err = float(torch.linalg.vector_norm(reference.double() - exact) / norm)
    err = float(torch.linalg.vector_norm(result.double() - exact) / norm)
    nonfinite = int((~torch.isfinite(result)).sum())
    del exact, reference, result
    free_after, _ = torch.cuda.mem_get_info(device)

    per_call = protocol["fastmm"]["median_ms"]
    native_per_call = protocol["native"]["median_ms"]
    saved = native_per_call - per_call
    record = {
        "workload": cfg["name"],
        "scheme": cfg["scheme"],
        "rows": m,
        "inner": k,
        "columns": n,
        "bias": cfg["bias"],
        "prepacked_weight": cfg["prepacked"],
        "ms_per_step": round(ms, 4),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "native_ms_per_step": round(native_ms, 4),
        "native_tflops": round(flops / (native_ms * 1e-3) / 1e12, 2),
        "speedup_vs_native": round(native_ms / ms, 4),
        "per_call": {"fastmm": protocol["fastmm"], "native": protocol["native"],
                     "speedup_vs_native": round(native_per_call / per_call, 4)},
        "native_op": native_op,
        "accuracy": {
            "rel_l2": err,
            "native_rel_l2": native_err,
            "error_ratio": round(err / native_err, 4),
            # Linear: the north-star 1.2x native BF16 error; FP16 mm: the reference's
            # rel-L2 < 5e-3 (native FP16 rounds only its output, so a ratio bound is moot)
            "bound": "rel_l2 < 5e-3" if mm else ERROR_RATIO_BOUND,
            "within_bound": (err < 5e-3) if mm else (err / native_err <= ERROR_RATIO_BOUND),
            "nonfinite": nonfinite,
        },
        "stages_ms": {name: round(v, 4) for name, v in stages.items()},
        "stages_pass_ms_per_step": round(staged_ms, 4),
        "leaf_ms_timed_region": round(leaf_live_ms, 4),
        "leaf": {
            "flops": leaf_flops,
            "tflops": round(leaf_tflops, 2),
            "mfma_frac": round(leaf_tflops / MFMA_16BIT_PEAK_TFLOPS, 4),
        },
        "packing": {
            "device_ms": round(pack_ms, 4),
            "wall_ms": round(pack_wall_ms, 4),
            "break_even_reuses_vs_native": (math.ceil(pack_ms / saved) if saved > 0 else None),
        },
        "memory": {
            "estimated_required_bytes": int(
                (m * k + n * k + 2 * m * n) * 2 + (n * 2 if cfg["bias"] else 0)
                + (plan.prepacked_workspace_bytes + plan.packed_right_bytes if cfg["prepacked"]
                   else plan.workspace_bytes) + plan.leaf_scratch_bytes),
            "free_before_bytes": free_before,
            "free_after_bytes": free_after,
            "total_bytes": total,
            "peak_allocated_bytes": torch.cuda.max_memory_allocated(device),
            "workspace_bytes": plan.workspace_bytes,
            "prepacked_workspace_bytes": plan.prepacked_workspace_bytes,
            "packed_weight_bytes": plan.packed_right_bytes,
            "leaf_scratch_bytes": plan.leaf_scratch_bytes,
        },
        "_leaf_kernel": leaf_kernel_name(
            plan.rank, shape.block_rows, shape.block_inner, shape.block_columns,
            "bf16" if compute == torch.bfloat16 else "fp16",
            torch.cuda.get_device_properties(device).multi_processor_count, workspace.leaf_scratch is not None,
        ) + (" + split-K tail (kPartial parts + tail_reduce_kernel) where the plan splits; timed as the whole "
             "stage" if workspace.leaf_scratch is not None else ""),
    }
    del workspace, packed, out, native_out, x, w, b, plan, clock
    torch.cuda.empty_cache()
    return record, (x_cpu, w_cpu, b_cpu)


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--rounds", type=int, default=9, help="rotated per-call rounds (reference protocol)")
    parser.add_argument("--config", default=HEADLINE, choices=sorted(c for c in CONFIGS if c != "c1"))
    parser.add_argument("--only", action="store_true", help="measure the headline configuration only")
    parser.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument(
        "--traffic-calibration",
        action="store_true",
        help="also run three 1 GiB device copies (a kernel of known HBM traffic) for counter scaling",
    )
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box in this setup has one MI355X, and the "
              "fast-matmul Linear path is single-GPU (row/column sharding needs no collective).",
              file=sys.stderr)
        return 2

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.traffic_calibration:
        source = torch.empty(1 << 29, device=device, dtype=torch.float16)
        target = torch.empty_like(source)
        for _ in range(3):
            target.copy_(source)
        torch.cuda.synchronize()
        del source, target

    head, head_inputs = measure(args.config, args.steps, args.warmup, args.rounds, device)
    points = {}
    if not args.only:
        for name in POINTS:
            if name != args.config:
                record, _ = measure(name, args.steps, args.warmup, args.rounds, device)
                record.pop("_leaf_kernel")
                points[name] = record
    cfg = CONFIGS[args.config]
    mm = bool(cfg.get("mm"))
    compute_bf16 = cfg.get("compute") == "bf16"
    leaf_kernel = head.pop("_leaf_kernel")
    line = {
        "metric": METRIC,
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{'fp16' if mm else 'bf16'} in/out, {'bf16' if compute_bf16 else 'fp16'} MFMA leaves, "
                 "fp32 accumulate",
        "data": "synthetic (seeded CPU torch.Generator: x~N(0,1), W~N(0,1/K), bias~N(0,0.02))",
        "config": {
            "workload": head["workload"],
            "scheme": head["scheme"],
            "rows": head["rows"],
            "inner": head["inner"],
            "columns": head["columns"],
            "bias": head["bias"],
            "prepacked_weight": head["prepacked_weight"],
            "parallelism": "single GPU",
        },
        "native_bf16": {
            "ms_per_step": head["native_ms_per_step"],
            "tflops": head["native_tflops"],
            "op": head["native_op"],
        },
        "speedup_vs_native": head["speedup_vs_native"],
        "per_call": head["per_call"],
        "accuracy": head["accuracy"],
        "stages_ms": head["stages_ms"],
        "stages_pass_ms_per_step": head["stages_pass_ms_per_step"],
        "leaf_ms_timed_region": head["leaf_ms_timed_region"],
        "packing": head["packing"],
        "memory": head["memory"],
        "roofline": {
            "kernel": leaf_kernel,
            "bound": "mfma",
            "achieved": head["leaf"]["tflops"],
            "peak": MFMA_16BIT_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": head["leaf"]["mfma_frac"],
            "traffic": measured_traffic(args.config),
            "work_per_launch": f"2*R*Mb*Kb*Nb = {head['leaf']['flops']:.4e} flop",
            "timing": f"HIP events on the launch stream around the leaf stage of each of the {args.steps} "
                      "timed calls (mean); stages_ms comes from a second pass with events at every stage",
        },
        "points": points,
        "provenance": provenance(),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, *head_inputs, args.cpu_budget)
        line["cpu_c1"] = cpu_c1()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
