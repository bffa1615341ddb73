"""Benchmark: one fast-matmul Linear per step on one MI355X, vs native BF16.

Default workload: rank-7 dynamic plan, MLP-up
linear M x K x N = 4096 x 4096 x 12288, x ~ N(0,1) BF16, weight[N, K] ~
N(0, 1/K) BF16, no bias, FP16 leaves, output allocated per call, workspace
reused. Inputs are generated on the CPU with a seeded torch.Generator and
copied to HBM before timing. Other configurations: --config c3|c4|c4-bf16|c5|
c5-rank7|c5-rank49|c3-rank48 (c4-bf16: the rank-49 plan with BF16 leaves).

Prints ONE JSON line (the driver's contract). ``value`` is effective TFLOP/s
= 2*M*N*K / t over the K timed steps; ``roofline`` is measured for the leaf
product kernel (the dominant one) with HIP events on the stream it runs on;
``cpu_baseline`` times the CPU oracle (the reference's scheme evaluation
restated in numpy) on a bounded row sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
from pathlib import Path
import sys
import time

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT / "rdna3-fastmm_amd"))

import torch  # noqa: E402

METRIC = "ms and effective TFLOP/s per linear vs native BF16 GEMM (speedup), 1 MI355X"
MFMA_16BIT_PEAK_TFLOPS = 2500.0  # dense FP16 and BF16 MFMA peak of MI355X
HBM_PEAK_GBPS = 8000.0

CONFIGS = {
    "c2": dict(scheme="rank7", rows=4096, inner=4096, columns=12288, bias=False, prepacked=False,
               name="rank7-dynamic-mlp-up-4096x4096x12288"),
    "c3": dict(scheme="rank7", rows=8214, inner=12288, columns=4608, bias=True, prepacked=True,
               name="rank7-prepacked-mlp-down-8214x12288x4608-bias"),
    "c3-rank48": dict(scheme="rank48", rows=8214, inner=12288, columns=4608, bias=False, prepacked=True,
                      name="rank48-prepacked-8214x12288x4608"),
    "c4": dict(scheme="rank49", rows=19968, inner=4096, columns=16384, bias=True, prepacked=True,
               name="rank49-prepacked-mlp-up-19968x4096x16384-bias"),
    "c4-bf16": dict(scheme="rank49", rows=19968, inner=4096, columns=16384, bias=True, prepacked=True,
                    compute="bf16", name="rank49-bf16-leaves-prepacked-mlp-up-19968x4096x16384-bias"),
    "c5": dict(scheme="rank48", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
               name="rank48-prepacked-square-8192"),
    "c5-rank7": dict(scheme="rank7", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
                     name="rank7-prepacked-square-8192"),
    "c5-rank49": dict(scheme="rank49", rows=8192, inner=8192, columns=8192, bias=False, prepacked=True,
                      name="rank49-prepacked-square-8192"),
    # FP16 mm (not Linear): the reference's rank-343 prepacked shape
    "c6-rank343": dict(scheme="rank343", rows=16384, inner=16384, columns=16384, bias=False, prepacked=True,
                       mm=True, name="rank343-prepacked-fp16-mm-16384"),
}


def _inputs(cfg: dict, seed: int = 0):
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


def _time_region(fn, steps: int) -> float:
    """ms per call over `steps` calls, synchronized on both sides."""
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - start) * 1e3 / steps


def _event_ms(fn, repeats: int) -> list[float]:
    """Per-call HIP-event durations on the current stream (where our kernels run)."""
    out = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        out.append(start.elapsed_time(end))
    return out


def _median(values: list[float]) -> float:
    ordered = sorted(values)
    return ordered[len(ordered) // 2]


def leaf_kernel_name(rank: int, mb: int, kb: int, nb: int, compute: str, cus: int, split_tail: bool) -> str:
    """The main leaf-GEMM kernel fastmm_leaf_products runs for the bench shapes (aligned
    16-bit products), by the library's launch rule: on the 16x16x32 path (Kb % 128 == 0)
    the persistent kernel when the tiles left after the split-K tail exceed one round
    (CUs rounded down to a multiple of 8), Kb >= 256 and a leaf's products fit 32-bit
    offsets; else one workgroup per tile; the 32x32x16 kernel for other Kb. A last tile
    row of at most 16 rows goes to fastmm::thin::thin_rows_kernel when that takes the
    256x256 tiles down a round and R * Nb <= 32768."""
    if kb % 128:
        return f"fastmm::fast::leaf_gemm_kernel<{compute}, {compute}> (fastmm_leaf_products)"
    tiles_n = -(-nb // 256)
    with_row = rank * -(-mb // 256) * tiles_n
    thin = (mb > 256 and 0 < mb % 256 <= 16 and rank * nb <= 32768
            and -(-(with_row - rank * tiles_n) // cus) < -(-with_row // cus))
    tiles = with_row - rank * tiles_n if thin else with_row
    tail = tiles % cus
    split = min(8, kb // 128, 3 * cus // (4 * tail)) if tail else 0
    main = tiles - tail if split_tail and split >= 2 else tiles
    extra = " + thin_rows_kernel for the last tile row" if thin else ""
    if main > cus // 8 * 8 and kb >= 256 and mb * nb * 2 <= 2**31 - 1:
        return f"fastmm::mfma16::persistent_kernel<{compute}, {compute}> (fastmm_leaf_products){extra}"
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


def cpu_baseline(cfg: dict, x, w, b, budget_s: float) -> dict:
    """Time the CPU oracle on a row sample of the workload; TFLOP/s of that sample."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import fastmm_oracle as O

    cores = min(16, os.cpu_count() or 1)
    scheme = O.load_oracle_scheme(cfg["scheme"])
    rows = 256
    xs = x[:rows].float().numpy()
    wn = w.float().numpy()
    bn = None if b is None else b.float().numpy()
    with threadpool_limits(limits=cores):
        blas_threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
        mm = bool(cfg.get("mm"))
        transform = O.right_transform if mm else O.weight_transform  # mm: w is right[K, N]
        columns = wn.shape[1] if mm else wn.shape[0]
        packed = transform(scheme, wn) if cfg["prepacked"] else None

        def one() -> None:
            a = O.left_transform(scheme, xs)
            bt = packed if packed is not None else transform(scheme, wn)
            p = O.leaf_products(a, bt, product_dtype="fp16", accumulate="f32")
            O.reconstruct(scheme, p, rows, columns, bn, "fp16" if mm else "bf16")

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
            f"{rows} of {cfg['rows']} rows ({cfg['scheme']}, "
            f"{'prepacked weight' if cfg['prepacked'] else 'weight transformed per call'}), "
            f"fp32 BLAS leaf sums, median of {len(times)} runs, {seconds * 1e3:.0f} ms each"
        ),
    }


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", default="c2", choices=sorted(CONFIGS))
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

    from rdna3_fastmm.runtime import PLAN_TYPES, Rank343Plan, operand_shape

    cfg = CONFIGS[args.config]
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
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
    workspace = plan.allocate_workspace(prepacked_right=cfg["prepacked"])
    if mm:
        packed = plan.pack_right(w)
    else:
        packed = plan.pack_weight(w) if cfg["prepacked"] else None
    out = torch.empty((m, n), device=device, dtype=io_dtype) if cfg["prepacked"] else None
    native_out = torch.empty((m, n), device=device, dtype=io_dtype)

    if mm:
        def step():
            plan.run_packed(x, packed, workspace, out)

        def native():
            torch.mm(x, w, out=native_out)
    elif cfg["prepacked"]:
        def step():
            plan.run_linear_packed(x, packed, workspace, b, out)

        def native():
            if b is None:
                torch.mm(x, w.T, out=native_out)
            else:
                torch.addmm(b, x, w.T, out=native_out)
    else:
        def step():
            plan.run_linear(x, w, workspace, b)

        def native():
            torch.nn.functional.linear(x, w, b)

    if args.traffic_calibration:
        source = torch.empty(1 << 29, device=device, dtype=torch.float16)
        target = torch.empty_like(source)
        for _ in range(3):
            target.copy_(source)
        torch.cuda.synchronize()
        del source, target
    for _ in range(args.warmup):
        step()
        native()
    ms = _time_region(step, args.steps)
    native_ms = _time_region(native, args.steps)

    # Per-stage HIP-event timing (same stream as the launches).
    shape = plan.shape
    stages = {
        "left_transform": lambda: plan._transform_left(x, workspace.left_transformed),
        "leaf_products": lambda: plan._leaf_products(
            workspace.left_transformed,
            packed.transformed if packed is not None else workspace.right_transformed,
            workspace.products,
            workspace.leaf_scratch,
        ),
        "reconstruct": lambda: plan._reconstruct(workspace.products, b, native_out),
    }
    if not cfg["prepacked"]:
        stages["weight_transform"] = lambda: plan._transform_weight(w, workspace.right_transformed)
    stage_ms = {name: _median(_event_ms(fn, 10)) for name, fn in stages.items()}
    leaf_flops = 2.0 * plan.rank * shape.block_rows * shape.block_inner * shape.block_columns
    leaf_tflops = leaf_flops / (stage_ms["leaf_products"] * 1e-3) / 1e12
    packing_buffer = workspace.products.new_empty(operand_shape(plan.rank, shape.block_columns, shape.block_inner))
    pack = (lambda: plan._transform_right(w, packing_buffer)) if mm else (
        lambda: plan._transform_weight(w, packing_buffer))
    pack_ms = _median(_event_ms(pack, 3))
    del packing_buffer

    # Accuracy on this workload (outside the timed region).
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
    native()
    native_err = float(torch.linalg.vector_norm(native_out.double() - exact) / norm) if cfg["prepacked"] else float(
        torch.linalg.vector_norm(torch.nn.functional.linear(x, w, b).double() - exact) / norm)
    err = float(torch.linalg.vector_norm(result.double() - exact) / norm)
    nonfinite = int((~torch.isfinite(result)).sum())
    del exact

    line = {
        "metric": METRIC,
        "value": round(flops / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{'fp16' if mm else 'bf16'} in/out, {'bf16' if compute == torch.bfloat16 else 'fp16'} MFMA leaves, "
                 "fp32 accumulate",
        "data": "synthetic (seeded CPU torch.Generator: x~N(0,1), W~N(0,1/K), bias~N(0,0.02))",
        "config": {
            "workload": cfg["name"],
            "scheme": cfg["scheme"],
            "rows": m,
            "inner": k,
            "columns": n,
            "bias": cfg["bias"],
            "prepacked_weight": cfg["prepacked"],
            "parallelism": "single GPU",
        },
        "native_bf16": {
            "ms_per_step": round(native_ms, 4),
            "tflops": round(flops / (native_ms * 1e-3) / 1e12, 2),
            "op": "torch.mm(left, right, out=) fp16" if mm
            else ("torch.addmm(bias, x, W.T, out=)" if b is not None else "torch.mm(x, W.T, out=)")
            if cfg["prepacked"]
            else "torch.nn.functional.linear",
            "blas": str(torch.backends.cuda.preferred_blas_library()),
            "TORCH_BLAS_PREFER_HIPBLASLT": os.environ.get("TORCH_BLAS_PREFER_HIPBLASLT"),
        },
        "speedup_vs_native": round(native_ms / ms, 4),
        "accuracy": {
            "rel_l2": err,
            "native_rel_l2": native_err,
            "error_ratio": round(err / native_err, 4),
            # Linear: the north-star 1.2x native BF16 error; FP16 mm: the reference's
            # rel-L2 < 5e-3 (native FP16 rounds only its output, so a ratio bound is moot)
            "bound": "rel_l2 < 5e-3" if mm else 1.2,
            "nonfinite": nonfinite,
        },
        "stages_ms": {name: round(v, 4) for name, v in stage_ms.items()},
        "packing_ms": round(pack_ms, 4),
        "roofline": {
            "kernel": leaf_kernel_name(
                plan.rank, shape.block_rows, shape.block_inner, shape.block_columns,
                "bf16" if compute == torch.bfloat16 else "fp16",
                torch.cuda.get_device_properties(device).multi_processor_count, workspace.leaf_scratch is not None,
            )
            + (" + split-K tail (kPartial parts + tail_reduce_kernel) where the plan splits;"
               " timed as the whole stage" if workspace.leaf_scratch is not None else ""),
            "bound": "mfma",
            "achieved": round(leaf_tflops, 2),
            "peak": MFMA_16BIT_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(leaf_tflops / MFMA_16BIT_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(args.config),
            "work_per_launch": f"2*R*Mb*Kb*Nb = {leaf_flops:.4e} flop",
        },
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, x_cpu, w_cpu, b_cpu, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
