"""Leaf-stage benchmark: the batched products alone, on chosen operand data.

``python -m rdna3_fastmm.leafbench --shape R,Mb,Kb,Nb [--data KIND ...] [--bmm]``
times ``fastmm_leaf_products`` (with its split-K scratch) on R leaves of
``[Mb, Kb] @ [Kb, Nb]`` and, with ``--bmm``, the library GEMMs the reference
would call on the same problem: ``torch.bmm`` in FP16 and in BF16. One JSON
line per (kernel, data) with the median of ``--reps`` HIP-event timings.

The operand data matters on MI355X: MFMA throughput under the board's power
and current limits depends on how many operand bits toggle. ``--data``:

* ``zeros``: all-zero operands (the cheapest the MFMA pipes can run);
* ``bf16``: N(0,1) values rounded to BF16 (8 significant bits), stored in the
  operand type, like the BF16 inputs a rank-7 plane copies;
* ``fp16``: N(0,1) values with full 11-bit FP16 significands, like planes
  that are sums or scaled sums of inputs.

Run it under ``rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES ...`` to
see achieved clock and MFMA-busy cycles per data kind.
"""

from __future__ import annotations

import argparse
import json
import statistics

import torch

from . import _stages


def _operands(kind: str, shape: tuple[int, int, int, int], dtype: torch.dtype, device: torch.device, seed: int):
    rank, mb, kb, nb = shape
    if kind == "zeros":
        return (torch.zeros((rank, mb, kb), device=device, dtype=dtype),
                torch.zeros((rank, nb, kb), device=device, dtype=dtype))
    g = torch.Generator(device=device).manual_seed(seed)
    a = torch.randn((rank, mb, kb), generator=g, device=device)
    b = torch.randn((rank, nb, kb), generator=g, device=device) / kb**0.5
    if kind == "bf16":
        a, b = a.to(torch.bfloat16), b.to(torch.bfloat16)
    elif kind != "fp16":
        raise ValueError(f"unknown data kind {kind!r}")
    return a.to(dtype), b.to(dtype)


def _median_ms(fn, reps: int, warmups: int = 3) -> float:
    for _ in range(warmups):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
    return statistics.median(times)


def run(shape: tuple[int, int, int, int], kinds: list[str], reps: int, bmm: bool, device: torch.device) -> list[dict]:
    rank, mb, kb, nb = shape
    flops = 2.0 * rank * mb * kb * nb
    records = []
    scratch_bytes = _stages.leaf_scratch_bytes(rank, torch.float16, torch.float16, mb, kb, nb, device)
    scratch = torch.empty(scratch_bytes, device=device, dtype=torch.uint8) if scratch_bytes else None
    for kind in kinds:
        a, b = _operands(kind, shape, torch.float16, device, seed=1)
        p = torch.empty((rank, mb, nb), device=device, dtype=torch.float16)

        def leaf():
            _stages.leaf_products(rank, a, b, p, mb, kb, nb, scratch)

        kernels = {"fastmm_leaf_products fp16": leaf}
        if bmm:
            bt = b.transpose(1, 2).contiguous()
            a16, b16 = a.to(torch.bfloat16), bt.to(torch.bfloat16)
            kernels["torch.bmm fp16"] = lambda: torch.bmm(a, bt, out=p)
            kernels["torch.bmm bf16"] = lambda: torch.bmm(a16, b16)
        for name, fn in kernels.items():
            ms = _median_ms(fn, reps)
            records.append({"kernel": name, "data": kind, "shape": list(shape), "ms": round(ms, 4),
                            "tflops": round(flops / (ms * 1e-3) / 1e12, 1)})
    return records


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--shape", required=True, help="R,Mb,Kb,Nb")
    parser.add_argument("--data", action="append", choices=("zeros", "bf16", "fp16"))
    parser.add_argument("--reps", type=int, default=15)
    parser.add_argument("--bmm", action="store_true", help="also time torch.bmm in FP16 and BF16")
    args = parser.parse_args()
    shape = tuple(int(v) for v in args.shape.split(","))
    if len(shape) != 4 or min(shape) < 1:
        parser.error("--shape needs four positive integers R,Mb,Kb,Nb")
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    for record in run(shape, args.data or ["zeros", "bf16", "fp16"], args.reps, args.bmm, device):
        print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
