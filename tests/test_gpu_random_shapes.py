"""Seeded random and kernel-threshold shapes through every Linear plan (GPU).

The launcher picks the leaf kernel from the block shape: the register-staged
generic kernel (ragged Kb or Nb), the 32x32x16 kernel (Kb % 32 == 0, Kb >= 96),
the 16x16x32 kernels (Kb % 128 == 0; persistent beyond one round of tiles), a
last tile row of at most 16 rows (fused into the persistent kernel as a strip, or
the thin last-row kernel) and the split-K tail;
the transforms pick a vector or a scalar path. These shapes cross those
thresholds for each scheme, plus a seeded random sample. Every case runs the
dynamic plan, checks its stages against the oracle on a sample of block rows and
columns that includes every ragged edge (A'/B' bit-exact, products within the
fp32-accumulation bound, output bits equal to the oracle's recombination of the
GPU's products), and checks that the prepacked plan gives the same bits. Small
cases compare the whole output with the oracle's recombination.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import baseline_inputs, check_sampled_stages
from oracle import fastmm_oracle as O
from rdna3_fastmm.runtime import PLAN_TYPES

pytestmark = pytest.mark.gpu
DEVICE = torch.device("cuda", 0)


def _threshold_shapes(key: str) -> list[tuple[int, int, int]]:
    s = PLAN_TYPES[key].scheme_size
    shapes = [
        (1, 4096, 4096),  # one row (decode), Mb = 1
        (s * 64, s * 96, s * 64),  # Kb = 96: the 32x32x16 kernel's smallest K
        (s * 128, s * 128, s * 128),  # Kb = 128: the 16x16x32 kernel, one round
        (s * 50 - 1, s * 160, s * 37 + 1),  # Nb % 8 != 0: the generic kernel, padding everywhere
        (s * 300 + 1, s * 33, s * 70 - 3),  # Kb odd: row-major planes, scalar transforms
    ]
    # a last tile row of 11 rows that the thin kernel takes (rank x Nb <= 32768, and
    # dropping the row saves a round of 256 x 256 tiles)
    shapes.append({"rank7": (534, 512, 9360), "rank48": (1068, 1024, 2720), "rank49": (1068, 1024, 2656)}[key])
    # the north star's M = 8214 with a short K: a last tile row of 11 (rank 7) or 6
    # (rank 48/49) rows below a last group of 8 tile rows, fused into the persistent
    # kernel as a strip
    shapes.append((8214, 256 * s, 4608))
    return shapes


def _random_shapes(count: int = 12) -> list[tuple[int, int, int]]:
    rng = np.random.default_rng(2026)
    return [tuple(int(v) for v in rng.integers(1, 601, size=3)) for _ in range(count)]


CASES = [(key, shape) for key in ("rank7", "rank48", "rank49") for shape in _threshold_shapes(key) + _random_shapes()]


@pytest.mark.parametrize("key, shape", CASES, ids=[f"{k}-{m}x{n_}x{c}" for k, (m, n_, c) in CASES])
def test_plan_matches_the_oracle(key: str, shape: tuple[int, int, int]) -> None:
    m, k, n = shape
    with_bias = (m + k + n) % 2 == 0
    print(f"\n[case] {key} {m}x{k}x{n} bias={with_bias}", flush=True)
    x_cpu, w_cpu, b_cpu = baseline_inputs(m, k, n, with_bias, seed=m * 7 + k * 3 + n)
    x, w = x_cpu.to(DEVICE), w_cpu.to(DEVICE)
    b = None if b_cpu is None else b_cpu.to(DEVICE)
    plan = PLAN_TYPES[key](m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    scheme = O.load_oracle_scheme(key)
    workspace = plan.allocate_workspace(max_free_memory_fraction=0.5)
    dynamic = plan.run_linear(x, w, workspace, b)
    torch.cuda.synchronize()
    check_sampled_stages(plan, scheme, x_cpu, w_cpu, b_cpu, workspace, dynamic, np.random.default_rng(m + n))
    if plan.rank * plan.shape.block_rows * plan.shape.block_columns <= 8_000_000:
        # the whole output against the oracle's recombination of the GPU's products
        recombined = O.reconstruct(scheme, workspace.products.cpu().numpy(), m, n,
                                   None if b_cpu is None else b_cpu.float().numpy(), "bf16")
        assert np.array_equal(dynamic.cpu().view(torch.int16).numpy(), recombined.view(np.int16))
    packed_workspace = plan.allocate_workspace(max_free_memory_fraction=0.5, prepacked_right=True)
    assert torch.equal(plan.run_linear_packed(x, plan.pack_weight(w), packed_workspace, b), dynamic)
    assert torch.isfinite(dynamic).all()
