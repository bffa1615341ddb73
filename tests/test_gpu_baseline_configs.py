"""Every BASELINE configuration at its full size, through the HIP library.

The reference validates each benchmark run on a centred CPU-FP32 tile in every
one of the s*s output macroblocks (benchmarks/benchmark.py:160-265) and tests
its plans end to end on ragged shapes (tests/test_rdna3.py:433-613). Here each
configuration (C1..C5 of the BASELINE file, the C5 controls, and the north
star's rank-48 point at 8214 x 12288 x 4608) runs on its own seeded inputs
(CPU generator: x ~ N(0,1), W ~ N(0,1/K), bias ~ N(0, 0.02), all BF16), and:

* the transformed planes A' and B' are bit-exact against the oracle on a
  sample of block rows / block columns (first, last, tile edges, padding rows,
  random), computed by the oracle from just the input rows those planes read;
* the leaf products on that row x column sample stay within the fp32
  accumulation bound of the oracle's near-exact sums (plus one fp16 rounding);
* the output at those positions, in every output macroblock, is bit-equal to
  the oracle's recombination (+ bias, one BF16 rounding) of the GPU's own
  products;
* the dynamic and the prepacked plan agree bitwise over the whole output, the
  packed weight equals the dynamic B', and a reused output buffer gives the
  same bits again;
* no value is non-finite, and the full-output relative L2 error against an
  fp64 product is at most 1.2x native BF16 F.linear's (rank 49: inside the
  band its fp16 operand rounding puts it in, above the bound, as the oracle
  predicts);
* the reference's per-macroblock centred tiles against a CPU fp32 product
  stay below its rel-L2 5e-3 bound.

C1 (1024^3, rank 7) is small enough to check against the oracle's whole
evaluation. The same checks run on open-model MLP down projections at row counts
inside families of the shipped dispatch table (the shapes the Linear rewrite
sends to the plans).
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from _parity import baseline_inputs, check_sampled_stages, gather_plane_rows, rel_l2
from oracle import fastmm_oracle as O
from rdna3_fastmm.runtime import PLAN_TYPES

pytestmark = pytest.mark.gpu
DEVICE = torch.device("cuda", 0)
TILE = 16  # centred tile per output macroblock (the reference uses 8..32)

# id: (scheme, rows, inner, columns, bias)
CONFIGS = {
    "C1-rank7-1024": ("rank7", 1024, 1024, 1024, False),
    "C2-rank7-4096x4096x12288": ("rank7", 4096, 4096, 12288, False),
    "C3-rank7-8214x12288x4608-bias": ("rank7", 8214, 12288, 4608, True),
    "C4-rank49-19968x4096x16384-bias": ("rank49", 19968, 4096, 16384, True),
    "C5-rank48-8192": ("rank48", 8192, 8192, 8192, False),
    "C5-control-rank7-8192": ("rank7", 8192, 8192, 8192, False),
    "C5-control-rank49-8192": ("rank49", 8192, 8192, 8192, False),
    "target-rank48-8214x12288x4608": ("rank48", 8214, 12288, 4608, False),
}
# open-model down projections (rows, K -> N) inside measured prepacked families
MODEL_SHAPES = {
    "Qwen2.5-32B-down-8192-rank7": ("rank7", 8192, 27648, 5120, False),
    "Qwen2.5-32B-down-8192-rank48": ("rank48", 8192, 27648, 5120, False),
    "Mistral-Nemo-12B-down-5000-rank7": ("rank7", 5000, 14336, 5120, False),
    "Gemma-2-9B-down-7500-rank48": ("rank48", 7500, 14336, 3584, False),
    "Qwen2.5-7B-down-12000-rank7": ("rank7", 12000, 18944, 3584, False),
    "Qwen3-32B-down-6000-rank48": ("rank48", 6000, 25600, 5120, False),
    "Yi-34B-down-4100-rank7": ("rank7", 4100, 20480, 7168, False),  # Mb = 2050: a 2-row strip
}
# Rank 49's fp16 planes alone cost ~1.4x native BF16's error (the oracle's
# prediction; measured 1.67x with fp16 products), beyond the 1.2x bound.
RANK49_BAND = (1.2, 1.9)
ERROR_RATIO_BOUND = 1.2


def macroblock_tile_errors(plan, x, w, b, output) -> list[float]:
    """reference benchmark.py:160-265: a centred tile per macroblock vs CPU fp32."""
    s = plan.scheme_size
    m, k, n = plan.shape.dimensions
    errors = []
    for br in range(s):
        r0 = br * plan.shape.block_rows
        r1 = min(r0 + plan.shape.block_rows, m)
        rs = r0 + (r1 - r0 - TILE) // 2
        for bc in range(s):
            c0 = bc * plan.shape.block_columns
            c1 = min(c0 + plan.shape.block_columns, n)
            cs = c0 + (c1 - c0 - TILE) // 2
            reference = x[rs:rs + TILE].float() @ w[cs:cs + TILE].float().T
            if b is not None:
                reference += b[cs:cs + TILE].float()
            candidate = output[rs:rs + TILE, cs:cs + TILE].float().cpu()
            assert torch.isfinite(candidate).all()
            errors.append(float(torch.linalg.vector_norm(candidate - reference) / torch.linalg.vector_norm(reference)))
    return errors


@pytest.mark.parametrize("config", list(CONFIGS) + list(MODEL_SHAPES))
def test_baseline_config_through_the_hip_path(config: str) -> None:
    key, m, k, n, has_bias = {**CONFIGS, **MODEL_SHAPES}[config]
    print(f"\n[case] {config}: {key} {m}x{k}x{n} bias={has_bias}", flush=True)
    torch.cuda.empty_cache()
    rng = np.random.default_rng(zlib.crc32(config.encode()))
    x_cpu, w_cpu, b_cpu = baseline_inputs(m, k, n, has_bias)
    x, w = x_cpu.to(DEVICE), w_cpu.to(DEVICE)
    b = None if b_cpu is None else b_cpu.to(DEVICE)
    plan = PLAN_TYPES[key](m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    scheme = O.load_oracle_scheme(key)

    workspace = plan.allocate_workspace()
    dynamic = plan.run_linear(x, w, workspace, b)  # output allocated per call
    torch.cuda.synchronize()
    check_sampled_stages(plan, scheme, x_cpu, w_cpu, b_cpu, workspace, dynamic, rng)

    packed = plan.pack_weight(w)
    assert torch.equal(packed.transformed, workspace.right_transformed)
    packed_workspace = plan.allocate_workspace(prepacked_right=True)
    out = torch.empty((m, n), device=DEVICE, dtype=torch.bfloat16)
    first = plan.run_linear_packed(x, packed, packed_workspace, b, out)
    assert first.data_ptr() == out.data_ptr()
    assert torch.equal(first, dynamic), "prepacked output differs from the dynamic one"
    snapshot = first.clone()
    assert torch.equal(plan.run_linear_packed(x, packed, packed_workspace, b, out), snapshot)
    del packed_workspace, snapshot, first

    assert int((~torch.isfinite(dynamic)).sum()) == 0
    exact = x.double() @ w.double().T
    if b is not None:
        exact += b.double()
    native = rel_l2(torch.nn.functional.linear(x, w, b), exact)
    ratio = rel_l2(dynamic, exact) / native
    del exact
    tiles = macroblock_tile_errors(plan, x_cpu, w_cpu, b_cpu, dynamic)
    print(f"[ratio] {config}: native rel-L2 {native:.3e}, error ratio {ratio:.4f}, "
          f"macroblock tiles max rel-L2 {max(tiles):.2e}", flush=True)
    assert max(tiles) < 5e-3
    if key == "rank49":
        assert RANK49_BAND[0] < ratio < RANK49_BAND[1]
    else:
        assert ratio <= ERROR_RATIO_BOUND


def test_c1_matches_the_whole_oracle_evaluation() -> None:
    """C1 (rank 7, 1024^3): every plane bit-exact, every product within the bound,
    the output bit-equal to the oracle's recombination of the GPU's products and
    within one product rounding of the oracle's own end-to-end evaluation."""
    print("\n[case] C1 full oracle 1024^3", flush=True)
    m = k = n = 1024
    x_cpu, w_cpu, _ = baseline_inputs(m, k, n, False)
    plan = PLAN_TYPES["rank7"](m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    workspace = plan.allocate_workspace()
    out = plan.run_linear(x_cpu.to(DEVICE), w_cpu.to(DEVICE), workspace).cpu()
    scheme = O.load_oracle_scheme("rank7")
    xn, wn = x_cpu.float().numpy(), w_cpu.float().numpy()
    a = O.left_transform(scheme, xn)
    bt = O.weight_transform(scheme, wn)
    rank, mb, kb = a.shape
    nb = bt.shape[1]
    everything = np.arange(mb)
    assert np.array_equal(gather_plane_rows(workspace.left_transformed, rank, mb, kb, everything), a.view(np.int16))
    assert np.array_equal(gather_plane_rows(workspace.right_transformed, rank, nb, kb, np.arange(nb)),
                          bt.view(np.int16))
    products = workspace.products.cpu().numpy()
    exact = O.leaf_products(a, bt, product_dtype="fp32").astype(np.float64)
    magnitude = np.matmul(np.abs(a.astype(np.float64)), np.abs(np.swapaxes(bt.astype(np.float64), 1, 2)))
    bound = kb * 2.0**-24 * magnitude + np.abs(exact) * 2.0**-11 + 2.0**-24
    assert np.all(np.abs(products.astype(np.float64) - exact) <= bound)
    assert np.array_equal(out.view(torch.int16).numpy(), O.reconstruct(scheme, products, m, n).view(np.int16))
    # the oracle's own evaluation (near-exact leaf sums): products may differ by one
    # fp16 rounding where the fp32 sum sits at a rounding boundary
    whole = O.bf16_bits_to_f32(O.linear(scheme, xn, wn))
    got = out.float().numpy()
    reference = xn.astype(np.float64) @ wn.astype(np.float64).T
    oracle_error = np.linalg.norm(whole - reference)
    assert np.linalg.norm(got - whole) <= 0.1 * oracle_error
    assert np.mean(got != whole) < 0.01


def test_c4_rank49_bf16_leaves_at_full_size() -> None:
    """The reference's rank-49 (bf16, bf16) precision pair (runtime.py:852-858) at C4's
    size: BF16 planes bit-exact, BF16-MFMA products within their bound, the output
    bit-equal to the oracle's recombination of the GPU's products, dynamic ==
    prepacked. Its error is far above the 1.2x bound (BF16 planes round the
    transformed sums to 8 bits), which is the pair's nature, asserted as a band."""
    m, k, n = 19968, 4096, 16384
    print(f"\n[case] C4 rank49 bf16 leaves {m}x{k}x{n}", flush=True)
    torch.cuda.empty_cache()
    x_cpu, w_cpu, b_cpu = baseline_inputs(m, k, n, True)
    x, w, b = x_cpu.to(DEVICE), w_cpu.to(DEVICE), b_cpu.to(DEVICE)
    plan = PLAN_TYPES["rank49"](m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.bfloat16)
    workspace = plan.allocate_workspace()
    assert workspace.products.dtype == torch.bfloat16
    dynamic = plan.run_linear(x, w, workspace, b)
    torch.cuda.synchronize()
    check_sampled_stages(plan, O.load_oracle_scheme("rank49"), x_cpu, w_cpu, b_cpu, workspace, dynamic,
                         np.random.default_rng(49), plane="bf16")
    packed_workspace = plan.allocate_workspace(prepacked_right=True)
    assert torch.equal(plan.run_linear_packed(x, plan.pack_weight(w), packed_workspace, b), dynamic)
    del packed_workspace, workspace
    assert int((~torch.isfinite(dynamic)).sum()) == 0
    exact = x.double() @ w.double().T + b.double()
    ratio = rel_l2(dynamic, exact) / rel_l2(torch.nn.functional.linear(x, w, b), exact)
    print(f"[ratio] C4 rank49 bf16 leaves: error ratio {ratio:.2f}", flush=True)
    assert 5.0 < ratio < 20.0
