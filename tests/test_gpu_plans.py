"""Plans and operators end to end on the GPU (the reference's GPU tests, ported).

Sources (reference repository): tests/test_rdna3.py:406-709. Tolerances are
written next to each assertion; the headline bound is the north star's:
rel-L2 vs an fp64 product no worse than 1.2x native BF16 torch.mm's, and no
non-finite values.
"""

import numpy as np
import pytest
import torch

from _layout import from_operand
from oracle import fastmm_oracle as O
from rdna3_fastmm.linear import rdna3_linear, rdna3_rank7_linear, rdna3_rank48_linear
from rdna3_fastmm.runtime import PLAN_TYPES, Rank7Plan, Rank48Plan, Rank49Plan

pytestmark = pytest.mark.gpu
DEVICE = torch.device("cuda", 0)
LINEAR_PLANS = (Rank7Plan, Rank48Plan, Rank49Plan)


def _rel(candidate: torch.Tensor, reference: torch.Tensor) -> float:
    return float(torch.linalg.vector_norm(candidate.double() - reference) / torch.linalg.vector_norm(reference))


@pytest.mark.parametrize("plan_type", (Rank7Plan, Rank49Plan))
def test_dynamic_and_packed_match_exact_small_product(plan_type) -> None:
    """reference test_rdna3.py:406-430 (fp16 mm path)."""
    print(f"\n[case] exact small product {plan_type.__name__}", flush=True)
    torch.manual_seed(11)
    shape = (5, 6, 7)
    left = torch.randint(-2, 3, shape[:2], device=DEVICE, dtype=torch.float16)
    right = torch.randint(-2, 3, shape[1:], device=DEVICE, dtype=torch.float16)
    reference = (left.float() @ right.float()).half()
    plan = plan_type(*shape, device=DEVICE)
    dynamic_workspace = plan.allocate_workspace(max_free_memory_fraction=0.1)
    packed = plan.pack_right(right, max_free_memory_fraction=0.1)
    packed_workspace = plan.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    for _ in range(3):
        assert torch.equal(plan.run(left, right, dynamic_workspace), reference)
        assert torch.equal(plan.run_packed(left, packed, packed_workspace), reference)
    packed_result = plan.run_packed(left, packed, packed_workspace).clone()
    right.zero_()
    assert torch.equal(plan.run_packed(left, packed, packed_workspace), packed_result)
    r = plan.rank
    s = plan.scheme_size
    mb, kb, nb = -(-5 // s), -(-6 // s), -(-7 // s)
    assert plan.workspace_bytes == r * (mb * kb + kb * nb + mb * nb) * 2
    assert plan.prepacked_workspace_bytes == r * (mb * kb + mb * nb) * 2
    assert plan.packed_right_bytes == r * kb * nb * 2


@pytest.mark.parametrize("plan_type", LINEAR_PLANS)
@pytest.mark.parametrize("shape", ((5, 6, 7), (17, 19, 23), (64, 72, 80), (131, 96, 70)))
def test_linear_exact_small_integer_product(plan_type, shape) -> None:
    """BF16 Linear path: small integers are exact through every stage."""
    print(f"\n[case] exact linear {plan_type.__name__} {shape}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    m, k, n = shape
    x = torch.randint(-2, 3, (m, k), generator=g).to(torch.bfloat16).to(DEVICE)
    w = torch.randint(-2, 3, (n, k), generator=g).to(torch.bfloat16).to(DEVICE)
    bias = torch.randint(-3, 4, (n,), generator=g).to(torch.bfloat16).to(DEVICE)
    reference = (x.float() @ w.float().T + bias.float()).to(torch.bfloat16)
    plan = plan_type(m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    workspace = plan.allocate_workspace(max_free_memory_fraction=0.1)
    assert torch.equal(plan.run_linear(x, w, workspace, bias), reference)
    packed = plan.pack_weight(w, max_free_memory_fraction=0.1)
    packed_workspace = plan.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    assert torch.equal(plan.run_linear_packed(x, packed, packed_workspace, bias), reference)


@pytest.mark.parametrize("plan_type", LINEAR_PLANS)
@pytest.mark.parametrize(
    "shape",
    (
        (257, 263, 269),  # ragged blocks, row-major operands, generic leaf kernel
        (200, 512, 544),  # Kb % 128 == 0: K-slab operands and the 16x16x32 leaf kernel
    ),
)
def test_linear_matches_oracle_and_bounded_error(plan_type, shape) -> None:
    """reference test_rdna3.py:487-613 at 257x263x269, plus the stage-by-stage oracle check.

    After a dynamic run the workspace holds every intermediate, so each stage
    is pinned on its own: A' and B' bit-exact, the products within the fp32
    accumulation bound of the oracle's near-exact leaf sums (plus one fp16
    rounding), and the output bit-exact to the oracle's recombination of the
    GPU's own products.
    """
    print(f"\n[case] bounded error {plan_type.__name__} {shape}", flush=True)
    g = torch.Generator().manual_seed(17)
    x = torch.randn(shape[:2], generator=g).to(torch.bfloat16)
    w = torch.randn((shape[2], shape[1]), generator=g).to(torch.bfloat16)
    bias = torch.randn(shape[2], generator=g).to(torch.bfloat16)
    xg, wg, bg = x.to(DEVICE), w.to(DEVICE), bias.to(DEVICE)
    reference = xg.double() @ wg.double().T + bg.double()
    plan = plan_type(*shape, device=DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    workspace = plan.allocate_workspace(max_free_memory_fraction=0.1)
    dynamic = plan.run_linear(xg, wg, workspace, bg)
    torch.cuda.synchronize()
    oracle = O.load_oracle_scheme(plan.scheme_key)
    a = O.left_transform(oracle, x.float().numpy())
    b = O.weight_transform(oracle, w.float().numpy())
    rank, mb, kb = a.shape
    nb = b.shape[1]
    left_bits = workspace.left_transformed.cpu().numpy().view(np.int16)
    right_bits = workspace.right_transformed.cpu().numpy().view(np.int16)
    assert np.array_equal(from_operand(left_bits, rank, mb, kb), a.view(np.int16))
    assert np.array_equal(from_operand(right_bits, rank, nb, kb), b.view(np.int16))
    products = workspace.products.cpu().numpy()
    exact = O.leaf_products(a, b, product_dtype="fp32").astype(np.float64)
    magnitude = np.matmul(np.abs(a.astype(np.float64)), np.abs(np.swapaxes(b.astype(np.float64), 1, 2)))
    bound = a.shape[2] * 2.0**-24 * magnitude + np.abs(exact) * 2.0**-11 + 2.0**-24
    assert np.all(np.abs(products.astype(np.float64) - exact) <= bound)
    recombined = O.reconstruct(oracle, products, shape[0], shape[2], bias.float().numpy(), "bf16")
    assert np.array_equal(dynamic.cpu().view(torch.int16).numpy(), recombined.view(np.int16))

    packed_weight = plan.pack_weight(wg, max_free_memory_fraction=0.1)
    packed_workspace = plan.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    packed = plan.run_linear_packed(xg, packed_weight, packed_workspace, bg)
    assert torch.isfinite(dynamic).all()
    assert _rel(dynamic, reference) < 0.005
    assert torch.equal(dynamic, packed)
    # packed snapshot independent of later weight mutation (test_rdna3.py:563-573)
    snapshot = packed.clone()
    wg.zero_()
    assert torch.equal(plan.run_linear_packed(xg, packed_weight, packed_workspace, bg), snapshot)
    assert packed_weight.source_shape == (shape[2], shape[1])
    assert packed_workspace.right_transformed is None
    assert plan.packed_weight_bytes == plan.packed_right_bytes


@pytest.mark.parametrize("shape", ((5, 6, 7), (257, 263, 269), (200, 512, 544)))
def test_rank49_bf16_leaves_match_oracle_stage_by_stage(shape) -> None:
    """The reference's (bf16, bf16) rank-49 pair (runtime.py:852-858): BF16 planes,
    BF16 MFMA leaves and BF16 products, each stage pinned against the oracle."""
    print(f"\n[case] rank49 bf16 leaves {shape}", flush=True)
    g = torch.Generator().manual_seed(41)
    m, k, n = shape
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = torch.randn((n, k), generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    xg, wg, bg = x.to(DEVICE), w.to(DEVICE), bias.to(DEVICE)
    plan = Rank49Plan(*shape, device=DEVICE, dtype=torch.bfloat16, compute_dtype=torch.bfloat16)
    workspace = plan.allocate_workspace(max_free_memory_fraction=0.1)
    assert workspace.products.dtype == torch.bfloat16
    dynamic = plan.run_linear(xg, wg, workspace, bg)
    torch.cuda.synchronize()
    oracle = O.load_oracle_scheme("rank49")
    a = O.left_transform(oracle, x.float().numpy(), "bf16")
    b = O.weight_transform(oracle, w.float().numpy(), "bf16")
    rank, mb, kb = a.shape
    nb = b.shape[1]
    left_bits = from_operand(workspace.left_transformed.cpu().view(torch.int16).numpy(), rank, mb, kb)
    right_bits = from_operand(workspace.right_transformed.cpu().view(torch.int16).numpy(), rank, nb, kb)
    assert np.array_equal(left_bits, O.round_to_bf16(a).view(np.int16))
    assert np.array_equal(right_bits, O.round_to_bf16(b).view(np.int16))
    products = workspace.products.float().cpu().numpy().astype(np.float64)
    exact = O.leaf_products(a, b, product_dtype="fp32").astype(np.float64)
    magnitude = np.matmul(np.abs(a.astype(np.float64)), np.abs(np.swapaxes(b.astype(np.float64), 1, 2)))
    bound = kb * 2.0**-24 * magnitude + np.abs(exact) * 2.0**-8 + 2.0**-126
    assert np.all(np.abs(products - exact) <= bound)
    recombined = O.reconstruct(oracle, workspace.products.float().cpu().numpy(), m, n, bias.float().numpy(), "bf16")
    assert np.array_equal(dynamic.cpu().view(torch.int16).numpy(), recombined.view(np.int16))
    packed = plan.pack_weight(wg, max_free_memory_fraction=0.1)
    packed_ws = plan.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    assert torch.equal(plan.run_linear_packed(xg, packed, packed_ws, bg), dynamic)
    assert torch.isfinite(dynamic).all()


def test_packed_weight_reuses_across_rows_and_rejects_other_shape() -> None:
    """reference test_rdna3.py:616-677."""
    torch.manual_seed(37)
    weight = torch.randn((7, 6), device=DEVICE, dtype=torch.bfloat16)
    source_plan = Rank7Plan(5, 6, 7, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    packed_weight = source_plan.pack_weight(weight, max_free_memory_fraction=0.1)
    x = torch.randn((9, 6), device=DEVICE, dtype=torch.bfloat16)
    target = Rank7Plan(9, 6, 7, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    dynamic_ws = target.allocate_workspace(max_free_memory_fraction=0.1)
    packed_ws = target.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    assert torch.equal(target.run_linear(x, weight, dynamic_ws), target.run_linear_packed(x, packed_weight, packed_ws))
    other = Rank7Plan(9, 8, 7, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    other_ws = other.allocate_workspace(max_free_memory_fraction=0.1, prepacked_right=True)
    with pytest.raises(ValueError, match="packed Linear weight shape"):
        other.run_linear_packed(torch.randn((9, 8), device=DEVICE, dtype=torch.bfloat16), packed_weight, other_ws)


def test_plans_reject_bad_arguments_before_launch() -> None:
    plan = Rank7Plan(8, 8, 8, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    ws = plan.allocate_workspace(max_free_memory_fraction=0.1)
    x = torch.randn((8, 8), device=DEVICE, dtype=torch.bfloat16)
    w = torch.randn((8, 8), device=DEVICE, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="shape"):
        plan.run_linear(x[:4], w, ws)
    with pytest.raises(ValueError, match="dtype"):
        plan.run_linear(x.half(), w, ws)
    with pytest.raises(ValueError, match="contiguous"):
        plan.run_linear(x.t(), w, ws)
    with pytest.raises(ValueError, match="overlap"):
        plan.run_linear(x, w, ws, output=x)
    with pytest.raises(MemoryError):
        Rank7Plan(1 << 20, 1 << 16, 1 << 16, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16).allocate_workspace()
    with pytest.raises(ValueError, match="does not support"):
        Rank48Plan(8, 8, 8, DEVICE, dtype=torch.float16)


@pytest.mark.parametrize("op", (rdna3_linear, rdna3_rank7_linear, rdna3_rank48_linear))
def test_linear_ops_support_leading_dimensions(op) -> None:
    """reference test_rdna3.py:680-709."""
    torch.manual_seed(29)
    x = torch.randn((2, 17, 19), device=DEVICE, dtype=torch.bfloat16)
    w = torch.randn((23, 19), device=DEVICE, dtype=torch.bfloat16)
    b = torch.randn((23,), device=DEVICE, dtype=torch.bfloat16)
    reference = x.double() @ w.double().T + b.double()
    candidate = op(x, w, b)
    assert candidate.shape == (2, 17, 23)
    assert _rel(candidate, reference) < 0.005


# Allocating operator -> scheme key, and one shape per scheme whose leaf GEMM
# runs the split-K tail (every 256 x 256 tile in the last partial round, split
# in 2-3 K parts: rank 7 56 tiles, rank 48 96 tiles, rank 49 49 tiles).
OPERATOR_SCHEMES = (("linear_rank7", "rank7"), ("linear_rank48", "rank48"), ("linear", "rank49"))
SPLIT_TAIL_SHAPES = {"rank7": (2048, 1024, 1024), "rank48": (2048, 1024, 1024), "rank49": (1024, 1024, 1024)}


@pytest.mark.parametrize("op_name, key", OPERATOR_SCHEMES)
@pytest.mark.parametrize("case", ("ragged", "split_tail", "no_bias"))
def test_linear_ops_equal_the_plan_bitwise(op_name, key, case) -> None:
    """The allocating operators (own buffers, early frees, own split-K scratch) give
    exactly the plan's run_linear bits: leading dimensions, bias, a ragged shape and
    a shape whose leaf GEMM runs the split-K tail. reference linear.py:50-167,
    tests/test_rdna3.py:680-709."""
    from rdna3_fastmm import _stages

    if case == "ragged":
        lead, (k, n) = (2, 17), (19, 23)
    else:
        m, k, n = SPLIT_TAIL_SHAPES[key]
        lead = (2, m // 2)
    print(f"\n[case] op {op_name} {case} lead={lead} K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(53)
    x = torch.randn((*lead, k), generator=g).to(torch.bfloat16).to(DEVICE)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16).to(DEVICE)
    b = None if case == "no_bias" else (torch.randn((n,), generator=g) * 0.02).to(torch.bfloat16).to(DEVICE)
    rows = x.numel() // k
    plan = PLAN_TYPES[key](rows, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    if case != "ragged":
        shape = plan.shape
        assert _stages.leaf_scratch_bytes(plan.rank, torch.float16, torch.float16, shape.block_rows,
                                          shape.block_inner, shape.block_columns, DEVICE) > 0
    candidate = getattr(torch.ops.rdna3_fastmm, op_name)(x, w, b)
    assert candidate.shape == (*lead, n) and candidate.dtype == torch.bfloat16
    workspace = plan.allocate_workspace(max_free_memory_fraction=0.1)
    expected = plan.run_linear(x.reshape(rows, k), w, workspace, b)
    assert torch.equal(candidate.reshape(rows, n), expected)
    if case != "ragged":
        return
    # at the ragged shape the plan's stages (hence the operator's output) against the oracle
    torch.cuda.synchronize()
    oracle = O.load_oracle_scheme(key)
    xn, wn = x.reshape(rows, k).float().cpu().numpy(), w.float().cpu().numpy()
    a, bt = O.left_transform(oracle, xn), O.weight_transform(oracle, wn)
    rank, mb, kb = a.shape
    assert np.array_equal(from_operand(workspace.left_transformed.cpu().numpy().view(np.int16), rank, mb, kb),
                          a.view(np.int16))
    assert np.array_equal(from_operand(workspace.right_transformed.cpu().numpy().view(np.int16), rank,
                                       bt.shape[1], kb), bt.view(np.int16))
    products = workspace.products.cpu().numpy()
    exact = O.leaf_products(a, bt, product_dtype="fp32").astype(np.float64)
    magnitude = np.matmul(np.abs(a.astype(np.float64)), np.abs(np.swapaxes(bt.astype(np.float64), 1, 2)))
    assert np.all(np.abs(products.astype(np.float64) - exact)
                  <= kb * 2.0**-24 * magnitude + np.abs(exact) * 2.0**-11 + 2.0**-24)
    recombined = O.reconstruct(oracle, products, rows, n, b.float().cpu().numpy(), "bf16")
    assert np.array_equal(candidate.reshape(rows, n).cpu().view(torch.int16).numpy(), recombined.view(np.int16))


@pytest.mark.parametrize("key", ("rank7", "rank48", "rank49"))
def test_error_ratio_against_native_bf16(key) -> None:
    """North-star tolerance at a moderate shape: candidate <= 1.2x native BF16 error.

    Rank 49 is expected to exceed the bound (its fp16 leaf operands alone cost
    ~1.4x, see the oracle's prediction); its ratio is asserted to stay in the
    band the oracle predicts rather than below 1.2.
    """
    m, k, n = 1024, 4096, 2048
    g = torch.Generator().manual_seed(0)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(DEVICE)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16).to(DEVICE)
    exact = x.double() @ w.double().T
    native = _rel(torch.mm(x, w.T), exact)
    plan = PLAN_TYPES[key](m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    packed = plan.pack_weight(w)
    out = plan.run_linear_packed(x, packed, plan.allocate_workspace(prepacked_right=True))
    ratio = _rel(out, exact) / native
    print(f"\n[ratio] {key} native {native:.3e} ratio {ratio:.3f}", flush=True)
    assert torch.isfinite(out).all()
    if key == "rank49":
        assert 1.2 < ratio < 1.9
    else:
        assert ratio <= 1.2


def test_rewritten_graph_runs_a_measured_family() -> None:
    """The shipped dispatch table selects rank 7 for the corpus's 4704 x 12288 -> 4608
    down projection; the rewritten FX graph runs it within the error bound."""
    from rdna3_fastmm.linear import RDNA3_RANK7_LINEAR_OP, rewrite_eligible_linears

    class Down(torch.nn.Module):
        def forward(self, input_tensor, weight):
            return torch.nn.functional.linear(input_tensor, weight)

    print("\n[case] rewritten graph, 4704x12288 -> 4608", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn((4704, 12288), generator=g).to(torch.bfloat16).to(DEVICE)
    w = (torch.randn((4608, 12288), generator=g) / 12288**0.5).to(torch.bfloat16).to(DEVICE)
    gm = torch.fx.symbolic_trace(Down())
    for node, tensor in zip((n for n in gm.graph.nodes if n.op == "placeholder"), (x, w)):
        node.meta["val"] = tensor
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    gm.recompile()
    assert RDNA3_RANK7_LINEAR_OP in {n.target for n in gm.graph.nodes if n.op == "call_function"}
    out = gm(x, w)
    exact = x.double() @ w.double().T
    ratio = _rel(out, exact) / _rel(torch.nn.functional.linear(x, w), exact)
    print(f"[ratio] rewritten rank7 {ratio:.3f}", flush=True)
    assert ratio <= 1.2


def test_rewritten_graph_runs_a_rank48_family(monkeypatch) -> None:
    """Llama-3-70B's 28672 -> 8192 down projection at 13952 rows is covered only by a
    rank-48 dynamic family of the shipped table: the rewritten graph runs
    linear_rank48, bit-equal to Rank48Plan.run_linear and within the error bound."""
    from rdna3_fastmm.linear import RDNA3_RANK48_LINEAR_OP, rewrite_eligible_linears

    class Down(torch.nn.Module):
        def forward(self, input_tensor, weight):
            return torch.nn.functional.linear(input_tensor, weight)

    m, k, n = 13952, 28672, 8192
    print(f"\n[case] rewritten graph, {m}x{k} -> {n} (rank 48)", flush=True)
    g = torch.Generator().manual_seed(4)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(DEVICE)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16).to(DEVICE)
    gm = torch.fx.symbolic_trace(Down())
    for node, tensor in zip((node for node in gm.graph.nodes if node.op == "placeholder"), (x, w)):
        node.meta["val"] = tensor
    assert rewrite_eligible_linears(gm, [x, w]) == 1
    assert RDNA3_RANK48_LINEAR_OP in {node.target for node in gm.graph.nodes if node.op == "call_function"}
    out = gm(x, w)
    plan = Rank48Plan(m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    assert torch.equal(out, plan.run_linear(x, w, plan.allocate_workspace()))
    exact = x.double() @ w.double().T
    ratio = _rel(out, exact) / _rel(torch.nn.functional.linear(x, w), exact)
    print(f"[ratio] rewritten rank48 {ratio:.3f}", flush=True)
    assert ratio <= 1.2


def test_external_mm_choice_runs_the_rank49_plan(monkeypatch) -> None:
    """reference external_mm.py:34-48: an eligible FP16 mm runs the rank-49 dynamic plan."""
    from rdna3_fastmm import external_mm
    from rdna3_fastmm.runtime import Rank49Plan

    calls = []
    original = Rank49Plan.run
    monkeypatch.setattr(Rank49Plan, "dynamic_shapes", frozenset({(200, 512, 520)}))
    monkeypatch.setattr(Rank49Plan, "run", lambda self, *a, **k: calls.append(1) or original(self, *a, **k))
    g = torch.Generator().manual_seed(5)
    left = torch.randn((200, 512), generator=g).to(torch.float16).to(DEVICE)
    right = (torch.randn((512, 520), generator=g) / 512**0.5).to(torch.float16).to(DEVICE)
    out = torch.empty((200, 520), device=DEVICE, dtype=torch.float16)
    with torch.inference_mode():
        external_mm.rdna3_rank49_dynamic_v1_out(left, right, out=out)
        assert calls == [1]
        exact = left.double() @ right.double()
        # the reference's mm bound (tests/test_rdna3.py:433-613); with an FP16 output,
        # native's one 2^-11 rounding makes a ratio test meaningless for rank 49
        assert _rel(out, exact) < 5e-3
        # an unmeasured shape is torch.mm, bit for bit
        other = torch.empty((200, 520), device=DEVICE, dtype=torch.float16)
        external_mm.rdna3_rank49_dynamic_v1_out(left[:199].contiguous(), right, out=other[:199])
        assert calls == [1]
        assert torch.equal(other[:199], torch.mm(left[:199], right))


def test_rank343_dynamic_and_packed_match_exact_small_product() -> None:
    """reference test_rdna3.py:726-752: small integers stay exact through rank 343."""
    from rdna3_fastmm.runtime import Rank343Plan

    torch.manual_seed(17)
    for shape in ((5, 6, 7), (37, 29, 41), (64, 64, 64)):
        print(f"\n[case] rank343 exact {shape}", flush=True)
        left = torch.randint(-2, 3, shape[:2], device=DEVICE, dtype=torch.float16)
        right = torch.randint(-2, 3, shape[1:], device=DEVICE, dtype=torch.float16)
        reference = (left.float() @ right.float()).half()
        plan = Rank343Plan(*shape, device=DEVICE)
        packed = plan.pack_right(right, max_free_memory_fraction=0.1)
        dynamic = plan.run(left, right, plan.allocate_workspace(max_free_memory_fraction=0.1))
        prepacked = plan.run_packed(left, packed, plan.allocate_workspace(0.1, prepacked_right=True))
        assert torch.equal(dynamic, reference) and torch.equal(prepacked, reference)


def test_rank343_matches_oracle_within_the_mm_bound() -> None:
    """Random FP16 operands: equal to the oracle's circuit evaluation up to leaf fp32
    accumulation, and inside the reference's mm bound (rel-L2 < 5e-3)."""
    from rdna3_fastmm.runtime import Rank343Plan

    m, k, n = 200, 264, 136
    print(f"\n[case] rank343 oracle {m}x{k}x{n}", flush=True)
    g = torch.Generator().manual_seed(23)
    left = torch.randn((m, k), generator=g).to(torch.float16)
    right = (torch.randn((k, n), generator=g) / k**0.5).to(torch.float16)
    plan = Rank343Plan(m, k, n, device=DEVICE)
    out = plan.run(left.to(DEVICE), right.to(DEVICE), plan.allocate_workspace(0.1)).float().cpu().numpy()
    scheme = O.load_oracle_scheme("rank343")
    circuit = O.matmul(scheme, left.float().numpy(), right.float().numpy()).astype(np.float32)
    dense = O.matmul(scheme, left.float().numpy(), right.float().numpy(), recombination="dense").astype(np.float32)
    exact = left.double().numpy() @ right.double().numpy()
    for expected in (circuit, dense):
        assert np.linalg.norm(out - expected) <= 0.2 * np.linalg.norm(expected - exact)
    assert np.linalg.norm(out - exact) / np.linalg.norm(exact) < 5e-3
