"""Plans captured in a HIP graph (``torch.cuda.CUDAGraph``) replay like eager calls.

Every stage of a plan is a kernel launch on the current stream with caller-owned
buffers: no allocation (given ``output``), no host synchronization, no memset. So
a captured ``run_linear`` / ``run_linear_packed`` replays exactly (bitwise) like
the eager call on the same inputs. The shapes put inside the graph the persistent
leaf GEMM with the split-K tail (rank 7), a persistent launch with whole rounds
(rank 48), the persistent kernel's strip form for a last tile row of 11 rows
(rank 7, M = 8214), and products large enough (1.6 GB, rank 49) that the leaf
GEMM stores and the recombination loads them non-temporally. Each replay follows
eager work and a synchronization, and is checked on its own.
"""

import pytest
import torch

from rdna3_fastmm.runtime import Rank7Plan, Rank48Plan, Rank49Plan

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda", 0)


def _tile_plan(plan) -> tuple[int, int]:
    """(256x256 leaf tiles, compute units) of the plan's leaf GEMM."""
    shape = plan.shape
    tiles = plan.rank * -(-shape.block_rows // 256) * -(-shape.block_columns // 256)
    return tiles, torch.cuda.get_device_properties(DEVICE).multi_processor_count


@pytest.mark.parametrize(
    ("plan_type", "shape", "packed"),
    (
        (Rank7Plan, (4608, 1024, 4608), True),  # 567 tiles: persistent rounds + split-K tail
        (Rank7Plan, (4608, 1024, 4608), False),
        (Rank48Plan, (4096, 2048, 4096), True),  # 768 tiles: three whole rounds
        (Rank7Plan, (8214, 512, 4608), True),  # a last tile row of 11 rows fused as a strip
        (Rank49Plan, (16384, 1024, 16384), True),  # 1.6 GB of products: streamed stores and loads
    ),
)
def test_captured_linear_replays_match_eager(plan_type, shape, packed) -> None:
    m, k, n = shape
    print(f"\n[case] graph replay {plan_type.__name__} {shape} packed={packed}", flush=True)
    g = torch.Generator().manual_seed(m + k + n)
    inputs = [torch.randn((m, k), generator=g).to(torch.bfloat16).to(DEVICE) for _ in range(3)]
    weight = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16).to(DEVICE)
    bias = (torch.randn((n,), generator=g) * 0.02).to(torch.bfloat16).to(DEVICE)
    plan = plan_type(m, k, n, DEVICE, dtype=torch.bfloat16, compute_dtype=torch.float16)
    tiles, cus = _tile_plan(plan)
    assert tiles > cus  # more than one round: the persistent kernel runs
    weight_arg = plan.pack_weight(weight) if packed else weight
    captured_workspace = plan.allocate_workspace(prepacked_right=packed)
    eager_workspace = plan.allocate_workspace(prepacked_right=packed)
    run = plan.run_linear_packed if packed else plan.run_linear

    static_input = torch.empty((m, k), device=DEVICE, dtype=torch.bfloat16)
    static_output = torch.empty((m, n), device=DEVICE, dtype=torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # first calls (one-time launch set-up) outside the capture
        static_input.copy_(inputs[0])
        run(static_input, weight_arg, captured_workspace, bias, static_output)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(static_input, weight_arg, captured_workspace, bias, static_output)

    for replay, x in enumerate(inputs + inputs[:1]):
        expected = run(x, weight_arg, eager_workspace, bias)  # eager, own workspace and output
        torch.cuda.synchronize()
        static_input.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(expected.float()).all()
        assert torch.equal(static_output.view(torch.int16), expected.view(torch.int16)), replay
