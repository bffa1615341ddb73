"""Every HIP stage against the CPU oracle on the same seeded inputs.

Transforms and recombination are bit-exact (same fp32 program order, same
round-to-nearest-even stores); transformed operands are compared in logical
plane order after undoing the kernels' K-slab layout (``tests/_layout.py``). Leaf products differ from the oracle's
near-exact fp64 sum only by fp32 accumulation: the bound below is the
standard ``K * 2^-24 * sum|a*b|`` (plus one fp16 ulp when stored as fp16).
"""

import numpy as np
import pytest
import torch

from _layout import from_operand, to_operand
from oracle import fastmm_oracle as O
from rdna3_fastmm import _stages
from rdna3_fastmm.runtime import operand_shape
from rdna3_fastmm.schemes import SCHEME_KEYS, load_scheme

pytestmark = pytest.mark.gpu

SHAPES = (
    (5, 6, 7),
    (17, 19, 23),
    (64, 64, 64),
    (257, 263, 269),
    (96, 128, 160),
    (300, 256, 192),
    (33, 255, 47),  # ragged K with Kb % 32 == 0: K-slab output from the scalar path
)
DTYPES = (torch.bfloat16, torch.float16)
DEVICE = torch.device("cuda", 0)


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


def _inputs(shape, dtype, seed):
    m, k, n = shape
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(dtype)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(dtype)
    bias = (torch.randn((n,), generator=g) * 0.02).to(dtype)
    return x, w, bias


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy()


def _fp16_only(scheme) -> bool:
    """The 8x8-block scheme (rank 343) runs FP16 operands, planes and outputs only."""
    return scheme.size > 4


def _dense_recombination(scheme, product_dtype, dtype, use_bias, n) -> bool:
    """Inputs the library recombines with the 8x8-block scheme's dense MFMA form:
    fp16 products, fp16 output, no bias and N a multiple of 64."""
    return (scheme.size == 8 and product_dtype == torch.float16 and dtype == torch.float16
            and not use_bias and n % 64 == 0)


def _fp16_order(bits: np.ndarray) -> np.ndarray:
    """fp16 bit patterns -> integers in value order (adjacent values differ by 1)."""
    b = bits.astype(np.int32) & 0xFFFF
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _assert_dense_match(out: torch.Tensor, oracle, products: np.ndarray, m: int, n: int) -> None:
    """The dense form's result: the exact sum rounded once (oracle), up to the fp32
    summation order, which is the MFMA's. Elementwise, |out - exact| is at most
    one fp16 ulp of the output plus 343 fp32 units of the sum of |terms| (the
    order's rounding; near cancellation that can exceed an fp16 ulp of a tiny
    result). Almost every element is bit-exact."""
    exact = O.reconstruct_dense(oracle, products, m, n, "fp32").astype(np.float64)
    got_bits = _bits(out)
    distance = np.abs(_fp16_order(got_bits) - _fp16_order(exact.astype(np.float16).view(np.int16)))
    assert np.count_nonzero(distance) <= max(1, distance.size // 1000)
    weights = np.abs(np.array(O.program_matrix(oracle.output), dtype=np.float64))  # [64, 343]
    mb, nb = products.shape[1:]
    magnitude = np.einsum("or,rmn->omn", weights, np.abs(products.astype(np.float64)))
    magnitude = magnitude.reshape(8, 8, mb, nb).transpose(0, 2, 1, 3).reshape(8 * mb, 8 * nb)[:m, :n]
    got = got_bits.view(np.float16)
    ulp = np.spacing(np.abs(got)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= ulp + 343 * 2.0**-24 * magnitude)


def _plane_bits(planes: np.ndarray, plane_dtype: str) -> np.ndarray:
    if plane_dtype == "bf16":
        return O.round_to_bf16(planes).view(np.int16)
    return planes.view(np.int16)


@pytest.mark.parametrize("key", SCHEME_KEYS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("plane_dtype", ("fp16", "bf16"))
def test_transforms_bit_exact(key, shape, dtype, plane_dtype) -> None:
    print(f"\n[case] transforms {key} {shape} {dtype} -> {plane_dtype} planes", flush=True)
    scheme = load_scheme(key)
    oracle = O.load_oracle_scheme(key)
    m, k, n = shape
    s, r = scheme.size, scheme.rank
    x, w, _ = _inputs(shape, dtype, seed=m + k + n)
    xg, wg = x.to(DEVICE), w.to(DEVICE)
    mb, kb, nb = _ceil(m, s), _ceil(k, s), _ceil(n, s)
    planes = torch.bfloat16 if plane_dtype == "bf16" else torch.float16
    a = torch.empty(operand_shape(r, mb, kb), device=DEVICE, dtype=planes)
    b = torch.empty(operand_shape(r, nb, kb), device=DEVICE, dtype=planes)
    b2 = torch.empty_like(b)
    if _fp16_only(scheme) and (dtype != torch.float16 or plane_dtype != "fp16"):
        for stage, args in ((_stages.left_transform, (xg, a, m, k)), (_stages.weight_transform, (wg, b, n, k)),
                            (_stages.right_transform, (wg.t().contiguous(), b2, k, n))):
            with pytest.raises(RuntimeError, match="takes fp16 input and planes"):
                stage(scheme, *args)
        return
    _stages.left_transform(scheme, xg, a, m, k)
    _stages.weight_transform(scheme, wg, b, n, k)
    right = wg.t().contiguous()
    _stages.right_transform(scheme, right, b2, k, n)
    torch.cuda.synchronize()
    expect_a = _plane_bits(O.left_transform(oracle, _np(x), plane_dtype), plane_dtype)
    expect_b = _plane_bits(O.weight_transform(oracle, _np(w), plane_dtype), plane_dtype)
    assert np.array_equal(from_operand(_bits(a), r, mb, kb), expect_a)
    assert np.array_equal(from_operand(_bits(b), r, nb, kb), expect_b)
    assert np.array_equal(from_operand(_bits(b2), r, nb, kb), expect_b)


@pytest.mark.parametrize("key", SCHEME_KEYS)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("product_dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_reconstruct_bit_exact(key, shape, product_dtype) -> None:
    print(f"\n[case] reconstruct {key} {shape} {product_dtype}", flush=True)
    scheme = load_scheme(key)
    oracle = O.load_oracle_scheme(key)
    m, _, n = shape
    s, r = scheme.size, scheme.rank
    g = torch.Generator().manual_seed(m * n)
    products = torch.randn((r, _ceil(m, s), _ceil(n, s)), generator=g).to(product_dtype)
    for dtype in DTYPES:
        bias = (torch.randn((n,), generator=g) * 0.1).to(dtype)
        if _fp16_only(scheme) and (dtype != torch.float16 or product_dtype == torch.bfloat16):
            out = torch.empty((m, n), device=DEVICE, dtype=dtype)
            with pytest.raises(RuntimeError, match="fp16 or fp32 products and an fp16 output"):
                _stages.reconstruct(scheme, products.to(DEVICE), None, out, m, n)
            continue
        for use_bias in (False, True):
            out = torch.empty((m, n), device=DEVICE, dtype=dtype)
            _stages.reconstruct(scheme, products.to(DEVICE), bias.to(DEVICE) if use_bias else None, out, m, n)
            torch.cuda.synchronize()
            if _dense_recombination(scheme, product_dtype, dtype, use_bias, n):
                _assert_dense_match(out, oracle, products.numpy(), m, n)
                continue
            expected = O.reconstruct(
                oracle,
                products.numpy() if product_dtype == torch.float16 else products.float().numpy(),
                m,
                n,
                _np(bias) if use_bias else None,
                "bf16" if dtype == torch.bfloat16 else "fp16",
            )
            assert np.array_equal(_bits(out), expected.view(np.int16)), (dtype, use_bias)


@pytest.mark.parametrize("shape", ((64, 64), (37, 128), (300, 192), (1000, 576), (2050, 1024)))
def test_rank343_dense_recombination_matches_the_dense_oracle(shape) -> None:
    """Rank 343, fp16 products and output, no bias: the dense MFMA contraction
    (reference output_transform_mfma_kernel) against the oracle's dense form.
    The shapes cover one and many tiles of 64 positions per wave, a partial last
    tile (plane 5 x 16 = 1.25 tiles at 37 x 128; 125 x 72 = 140.6 tiles at
    1000 x 576), padded output rows (M % 8 != 0) and small integers, which must
    come out exact."""
    m, n = shape
    print(f"\n[case] rank343 dense recombination {shape}", flush=True)
    scheme = load_scheme("rank343")
    oracle = O.load_oracle_scheme("rank343")
    g = torch.Generator().manual_seed(m + 7 * n)
    products = torch.randn((343, _ceil(m, 8), _ceil(n, 8)), generator=g).to(torch.float16)
    out = torch.empty((m, n), device=DEVICE, dtype=torch.float16)
    _stages.reconstruct(scheme, products.to(DEVICE), None, out, m, n)
    torch.cuda.synchronize()
    _assert_dense_match(out, oracle, products.numpy(), m, n)
    integers = torch.randint(-3, 4, products.shape, generator=g).to(torch.float16)
    _stages.reconstruct(scheme, integers.to(DEVICE), None, out, m, n)
    torch.cuda.synchronize()
    expected = O.reconstruct_dense(oracle, integers.numpy(), m, n, "fp16")
    assert np.array_equal(_bits(out), expected.view(np.int16))


@pytest.mark.parametrize(
    "dims",
    (
        # generic kernel: ragged or short K, unaligned rows
        (1, 5, 3, 7), (7, 33, 17, 129), (3, 256, 256, 64), (2, 300, 260, 136), (7, 129, 385, 2048), (5, 64, 64, 13),
        # 32x32x16 kernel: Kb % 32 == 0, Kb >= 96, Kb % 128 != 0
        (2, 300, 264, 96), (1, 4107, 16, 192), (3, 129, 72, 224), (2, 256, 256, 1056),
        # 16x16x32 kernel: Kb % 128 == 0 -- four slices only (no main-loop pass), one and
        # several passes, ragged Mb / Nb tails, a single 8-column tile, rows not a multiple of 16
        (3, 513, 520, 128), (2, 17, 24, 256), (7, 256, 256, 2048), (2, 40, 8, 3072), (1, 1000, 776, 640),
        (4, 255, 264, 512),
        # more tiles than one wave of 256 workgroups: ragged rows, one-row-tall last tiles,
        # narrow columns, many leaves
        (7, 2048, 2304, 256), (2, 4107, 2304, 384), (48, 520, 512, 256), (17, 4000, 40, 256),
        (49, 1024, 1024, 512),
        # split-K tail (with scratch): one tile in 8 K parts, ragged tiles, full rounds + a tail;
        # two persistent rounds (16-bit products) + a tail in 6 parts
        (1, 256, 256, 1024), (2, 300, 520, 1024), (3, 2560, 2560, 256), (3, 2300, 5120, 768),
    ),
)
@pytest.mark.parametrize(
    ("operand_dtype", "product_dtype"),
    (
        (torch.float16, torch.float16),
        (torch.float16, torch.float32),
        (torch.bfloat16, torch.bfloat16),
        (torch.bfloat16, torch.float32),
    ),
)
def test_leaf_products_within_fp32_accumulation_bound(dims, operand_dtype, product_dtype) -> None:
    rank, mb, nb, kb = dims
    print(f"\n[case] leaf products {dims} {operand_dtype} -> {product_dtype}", flush=True)
    g = torch.Generator().manual_seed(sum(dims))
    a = torch.randn((rank, mb, kb), generator=g).to(operand_dtype)
    b = torch.randn((rank, nb, kb), generator=g).to(operand_dtype)
    p = torch.empty((rank, mb, nb), device=DEVICE, dtype=product_dtype)
    # operand buffers in the kernels' layout (bit patterns moved as int16)
    a_dev = torch.from_numpy(to_operand(a.view(torch.int16).numpy())).to(DEVICE).view(operand_dtype)
    b_dev = torch.from_numpy(to_operand(b.view(torch.int16).numpy())).to(DEVICE).view(operand_dtype)
    _stages.leaf_products(rank, a_dev, b_dev, p, mb, kb, nb)
    # the same launch with the split-K tail's scratch, and with a scratch too small to use
    scratch_bytes = _stages.leaf_scratch_bytes(rank, operand_dtype, product_dtype, mb, kb, nb, DEVICE)
    runs = [p]
    for size in (scratch_bytes, 16) if scratch_bytes else ():
        scratch = torch.empty(size, device=DEVICE, dtype=torch.uint8)
        runs.append(torch.empty_like(p))
        _stages.leaf_products(rank, a_dev, b_dev, runs[-1], mb, kb, nb, scratch)
    print(f"[case] scratch bytes {scratch_bytes}", flush=True)
    torch.cuda.synchronize()
    a32, b32 = a.float().numpy(), b.float().numpy()
    exact = O.leaf_products(a32, b32, product_dtype="fp32")
    magnitude = np.matmul(np.abs(a32.astype(np.float64)), np.abs(np.swapaxes(b32.astype(np.float64), 1, 2)))
    bound = kb * 2.0**-24 * magnitude + 1e-30
    if product_dtype == torch.float16:
        # one fp16 rounding of a value within `bound` of the exact sum
        bound = bound + np.abs(exact.astype(np.float64)) * 2.0**-11 + 2.0**-24
    if product_dtype == torch.bfloat16:
        # one bf16 rounding (8-bit significand)
        bound = bound + np.abs(exact.astype(np.float64)) * 2.0**-8 + 2.0**-126
    for got in runs:
        assert np.all(np.abs(got.float().cpu().numpy().astype(np.float64) - exact) <= bound)


def test_leaf_scratch_sizes_follow_the_tail_plan() -> None:
    """The split-K tail plan: with one 256x256 tile per CU per round, a last round of
    `tail = tiles % CUs` tiles is split along K into min(8, Kb // 128, 3*CUs // (4*tail))
    parts (none below 2), each a 256 KB fp32 tile of scratch. A last tile row of at
    most 16 rows is left out when that takes the tiles down a round: as a strip fused
    into the persistent kernel (tiles without a split tail, a last group of 8 tile rows
    holding at least 4), else in the thin-row kernel when rank * Nb <= 32768."""
    cus = torch.cuda.get_device_properties(DEVICE).multi_processor_count

    def tail_bytes(tiles, kb):
        tail = tiles % cus
        if tail == 0:
            return 0
        split = min(8, kb // 128, 3 * cus // (4 * tail))
        return tail * split * 256 * 256 * 4 if split >= 2 else 0

    def expected(rank, mb, kb, nb):
        tiles_n = -(-nb // 256)
        with_row = rank * -(-mb // 256) * tiles_n
        without = with_row - rank * tiles_n
        if mb > 256 and 0 < mb % 256 <= 16 and -(-without // cus) < -(-with_row // cus):
            full = mb // 256
            if full - 8 * ((full - 1) // 8) >= 4 and tail_bytes(without, kb) == 0:
                return 0  # the strip
            if rank * nb <= 32768:
                return tail_bytes(without, kb)  # the thin-row kernel
        return tail_bytes(with_row, kb)

    # C3 (tail 47), C2 (64), whole rounds, one tile, K too short, split capped by
    # Kb, a tail of 128 (no split), 24 (split 8), 16 (capped at 8)
    for dims in ((7, 4107, 6144, 2304), (7, 2048, 2048, 6144), (48, 2048, 2048, 2048), (1, 256, 1024, 256),
                 (3, 2560, 256, 2560), (7, 4107, 128, 2304), (7, 4352, 6144, 2304), (48, 1100, 2048, 2048),
                 (7, 1280, 14336, 2048), (48, 2816, 3072, 256), (7, 4112, 6144, 2304), (7, 4113, 6144, 2304),
                 (48, 2054, 3072, 1152), (2, 2305, 256, 3328)):
        rank, mb, kb, nb = dims
        got = _stages.leaf_scratch_bytes(rank, torch.float16, torch.float16, mb, kb, nb, DEVICE)
        assert got == expected(rank, mb, kb, nb), dims
    # shapes off the 16x16x32 path need none
    assert _stages.leaf_scratch_bytes(7, torch.float16, torch.float16, 4107, 6150, 2304, DEVICE) == 0
    assert _stages.leaf_scratch_bytes(7, torch.float16, torch.float16, 4107, 6144, 2300, DEVICE) == 0


@pytest.mark.parametrize(
    ("rank", "mb", "kb", "nb", "scale", "dtype"),
    (
        (7, 1000, 384, 2776, 1.0, torch.float16),  # ragged rows and columns
        (3, 2304, 1024, 4096, 30.0, torch.float16),  # fp16 overflow to infinity
        (3, 2048, 256, 4096, 1e-3, torch.float16),  # fp16 subnormals; 8 slices, the minimum
        (7, 1000, 384, 2776, 1.0, torch.bfloat16),
        (40, 4096, 256, 4096, 1.0, torch.float16),  # 1.34 GB of products: stored non-temporally
    ),
)
def test_persistent_and_per_tile_kernels_agree_bitwise(rank, mb, kb, nb, scale, dtype) -> None:
    """16-bit products over more tiles than compute units run on the persistent kernel;
    the same leaves one at a time (fewer tiles than compute units) run one workgroup per
    tile. Both compute each tile with the same MFMA sequence and the same rounding, so
    the products agree bit for bit (no scratch: no split-K tail in either)."""
    print(f"\n[case] persistent vs per-tile {(rank, mb, kb, nb)} {dtype} scale {scale}", flush=True)
    cus = torch.cuda.get_device_properties(DEVICE).multi_processor_count
    per_leaf = -(-mb // 256) * -(-nb // 256)
    if not per_leaf <= cus < rank * per_leaf:
        pytest.skip(f"{cus} compute units: the shape does not split into both paths")
    g = torch.Generator().manual_seed(rank * mb + kb + nb)
    a = (torch.randn((rank, mb, kb), generator=g) * scale).to(dtype).to(DEVICE)
    b = (torch.randn((rank, nb, kb), generator=g) * scale).to(dtype).to(DEVICE)
    together = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=dtype)
    apart = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=dtype)
    _stages.leaf_products(rank, a, b, together, mb, kb, nb)
    for r in range(rank):
        _stages.leaf_products(1, a[r : r + 1], b[r : r + 1], apart[r : r + 1], mb, kb, nb)
    torch.cuda.synchronize()
    assert not torch.isnan(together).any()
    assert torch.equal(together.view(torch.int16), apart.view(torch.int16))
    if scale > 1:
        assert torch.isinf(together).any()
    if scale < 1:
        assert ((together != 0) & (together.abs() < 2.0**-14)).any()


def _persistent_random_shapes(count: int = 24) -> list[tuple[int, int, int, int]]:
    """Seeded (rank, Mb, Kb, Nb): one leaf fits a round of 256x256 tiles on a 256-CU
    device (the per-tile kernel), all of them need more (the persistent kernel)."""
    rng = np.random.default_rng(4242)
    shapes = []
    while len(shapes) < count:
        mb, nb = int(rng.integers(300, 3300)), int(rng.integers(40, 380)) * 8
        kb = int(rng.choice([256, 384, 512, 768, 1024]))
        per_leaf = -(-mb // 256) * -(-nb // 256)
        if not 4 <= per_leaf <= 256:
            continue
        low = 256 // per_leaf + 1
        rank = int(rng.integers(low, max(low + 1, 2200 // per_leaf)))
        if 256 < rank * per_leaf <= 2200 and rank * mb * nb * 2 <= 1.5e9:
            shapes.append((rank, mb, kb, nb))
    return shapes


@pytest.mark.parametrize(("rank", "mb", "kb", "nb"), _persistent_random_shapes())
def test_persistent_kernel_matches_per_tile_on_random_shapes(rank, mb, kb, nb) -> None:
    """Seeded random shapes, ragged rows and columns, every workgroup's first tile and
    later ones: the persistent kernel's products (all leaves in one call) equal the
    per-tile kernel's (one leaf per call) bit for bit, no scratch (no split-K tail)."""
    print(f"\n[case] persistent vs per-tile, random {(rank, mb, kb, nb)}", flush=True)
    cus = torch.cuda.get_device_properties(DEVICE).multi_processor_count
    per_leaf = -(-mb // 256) * -(-nb // 256)
    if not per_leaf <= cus < rank * per_leaf:
        pytest.skip(f"{cus} compute units: the shape does not split into both paths")
    g = torch.Generator(device=DEVICE).manual_seed(rank * mb + kb * nb)
    a = torch.randn((rank, mb, kb), device=DEVICE, generator=g).to(torch.float16)
    b = torch.randn((rank, nb, kb), device=DEVICE, generator=g).to(torch.float16)
    together = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=torch.float16)
    apart = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=torch.float16)
    _stages.leaf_products(rank, a, b, together, mb, kb, nb)
    for r in range(rank):
        _stages.leaf_products(1, a[r : r + 1], b[r : r + 1], apart[r : r + 1], mb, kb, nb)
    torch.cuda.synchronize()
    assert not torch.isnan(together).any()
    assert torch.equal(together.view(torch.int16), apart.view(torch.int16))


@pytest.mark.parametrize(
    ("rank", "mb", "kb", "nb", "dtype", "product_dtype"),
    (
        # the strip fused into the persistent kernel: C3's 11-row edge, rank 48 at C3
        # (6 rows; 8 and 16 slices), a last group of 4 tile rows with ragged columns,
        # 16 rows and 1 row, bf16
        (7, 4107, 1024, 2304, torch.float16, torch.float16),
        (48, 2054, 256, 1152, torch.float16, torch.float16),
        (48, 2054, 512, 1152, torch.float16, torch.float16),
        (5, 3077, 256, 2040, torch.float16, torch.float16),
        (7, 4112, 384, 2304, torch.float16, torch.float16),
        (7, 4097, 512, 2304, torch.bfloat16, torch.bfloat16),
        # the thin-row kernel: fp32 products (no persistent kernel), a last group of one
        # tile row (16 rows, ragged columns, 8 slices), one row
        (7, 4107, 256, 2304, torch.float16, torch.float32),
        (2, 2320, 256, 3320, torch.float16, torch.float16),
        (2, 2320, 512, 3328, torch.bfloat16, torch.bfloat16),
        (2, 2305, 384, 3328, torch.float16, torch.float32),
    ),
)
def test_thin_tile_row_matches_full_tiles_bitwise(rank, mb, kb, nb, dtype, product_dtype) -> None:
    """A last tile row of at most 16 rows is left out of the 256x256 tiles when that takes
    them down a round: fused into the persistent kernel as a strip, or run by the thin-row
    kernel. Padding the leaves with zero rows until that row holds more than 16 rows
    sends it through the 256x256 tiles instead; zero rows change no other row, and every
    path issues the same MFMA sequence per product, so the real rows agree bit for bit."""
    print(f"\n[case] thin tile row {(rank, mb, kb, nb)} {dtype} -> {product_dtype}", flush=True)
    cus = torch.cuda.get_device_properties(DEVICE).multi_processor_count
    tiles_n = -(-nb // 256)
    tiles = rank * -(-mb // 256) * tiles_n
    if not -(-(tiles - rank * tiles_n) // cus) < -(-tiles // cus):
        pytest.skip(f"{cus} compute units: the thin row does not take the tiles down a round")
    padded = mb + (17 - mb % 256 if mb % 256 <= 16 else 0)
    assert padded % 256 > 16
    g = torch.Generator().manual_seed(rank + mb + kb + nb)
    a = torch.randn((rank, mb, kb), generator=g).to(dtype)
    b = torch.randn((rank, nb, kb), generator=g).to(dtype)
    a_padded = torch.cat([a, torch.zeros((rank, padded - mb, kb), dtype=dtype)], dim=1)

    def device_operand(planes: torch.Tensor) -> torch.Tensor:
        return torch.from_numpy(to_operand(planes.view(torch.int16).numpy())).to(DEVICE).view(dtype)

    thin = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=product_dtype)
    full = torch.full((rank, padded, nb), float("nan"), device=DEVICE, dtype=product_dtype)
    _stages.leaf_products(rank, device_operand(a), device_operand(b), thin, mb, kb, nb)
    _stages.leaf_products(rank, device_operand(a_padded), device_operand(b), full, padded, kb, nb)
    torch.cuda.synchronize()
    assert not torch.isnan(thin).any()
    bits = torch.int32 if product_dtype == torch.float32 else torch.int16
    assert torch.equal(thin.view(bits), full[:, :mb].contiguous().view(bits))


def test_stage_operators_check_buffers_before_any_launch() -> None:
    """Undersized, non-contiguous, mistyped or host buffers raise ValueError in the
    operators before the C ABI sees a pointer: the sentinels in every buffer survive,
    and the same calls with whole buffers go through."""
    print("\n[case] stage operator buffer checks", flush=True)
    scheme = load_scheme("rank7")
    m, k, n = 64, 96, 80
    s, r = scheme.size, scheme.rank
    mb, kb, nb = m // s, k // s, n // s
    g = torch.Generator().manual_seed(11)
    x = torch.randn((m, k), generator=g).to(torch.float16).to(DEVICE)
    w = torch.randn((n, k), generator=g).to(torch.float16).to(DEVICE)
    bias = torch.zeros((n,), device=DEVICE, dtype=torch.float16)
    a = torch.full((r * mb * kb,), 7.0, device=DEVICE, dtype=torch.float16)
    b = torch.full((r * nb * kb,), 7.0, device=DEVICE, dtype=torch.float16)
    p = torch.full((r * mb * nb,), 7.0, device=DEVICE, dtype=torch.float16)
    out = torch.full((m, n), 7.0, device=DEVICE, dtype=torch.float16)
    right = w.t().contiguous()
    cases = (
        (lambda: _stages.left_transform(scheme, x, a[:-1], m, k), "planes holds"),
        (lambda: _stages.left_transform(scheme, x.t(), a, k, m), "source must be contiguous"),
        (lambda: _stages.left_transform(scheme, x, a.cpu(), m, k), "planes must be on the operands' ROCm device"),
        (lambda: _stages.weight_transform(scheme, w, b[:-1], n, k), "planes holds"),
        (lambda: _stages.right_transform(scheme, right[:-1], b, k, n), "source holds"),
        (lambda: _stages.leaf_products(r, a, b, p[:-1], mb, kb, nb), "products holds"),
        (lambda: _stages.leaf_products(r, a, b[:-1], p, mb, kb, nb), "right planes holds"),
        (lambda: _stages.leaf_products(r, a, b.bfloat16(), p, mb, kb, nb), "differ in dtype"),
        (lambda: _stages.leaf_products(r, a, b, p, mb, kb, nb, torch.zeros(64, dtype=torch.uint8)),
         "scratch must be on"),
        (lambda: _stages.reconstruct(scheme, p, None, out[:-1], m, n), "output holds"),
        (lambda: _stages.reconstruct(scheme, p[:-1], None, out, m, n), "products holds"),
        (lambda: _stages.reconstruct(scheme, p, bias[:-1], out, m, n), "bias holds"),
        (lambda: _stages.reconstruct(scheme, p, bias.float(), out, m, n), "bias must have the output's dtype"),
        (lambda: _stages.reconstruct(scheme, p.cpu(), None, out, m, n), "must be on a ROCm device"),
    )
    for call, message in cases:
        with pytest.raises(ValueError, match=message):
            call()
    torch.cuda.synchronize()
    for buffer in (a, b, p, out):
        assert bool((buffer == 7.0).all())
    _stages.left_transform(scheme, x, a, m, k)
    _stages.weight_transform(scheme, w, b, n, k)
    _stages.leaf_products(r, a, b, p, mb, kb, nb)
    _stages.reconstruct(scheme, p, bias, out, m, n)
    torch.cuda.synchronize()
    expected = x.float() @ w.float().t()
    assert torch.allclose(out.float(), expected, rtol=2e-2, atol=0.5)
