"""Pins of the CPU oracle (oracle/fastmm_oracle.py) against mathematics.

Each check is chosen so that a plausible mistake in the oracle (a wrong
block index, a transposed operand, a dropped term, a sign flip, a wrong
rounding) fails at least one of them; test_planted_sign_error_is_caught
shows it for a sign flip.
"""

from copy import deepcopy
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import fastmm_oracle as O
from rdna3_fastmm.schemes import SCHEME_KEYS, load_scheme

SHAPES = ((5, 6, 7), (9, 6, 7), (17, 19, 23), (8, 8, 8), (33, 40, 24))


def _brent_ok(scheme: O.OracleScheme) -> bool:
    """Exact Brent identity for square s-blocks, written out independently."""
    s = scheme.size
    u = O.program_matrix(scheme.left)
    v = O.program_matrix(scheme.right)
    w = O.program_matrix(scheme.output)
    for i in range(s):
        for k in range(s):
            for k2 in range(s):
                for j in range(s):
                    for i2 in range(s):
                        for j2 in range(s):
                            total = sum(
                                u[r][i * s + k] * v[r][k2 * s + j] * w[i2 * s + j2][r]
                                for r in range(scheme.rank)
                            )
                            expected = int(k == k2 and i == i2 and j == j2)
                            if total != expected:
                                return False
    return True


def _brent_integer_ok(scheme: O.OracleScheme) -> bool:
    """The full Brent tensor with integer arithmetic (numpy), for large schemes."""
    s = scheme.size
    u, v, w = (np.array(O.program_matrix(p), dtype=object) for p in (scheme.left, scheme.right, scheme.output))
    if any(c.denominator != 1 for m in (u, v, w) for c in m.ravel()):
        return False
    u, v, w = (m.astype(np.int64) for m in (u, v, w))
    tensor = np.einsum("ra,rb,cr->abc", u, v, w)  # a = (i, k), b = (k2, j), c = (i2, j2)
    expected = np.zeros((s * s, s * s, s * s), dtype=np.int64)
    for i in range(s):
        for k in range(s):
            for j in range(s):
                expected[i * s + k, k * s + j, i * s + j] = 1
    return bool(np.array_equal(tensor, expected))


@pytest.mark.parametrize("key", SCHEME_KEYS)
def test_oracle_scheme_satisfies_brent_identity(key: str) -> None:
    scheme = O.load_oracle_scheme(key)
    if scheme.size == 8:
        assert _brent_integer_ok(scheme)
    elif scheme.size == 4:
        # The 4096-entry brute force is slow in pure Python; the rank-7 case runs
        # in full and the s=4 schemes through the cheaper bilinear check below.
        rng = np.random.default_rng(3)
        x = [Fraction(int(v)) for v in rng.integers(-3, 4, 16)]
        y = [Fraction(int(v)) for v in rng.integers(-3, 4, 16)]
        a = O.evaluate_program(scheme.left, x, Fraction)
        b = O.evaluate_program(scheme.right, y, Fraction)
        c = O.evaluate_program(scheme.output, [p * q for p, q in zip(a, b)], Fraction)
        expected = [sum(x[i * 4 + k] * y[k * 4 + j] for k in range(4)) for i in range(4) for j in range(4)]
        assert c == expected
    else:
        assert _brent_ok(scheme)


@pytest.mark.parametrize("key", SCHEME_KEYS)
def test_oracle_matrices_equal_product_loader(key: str) -> None:
    """Two independent parsers (Python ast here, hand-written in the product)."""
    oracle = O.load_oracle_scheme(key)
    product = load_scheme(key)
    assert [tuple(r) for r in O.program_matrix(oracle.left)] == list(product.left.coefficients())
    assert [tuple(r) for r in O.program_matrix(oracle.right)] == list(product.right.coefficients())
    assert [tuple(r) for r in O.program_matrix(oracle.output)] == list(product.output.coefficients())


@pytest.mark.parametrize("key", SCHEME_KEYS)
@pytest.mark.parametrize("shape", SHAPES)
def test_exact_small_integer_product(key: str, shape: tuple[int, int, int]) -> None:
    """reference tests/test_rdna3.py:406-430: small integers stay exact end to end."""
    rng = np.random.default_rng(sum(shape))
    scheme = O.load_oracle_scheme(key)
    m, k, n = shape
    x = rng.integers(-2, 3, (m, k)).astype(np.float32)
    w = rng.integers(-2, 3, (n, k)).astype(np.float32)
    exact = x.astype(np.int64) @ w.T.astype(np.int64)
    out = O.linear(scheme, x, w, out_dtype="fp32")
    assert np.array_equal(out, exact.astype(np.float32))
    right = np.ascontiguousarray(w.T)
    assert np.array_equal(O.matmul(scheme, x, right, out_dtype="fp32"), exact.astype(np.float32))
    # bias is added after the scheme's sum
    bias = rng.integers(-3, 4, n).astype(np.float32)
    with_bias = O.linear(scheme, x, w, bias=bias, out_dtype="fp32")
    assert np.array_equal(with_bias, (exact + bias.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("key", SCHEME_KEYS)
def test_float64_stages_equal_closed_form(key: str) -> None:
    rng = np.random.default_rng(11)
    scheme = O.load_oracle_scheme(key)
    for m, k, n in ((37, 41, 29), (64, 64, 64)):
        x = rng.standard_normal((m, k))
        w = rng.standard_normal((n, k))
        exact = x @ w.T
        got = O.linear_float64(scheme, x, w)
        assert np.max(np.abs(got - exact)) <= 1e-12 * np.max(np.abs(exact)) * k


def test_planted_sign_error_is_caught() -> None:
    scheme = O.load_oracle_scheme("rank7")
    broken = deepcopy(scheme)
    signal, node = broken.output.assignments[0]
    broken.output.assignments[0] = (signal, ("neg", node))
    rng = np.random.default_rng(5)
    x = rng.integers(-2, 3, (6, 6)).astype(np.float32)
    w = rng.integers(-2, 3, (6, 6)).astype(np.float32)
    exact = (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32)
    assert not np.array_equal(O.linear(broken, x, w, out_dtype="fp32"), exact)
    xr, wr = rng.standard_normal((8, 8)), rng.standard_normal((8, 8))
    assert np.max(np.abs(O.linear_float64(broken, xr, wr) - xr @ wr.T)) > 1e-3
    assert not _brent_ok(broken)
    # the integer check used for the 8x8-block scheme agrees on both
    assert _brent_integer_ok(scheme) and not _brent_integer_ok(broken)
    broken343 = deepcopy(O.load_oracle_scheme("rank343"))
    signal, node = broken343.left.assignments[-1]
    broken343.left.assignments[-1] = (signal, ("neg", node))
    assert not _brent_integer_ok(broken343)


def test_rank343_dense_recombination_matches_the_circuit() -> None:
    """The reference's dense rank-343 recombination (one fp32-accumulated dot) and the
    certificate's output circuit evaluated in fp32 agree to one fp16 rounding; on
    small integers both are exact."""
    scheme = O.load_oracle_scheme("rank343")
    rng = np.random.default_rng(7)
    products = rng.standard_normal((343, 6, 5)).astype(np.float16)
    dense = O.reconstruct_dense(scheme, products, 45, 38, out_dtype="fp32")
    circuit = O.reconstruct(scheme, products, 45, 38, out_dtype="fp32")
    # fp32 summation-order differences only: far below one fp16 ulp of the output
    scale = np.abs(np.einsum("or,rmn->omn", np.abs(np.array(O.program_matrix(scheme.output), dtype=np.float64)),
                             np.abs(products.astype(np.float64)))).max()
    assert np.max(np.abs(dense - circuit)) <= 343 * 2.0**-24 * scale
    assert np.max(np.abs(dense.astype(np.float16).astype(np.float32) -
                         circuit.astype(np.float16).astype(np.float32))) <= 2.0**-10 * np.abs(dense).max()
    x = rng.integers(-2, 3, (37, 29)).astype(np.float16)
    y = rng.integers(-2, 3, (29, 41)).astype(np.float16)
    exact = (x.astype(np.int64) @ y.astype(np.int64)).astype(np.float16)
    for recombination in ("dense", "program"):
        got = O.matmul(scheme, x.astype(np.float32), y.astype(np.float32), recombination=recombination)
        assert np.array_equal(got, exact), recombination


def test_planted_transposed_weight_is_caught() -> None:
    """Reading W instead of W^T blocks (a transposed operand) breaks exactness."""
    scheme = O.load_oracle_scheme("rank49")
    rng = np.random.default_rng(9)
    x = rng.integers(-2, 3, (8, 8)).astype(np.float32)
    w = rng.integers(-2, 3, (8, 8)).astype(np.float32)
    exact = (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32)
    wrong = O.matmul(scheme, x, w, out_dtype="fp32")  # passes W as right[K, N]
    assert not np.array_equal(wrong, exact)


def test_round_to_bf16_matches_torch() -> None:
    rng = np.random.default_rng(1)
    values = np.concatenate(
        [
            rng.standard_normal(100_000).astype(np.float32) * np.float32(1e3),
            rng.standard_normal(10_000).astype(np.float32) * np.float32(1e-40),  # subnormals
            np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1.0 + 2**-8, 1.0 + 3 * 2**-8], dtype=np.float32),
        ]
    )
    # exact ties in both directions
    ties = (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    values = np.concatenate([values, ties, -ties])
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.round_to_bf16(values), expected)
    nan = O.round_to_bf16(np.array([np.nan], dtype=np.float32))
    assert np.isnan(O.bf16_bits_to_f32(nan))[0]


def test_fp16_store_matches_torch() -> None:
    rng = np.random.default_rng(2)
    values = np.concatenate(
        [
            rng.standard_normal(100_000).astype(np.float32) * np.float32(100.0),
            rng.standard_normal(10_000).astype(np.float32) * np.float32(1e-6),  # fp16 subnormals
            np.array([65504.0, 65520.0, 1e6, -1e6], dtype=np.float32),
        ]
    )
    expected = torch.from_numpy(values).to(torch.float16).numpy()
    assert np.array_equal(values.astype(np.float16).view(np.uint16), expected.view(np.uint16))


@pytest.mark.parametrize("key", SCHEME_KEYS)
def test_exact_small_integer_product_with_bf16_planes(key: str) -> None:
    """bf16 planes of small integers are exact; with fp32 products the result is x @ W^T."""
    rng = np.random.default_rng(23)
    scheme = O.load_oracle_scheme(key)
    x = rng.integers(-2, 3, (13, 17)).astype(np.float32)
    w = rng.integers(-2, 3, (11, 17)).astype(np.float32)
    exact = (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32)
    out = O.linear(scheme, x, w, product_dtype="fp32", out_dtype="fp32", plane_dtype="bf16")
    assert np.array_equal(out, exact)
    a = O.left_transform(scheme, x, "bf16")
    assert a.dtype == np.float32 and np.array_equal(a, O.left_transform(scheme, x).astype(np.float32))


def test_bf16_plane_and_product_stores_match_torch() -> None:
    """Planes and products in bf16 are the fp32 value rounded like ``Tensor.to(bfloat16)``."""
    rng = np.random.default_rng(29)
    scheme = O.load_oracle_scheme("rank7")
    x = (rng.standard_normal((40, 36)) * 3).astype(np.float32)
    planes = O.left_transform(scheme, x, "bf16")
    fp32_planes = np.stack(
        [np.asarray(p, dtype=np.float32) for p in O.evaluate_program(scheme.left, O._blocks(x, 2, 20, 18, False))]
    )
    expected = torch.from_numpy(fp32_planes).to(torch.bfloat16).float().numpy()
    assert np.array_equal(planes, expected)
    a = planes[:, :, :16]
    b = planes[:, :12, 2:18]
    products = O.leaf_products(a, b, product_dtype="bf16")
    exact32 = O.leaf_products(a, b, product_dtype="fp32")
    assert np.array_equal(products, torch.from_numpy(exact32).to(torch.bfloat16).float().numpy())


def test_leaf_products_f64_equal_exact_sum() -> None:
    rng = np.random.default_rng(4)
    a = rng.standard_normal((2, 3, 19)).astype(np.float16)
    b = rng.standard_normal((2, 5, 19)).astype(np.float16)
    got = O.leaf_products(a, b, product_dtype="fp32")
    for r in range(2):
        for i in range(3):
            for j in range(5):
                exact = sum(Fraction(float(a[r, i, k])) * Fraction(float(b[r, j, k])) for k in range(19))
                assert got[r, i, j] == np.float32(float(exact))


def test_error_ratio_prediction() -> None:
    """Rank 7 and 48 fit the 1.2x-native bound with fp16 products; rank 49 does not.

    Native BF16 = bf16(fp32 sum of bf16 products). The stated tolerance is
    rel-L2(candidate) <= 1.2 * rel-L2(native) against an fp64 product.
    """
    rng = np.random.default_rng(0)

    def bf16(a: np.ndarray) -> np.ndarray:
        return O.bf16_bits_to_f32(O.round_to_bf16(a.astype(np.float32)))

    m, k, n = 256, 2048, 512
    x = bf16(rng.standard_normal((m, k)))
    w = bf16(rng.standard_normal((n, k)) / np.sqrt(k))
    exact = x.astype(np.float64) @ w.T.astype(np.float64)
    norm = np.linalg.norm(exact)
    native = np.linalg.norm(bf16(x @ w.T) - exact) / norm
    ratios = {}
    for key in SCHEME_KEYS:
        out = O.bf16_bits_to_f32(O.linear(O.load_oracle_scheme(key), x, w))
        ratios[key] = np.linalg.norm(out - exact) / norm / native
    assert ratios["rank7"] < 1.2 and ratios["rank48"] < 1.2
    assert ratios["rank49"] > 1.2


def test_c1_cpu_scheme_path_meets_the_error_bound() -> None:
    """BASELINE C1: rank 7 at 1024^3 through the CPU scheme evaluation (the path
    bench.py's cpu_c1 times), on the BASELINE inputs (seeded CPU torch.Generator,
    x ~ N(0,1), W ~ N(0,1/K), BF16): rel-L2 against an fp64 product within 1.2x
    of native BF16's (fp32 sum of the bf16 inputs, rounded once to bf16), with
    fp32 (BLAS) and near-exact leaf sums alike, and no non-finite values."""
    import torch

    g = torch.Generator().manual_seed(0)
    x = torch.randn((1024, 1024), generator=g).to(torch.bfloat16).float().numpy()
    w = (torch.randn((1024, 1024), generator=g) / 1024**0.5).to(torch.bfloat16).float().numpy()
    exact = x.astype(np.float64) @ w.T.astype(np.float64)
    norm = np.linalg.norm(exact)
    native = np.linalg.norm(O.bf16_bits_to_f32(O.round_to_bf16(x @ w.T)) - exact) / norm
    scheme = O.load_oracle_scheme("rank7")
    for accumulate in ("f32", "f64"):
        out = O.bf16_bits_to_f32(O.linear(scheme, x, w, accumulate=accumulate))
        assert np.isfinite(out).all()
        assert np.linalg.norm(out - exact) / norm <= 1.2 * native
