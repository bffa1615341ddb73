"""fastmm_leaf_products_noalloc against fastmm_leaf_products, through the C ABI.

The allocation-free entry point runs the same kernels with the split-K tail's
fp32 parts in the library's own device array instead of caller scratch, so
its products must be the same bits as the scratch-taking entry point's given
enough scratch. Two calls in a row on one GPU (the second smaller, so the
array still holds the first call's parts) must both match; so must shapes
with no tail, fp32 products, the generic kernel, and the largest tail a
256-CU device plans (192 parts = the whole array).
"""

import ctypes

import pytest
import torch

from rdna3_fastmm import _native
from rdna3_fastmm._stages import leaf_scratch_bytes

pytestmark = pytest.mark.gpu
DEVICE = torch.device("cuda", 0)
STATIC_SCRATCH_BYTES = 48 << 20


def _operands(rank: int, mb: int, kb: int, nb: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((rank, mb, kb), generator=g).to(torch.float16).to(DEVICE)
    b = torch.randn((rank, nb, kb), generator=g).to(torch.float16).to(DEVICE)
    return a, b


def _with_scratch(a, b, products, rank, mb, kb, nb) -> int:
    need = leaf_scratch_bytes(rank, a.dtype, products.dtype, mb, kb, nb, DEVICE)
    scratch = torch.empty(max(need, 1), device=DEVICE, dtype=torch.uint8)
    _native.call("fastmm_leaf_products", rank, _native.dtype_code(a.dtype), a.data_ptr(), b.data_ptr(),
                 products.data_ptr(), _native.dtype_code(products.dtype), mb, kb, nb,
                 scratch.data_ptr() if need else None, need, _native.stream_handle(DEVICE))
    torch.cuda.synchronize()
    return need


def _no_alloc(a, b, products, rank, mb, kb, nb) -> None:
    _native.call("fastmm_leaf_products_noalloc", rank, _native.dtype_code(a.dtype), a.data_ptr(), b.data_ptr(),
                 products.data_ptr(), _native.dtype_code(products.dtype), mb, kb, nb, _native.stream_handle(DEVICE))


# (rank, Mb, Kb, Nb): split tails of 56 tiles x 3 parts (42 MiB) then 28 x 4 (28 MiB),
# the 192-part maximum (64 tiles x 3 = 48 MiB), no tail (256 tiles), and the generic kernel.
SEQUENCE = ((7, 1024, 512, 512), (7, 512, 512, 512), (1, 2048, 512, 2048), (4, 2048, 256, 2048), (3, 100, 72, 88))


@pytest.mark.parametrize("products_dtype", (torch.float16, torch.float32))
def test_no_alloc_products_equal_the_scratch_entry_point(products_dtype) -> None:
    needs = []
    for index, (rank, mb, kb, nb) in enumerate(SEQUENCE):
        print(f"\n[case] no-alloc {products_dtype} rank={rank} Mb={mb} Kb={kb} Nb={nb}", flush=True)
        a, b = _operands(rank, mb, kb, nb, seed=index)
        expected = torch.empty((rank, mb, nb), device=DEVICE, dtype=products_dtype)
        needs.append(_with_scratch(a, b, expected, rank, mb, kb, nb))
        got = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=products_dtype)
        torch.cuda.synchronize()
        _no_alloc(a, b, got, rank, mb, kb, nb)
        torch.cuda.synchronize()
        assert torch.equal(got, expected), f"no-alloc products differ at {(rank, mb, kb, nb)}"
    # the sequence exercised shrinking tails and the whole array
    assert needs[0] > needs[1] > 0 and needs[2] == STATIC_SCRATCH_BYTES and needs[3] == needs[4] == 0


@pytest.mark.parametrize(
    "dims",
    (
        (7, 4107, 256, 2304),  # a last tile row of 11 rows fused into the persistent kernel
        (40, 4096, 256, 4096),  # 1.34 GB of products, stored non-temporally
    ),
)
def test_no_alloc_runs_the_strip_and_streamed_forms(dims) -> None:
    rank, mb, kb, nb = dims
    print(f"\n[case] no-alloc {dims}", flush=True)
    a, b = _operands(rank, mb, kb, nb, seed=sum(dims))
    expected = torch.empty((rank, mb, nb), device=DEVICE, dtype=torch.float16)
    assert _with_scratch(a, b, expected, rank, mb, kb, nb) == 0
    got = torch.full((rank, mb, nb), float("nan"), device=DEVICE, dtype=torch.float16)
    torch.cuda.synchronize()
    _no_alloc(a, b, got, rank, mb, kb, nb)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)


def test_no_alloc_allocates_nothing() -> None:
    """No allocation through torch's allocator, and the driver's free memory unchanged
    beyond what the library's own array took on its first use."""
    rank, mb, kb, nb = 7, 1024, 512, 512
    a, b = _operands(rank, mb, kb, nb, seed=9)
    products = torch.empty((rank, mb, nb), device=DEVICE, dtype=torch.float16)
    _no_alloc(a, b, products, rank, mb, kb, nb)  # first use on this device
    torch.cuda.synchronize()
    allocated = torch.cuda.memory_allocated(DEVICE)
    free_before, _ = torch.cuda.mem_get_info(DEVICE)
    for _ in range(3):
        _no_alloc(a, b, products, rank, mb, kb, nb)
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info(DEVICE)
    assert torch.cuda.memory_allocated(DEVICE) == allocated
    assert free_after == free_before


def test_no_alloc_reports_argument_errors() -> None:
    lib = _native.library()
    status = lib.fastmm_leaf_products_noalloc(7, 1, None, 16, 16, 1, 2, 2, 2, None)
    assert status == 1 and b"null pointer" in lib.fastmm_last_error()
    size = ctypes.c_int64(0)
    assert lib.fastmm_leaf_scratch_bytes(1, 1, 1, 2048, 512, 2048, ctypes.byref(size)) == 0
    assert size.value <= STATIC_SCRATCH_BYTES
