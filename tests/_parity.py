"""Parity helpers shared by the GPU tests: BASELINE inputs, sampled oracle checks.

The sampled check compares a plan's intermediate buffers with the oracle on a
sample of block rows and block columns: the oracle transforms only the input
rows those planes read, so it stays cheap at any matrix size.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import fastmm_oracle as O


def baseline_inputs(rows: int, inner: int, columns: int, bias: bool, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((rows, inner), generator=g).to(torch.bfloat16)
    w = (torch.randn((columns, inner), generator=g) / inner**0.5).to(torch.bfloat16)
    b = (torch.randn((columns,), generator=g) * 0.02).to(torch.bfloat16) if bias else None
    return x, w, b


def sample_block_indices(size: int, count: int, rng: np.random.Generator, extent: int, s: int) -> np.ndarray:
    """First and last block rows, the last valid row of each of the s blocks of a
    dimension of ``extent`` (ragged edges), the leaf GEMM's tile edges, and random ones."""
    chosen = {min(size, extent - i * size) - 1 for i in range(s) if extent > i * size}
    chosen |= {v for v in (0, 1, size // 2, size - 2, size - 1, 15, 16, 255, 256, 257, (size // 256) * 256)
               if 0 <= v < size}
    chosen |= set(rng.choice(size, size=min(count, size), replace=False).tolist())
    index = np.array(sorted(chosen), dtype=np.int64)
    assert index.size and index[0] >= 0 and index[-1] < size, (size, index)
    return index


def device_index(index: np.ndarray, size: int, device: torch.device) -> torch.Tensor:
    """``index`` as a device tensor, checked on the host first: an out-of-range index
    in a GPU gather would trip torch's device-side bound check and end the process."""
    assert index.size and int(index.min()) >= 0 and int(index.max()) < size, (size, index)
    return torch.from_numpy(index).to(device)


def source_rows(source: torch.Tensor, s: int, block: int, index: np.ndarray):
    """Rows i*block + index of ``source`` for i < s, zero past its end (fp32).

    Transforming this [s*len(index), K] matrix gives exactly the planes' rows
    ``index`` (block i of the sub-matrix holds block i's sampled rows)."""
    rows = (np.arange(s)[:, None] * block + index[None, :]).reshape(-1)
    valid = rows < source.shape[0]
    out = np.zeros((rows.size, source.shape[1]), dtype=np.float32)
    out[valid] = source[torch.from_numpy(rows[valid])].float().numpy()
    return out, rows, valid


def gather_plane_rows(buffer: torch.Tensor, rank: int, rows: int, inner: int, index: np.ndarray) -> np.ndarray:
    """Plane rows ``index`` of an operand buffer (either layout) as int16 bits [R, n, inner]."""
    at = device_index(index, rows, buffer.device)
    if inner % 32 == 0:
        view = buffer.view(rank, inner // 32, rows, 32)[:, :, at, :].permute(0, 2, 1, 3).reshape(rank, -1, inner)
    else:
        view = buffer.view(rank, rows, inner)[:, at, :]
    return view.contiguous().view(torch.int16).cpu().numpy()


def rel_l2(candidate: torch.Tensor, exact: torch.Tensor) -> float:
    return float(torch.linalg.vector_norm(candidate.double() - exact) / torch.linalg.vector_norm(exact))


def check_sampled_stages(plan, scheme, x, w, b, workspace, output, rng, plane: str = "fp16") -> None:
    """A'/B' bits, products within bound and output bits on a block-row x block-column sample.

    ``plane`` is the plan's compute type: ``"fp16"`` (fp16 planes and products) or
    ``"bf16"`` (the rank-49 BF16-leaf pair: bf16 planes, BF16 MFMA, bf16 products)."""
    s, rank = plan.scheme_size, plan.rank
    shape = plan.shape
    mb, kb, nb = shape.block_rows, shape.block_inner, shape.block_columns
    ri = sample_block_indices(mb, 12, rng, shape.rows, s)
    ci = sample_block_indices(nb, 12, rng, shape.columns, s)
    x_sub, out_rows, row_ok = source_rows(x, s, mb, ri)
    w_sub, out_cols, col_ok = source_rows(w, s, nb, ci)
    a = O.left_transform(scheme, x_sub, plane)
    bt = O.weight_transform(scheme, w_sub, plane)
    assert a.shape == (rank, ri.size, kb) and bt.shape == (rank, ci.size, kb)

    def bits(planes: np.ndarray) -> np.ndarray:  # fp16 values, or fp32 holding bf16 values
        return planes.view(np.int16) if plane == "fp16" else O.round_to_bf16(planes).view(np.int16)

    left_bits = gather_plane_rows(workspace.left_transformed, rank, mb, kb, ri)
    right_bits = gather_plane_rows(workspace.right_transformed, rank, nb, kb, ci)
    assert np.array_equal(left_bits, bits(a)), "A' differs from the oracle"
    assert np.array_equal(right_bits, bits(bt)), "B' differs from the oracle"

    device = workspace.products.device
    at_r, at_c = device_index(ri, mb, device), device_index(ci, nb, device)
    sampled = workspace.products[:, at_r][:, :, at_c]
    products = sampled.cpu().numpy() if plane == "fp16" else sampled.float().cpu().numpy()
    exact = O.leaf_products(a, bt, product_dtype="fp32").astype(np.float64)
    magnitude = np.matmul(np.abs(a.astype(np.float64)), np.abs(np.swapaxes(bt.astype(np.float64), 1, 2)))
    # fp32 accumulation over Kb terms, then one rounding to the products' type
    unit, tiny = (2.0**-11, 2.0**-24) if plane == "fp16" else (2.0**-8, 2.0**-126)
    bound = kb * 2.0**-24 * magnitude + np.abs(exact) * unit + tiny
    assert np.all(np.abs(products.astype(np.float64) - exact) <= bound), "leaf products outside the bound"

    bias_sub = None
    if b is not None:
        bias_sub = np.zeros(out_cols.size, dtype=np.float32)
        bias_sub[col_ok] = b[torch.from_numpy(out_cols[col_ok])].float().numpy()
    recombined = O.reconstruct(scheme, products, out_rows.size, out_cols.size, bias_sub, "bf16")
    gpu_rows = device_index(out_rows[row_ok], output.shape[0], output.device)
    gpu_cols = device_index(out_cols[col_ok], output.shape[1], output.device)
    got = output[gpu_rows][:, gpu_cols].view(torch.int16).cpu().numpy()
    want = recombined[row_ok][:, col_ok].view(np.int16)
    assert np.array_equal(got, want), "output differs from the oracle's recombination of the GPU's products"
