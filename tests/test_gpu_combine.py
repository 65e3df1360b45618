"""Combine on the GPU (mep_combine) vs the oracle, with absent cells and masked tokens.

Cells of entries that were not dispatched hold whatever the buffer held: here
NaN, which must never reach an output.  k = 8 runs the kernel that loads every
cell speculatively and skips absent ones with a select; k = 4 the general one,
which loads present cells only.
Bar: max |out - ref| <= tol * max |ref| (1e-5 fp32, 2e-2 bf16); invalid tokens
give exact zeros.
"""
import numpy as np
import pytest
import torch

from helpers import TOL_BF16, TOL_F32, banner, rel_err, to_np
from miniep_amd import ops
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("k", [8, 4])
@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 1024), (torch.float32, 1024), (torch.bfloat16, 1544),
                                     (torch.bfloat16, 4096), (torch.float32, 2048), (torch.float32, 1028)])
def test_combine_absent_cells_and_masks(k, dtype, H):
    """Rows of any length the 16-byte chunks allow (H % 8 bf16, H % 4 fp32),
    including rows longer than one workgroup and rows that straddle two."""
    banner(f"combine k={k} {dtype} H={H}")
    n = 301
    g = torch.Generator().manual_seed(11 + k)
    y = torch.randn(n * k, H, generator=g).to(dtype)
    gate = torch.softmax(torch.randn(n, k, generator=g), -1).to(dtype)
    present = torch.rand(n * k, generator=g) < 0.8
    row = torch.where(present, torch.arange(n * k), torch.full((n * k,), -1)).to(torch.int32)
    valid = torch.rand(n, generator=g) < 0.9
    y_dev = y.clone()
    y_dev[~present] = float("nan")                      # never written by any expert
    out = to_np(ops.combine(y_dev.to(DEV), gate.to(DEV), row.to(DEV), valid.to(DEV))).astype(np.float32)
    keep = present.numpy() & np.repeat(valid.numpy(), k)
    ref = O.combine(y.float().numpy(), gate.float().numpy(), keep, n, k)
    assert np.isfinite(out).all()
    assert (out[~valid.numpy()] == 0).all()
    assert rel_err(out, ref) <= (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)
    # run to run: bitwise identical
    out2 = to_np(ops.combine(y_dev.to(DEV), gate.to(DEV), row.to(DEV), valid.to(DEV))).astype(np.float32)
    assert np.array_equal(out, out2)


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 1024), (torch.bfloat16, 1160), (torch.float32, 2052)])
def test_combine_rows_indexed(dtype, H):
    """mep_combine_rows: cell (t, s) is row row_of_entry[t*k+s] of y (the
    expert-parallel return path), summed in slot order."""
    banner(f"combine_rows {dtype} H={H}")
    n, k = 257, 8
    g = torch.Generator().manual_seed(5)
    present = torch.rand(n * k, generator=g) < 0.75
    m = int(present.sum())
    rows = torch.full((n * k,), -1, dtype=torch.int32)
    rows[present] = torch.randperm(m, generator=g).to(torch.int32)
    y = torch.randn(m, H, generator=g).to(dtype)
    gate = torch.softmax(torch.randn(n, k, generator=g), -1).to(dtype)
    out = to_np(ops.combine_rows(y.to(DEV), gate.to(DEV), rows.to(DEV))).astype(np.float32)
    cells = np.zeros((n * k, H), np.float32)
    cells[present.numpy()] = y.float().numpy()[rows.numpy()[present.numpy()]]
    ref = O.combine(cells, gate.float().numpy(), present.numpy(), n, k)
    assert rel_err(out, ref) <= (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)
