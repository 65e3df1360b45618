"""Combine on the GPU (mep_combine) vs the oracle, with absent cells and masked tokens.

Cells of entries that were not dispatched hold whatever the buffer held: here
NaN, which must never reach an output.  k = 8 runs the kernel that loads every
cell speculatively and skips absent ones with a select; k = 4 the staged one.
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
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_combine_absent_cells_and_masks(k, dtype):
    banner(f"combine k={k} {dtype}")
    n, H = 301, 1024
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
