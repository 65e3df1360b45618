"""PyTorch-CPU restatement of the reference MoE block, fp32: the timed CPU
baseline.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/`` and the
``cpu_baseline`` leg of ``bench.py`` use it: the baseline times the
reference's own algorithm with torch on the host cores, in the same process as
the GPU measurement.  The HIP path never calls into it.

It follows the reference's ops one for one:
  route          modeling.py:193-195   logits = x @ W_r^T, topk(k), fp32 softmax
  flatten        modeling.py:107-117   entries t*k+s, invalid tokens dropped
  run_experts    modeling.py:83-104    stable argsort by expert, counts of the
                                       non-empty experts, per-expert
                                       (silu(x W_g^T) * x W_u^T) W_out^T
  gate + combine modeling.py:120-128,144  gated rows into (token, slot) cells,
                                       sum over the slot axis
and is pinned against the numpy oracle (tests/test_oracle.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def route(x: torch.Tensor, w_router: torch.Tensor, k: int):
    """(topk_idx (N,k) int64, topk_gate (N,k)) of modeling.py:193-195."""
    vals, idx = (x @ w_router.T).topk(k, dim=-1)
    return idx, torch.softmax(vals.float(), dim=-1).to(x.dtype)


def moe_local(x: torch.Tensor, topk_idx: torch.Tensor, topk_gate: torch.Tensor,
              w_in: torch.Tensor, w_out: torch.Tensor, valid_mask: torch.Tensor | None = None) -> torch.Tensor:
    """LocalMoEBackend.__call__ (modeling.py:138-145) -> (N, H)."""
    n, k = topk_idx.shape
    H = x.shape[1]
    keep = torch.ones(n, dtype=torch.bool) if valid_mask is None else valid_mask
    keep_flat = keep.repeat_interleave(k)
    tok = torch.arange(n).repeat_interleave(k)[keep_flat]
    slot = torch.arange(k).repeat(n)[keep_flat]
    experts = topk_idx.reshape(-1)[keep_flat]
    rows = x[tok]
    y = torch.zeros(rows.shape[0], H, dtype=x.dtype)
    if rows.shape[0]:
        order = torch.argsort(experts, stable=True)
        ids, counts = torch.unique_consecutive(experts[order], return_counts=True)
        inter = w_in.shape[1] // 2
        start = 0
        for e, c in zip(ids.tolist(), counts.tolist()):
            sel = order[start:start + c]
            start += c
            h = rows[sel] @ w_in[e].T
            y[sel] = (F.silu(h[:, :inter]) * h[:, inter:]) @ w_out[e].T
    cells = torch.zeros(n, k, H, dtype=x.dtype)
    cells[tok, slot] = y * topk_gate.reshape(-1)[keep_flat].unsqueeze(1)
    return cells.sum(dim=1)


def moe_block(x, w_router, w_in, w_out, k, valid_mask=None):
    """Router + LocalMoEBackend: what Block.forward runs after its
    post-attention norm (modeling.py:192-196), without the residual."""
    idx, gate = route(x, w_router, k)
    return moe_local(x, idx, gate, w_in, w_out, valid_mask)
