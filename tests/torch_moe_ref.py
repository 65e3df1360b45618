"""Torch restatement of the reference router + LocalMoEBackend for whole-model
tests (test infrastructure only).

Follows miniep/modeling.py: router (:193-195, with fp32 logits as the HIP
router computes them), flatten_topk (:107-117), run_experts (:83-104: stable
grouping by expert, gate|up halves, silu(gate) * up), gate weighting (:144)
and scatter_combine (:120-128: one cell per (token, slot), summed over the
slot axis).  Precision convention of the HIP path: fp32 products, the SwiGLU
activation and each expert output rounded to the model dtype, the gate-weighted
slot sum in fp32 and rounded once.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def torch_route(x_flat: torch.Tensor, w_router: torch.Tensor, k: int):
    logits = x_flat.float() @ w_router.float().T
    vals, idx = logits.topk(k, dim=-1)
    return idx, torch.softmax(vals, dim=-1).to(x_flat.dtype)


class TorchMoERef:
    def __init__(self, w_in: torch.Tensor, w_out: torch.Tensor):
        self.w_in = w_in        # (E, 2I, H)
        self.w_out = w_out      # (E, H, I)

    def __call__(self, x_flat, topk_idx, topk_gate, valid_mask=None):
        n, k = topk_idx.shape
        H = x_flat.shape[1]
        inter = self.w_in.shape[1] // 2
        dev, dt = x_flat.device, x_flat.dtype
        keep = torch.ones(n, dtype=torch.bool, device=dev) if valid_mask is None else valid_mask.to(dev)
        keep_e = keep.repeat_interleave(k)
        ids = topk_idx.reshape(-1)
        tok = torch.arange(n, device=dev).repeat_interleave(k)
        x = x_flat.float()
        y = torch.zeros(n * k, H, dtype=torch.float32, device=dev)
        for e in torch.unique(ids[keep_e]).tolist():
            rows = torch.nonzero((ids == e) & keep_e).squeeze(1)
            h = x[tok[rows]] @ self.w_in[e].float().T
            act = (F.silu(h[:, :inter]) * h[:, inter:]).to(dt).float()
            y[rows] = (act @ self.w_out[e].float().T).to(dt).float()
        g = topk_gate.float() * keep[:, None]
        return (y.view(n, k, H) * g[:, :, None]).sum(dim=1).to(dt)
