"""Seeded synthetic inputs for the MoE-layer workloads (CPU generation).

Shapes are GraniteMoE's (granite-3.0-1b-a400m): hidden 1024, 32 experts,
top-8, expert intermediate 512 (EXPLANATION.md of the reference; weight layout
of miniep/weights.py:17-26).  Weights are N(0, 0.02), hidden states N(0, 1).

Skewed routing: the router has no bias (modeling.py:193), so popularity is
put into the inputs.  With p_e proportional to rank(e)^-s under a seeded
expert permutation, every token gets x = z + alpha * u where u is the
minimum-norm solution of W_r u = log p; the logits become W_r z + alpha log p.
alpha is found by bisection so that the hottest expert receives
``target`` times the mean load (at most E/k = 4 for top-8 of 32).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

HIDDEN = 1024
EXPERTS = 32
TOP_K = 8
INTER = 512


@dataclass
class Layer:
    """One MoE layer's inputs (CPU float32 unless noted)."""
    x: torch.Tensor            # (T, H) hidden states entering the MoE block
    w_router: torch.Tensor     # (E, H)
    w_in: torch.Tensor         # (E, 2I, H)  [gate rows | up rows]
    w_out: torch.Tensor        # (E, H, I)
    top_k: int
    alpha: float = 0.0         # input bias strength used for the skew
    zipf_s: float = 0.0


def expert_weights(gen: torch.Generator, n_experts=EXPERTS, hidden=HIDDEN, inter=INTER):
    w_in = torch.randn(n_experts, 2 * inter, hidden, generator=gen) * 0.02
    w_out = torch.randn(n_experts, hidden, inter, generator=gen) * 0.02
    return w_in, w_out


def hottest_over_mean(logits: torch.Tensor, k: int) -> float:
    idx = logits.topk(k, dim=-1).indices.reshape(-1)
    counts = torch.bincount(idx, minlength=logits.shape[1]).double()
    return float(counts.max() / counts.mean())


def zipf_bias(w_router: torch.Tensor, z: torch.Tensor, s: float, k: int, target: float,
              gen: torch.Generator, steps: int = 40):
    """(u, alpha): input direction u with W_r u = log p and the bisected alpha."""
    E = w_router.shape[0]
    perm = torch.randperm(E, generator=gen)
    rank = torch.empty(E)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32)
    logp = -s * torch.log(rank)
    logp = logp - logp.mean()
    u = torch.linalg.lstsq(w_router.double(), logp.double().unsqueeze(1),
                           driver="gelsd").solution.squeeze(1).float()  # min-norm (E < H)
    base = z @ w_router.T
    dir_logits = (u @ w_router.T)
    lo, hi = 0.0, 1.0
    while hottest_over_mean(base + hi * dir_logits, k) < target and hi < 1e4:
        hi *= 2.0
    for _ in range(steps):
        mid = 0.5 * (lo + hi)
        if hottest_over_mean(base + mid * dir_logits, k) < target:
            lo = mid
        else:
            hi = mid
    return u, hi


def make_layer(tokens: int, seed: int = 0, zipf_s: float = 0.0, target: float = 3.9,
               hidden=HIDDEN, n_experts=EXPERTS, top_k=TOP_K, inter=INTER) -> Layer:
    """Seeded layer inputs; zipf_s > 0 skews routing to hottest/mean = target."""
    gen = torch.Generator().manual_seed(seed)
    w_router = torch.randn(n_experts, hidden, generator=gen) * 0.02
    w_in, w_out = expert_weights(gen, n_experts, hidden, inter)
    z = torch.randn(tokens, hidden, generator=gen)
    alpha = 0.0
    if zipf_s > 0:
        u, alpha = zipf_bias(w_router, z, zipf_s, top_k, target, gen)
        z = z + alpha * u
    return Layer(z, w_router, w_in, w_out, top_k, alpha, zipf_s)


def bf16_values(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 and back: the exact values a bf16 model holds."""
    return t.to(torch.bfloat16).to(torch.float32)


# Named workloads: (tokens, zipf s, dtype, sources) -- the single-layer configurations
WORKLOADS = {
    "fp32_layer_t512": dict(tokens=512, zipf_s=0.0, dtype=torch.float32),
    "decode_bf16_t32": dict(tokens=32, zipf_s=0.0, dtype=torch.bfloat16),
    "ep4_share_bf16_t8192_zipf1.1": dict(tokens=8192, zipf_s=1.1, dtype=torch.bfloat16, sources=4),
    "skewed_bf16_t16384_zipf1.2": dict(tokens=16384, zipf_s=1.2, dtype=torch.bfloat16),
}
