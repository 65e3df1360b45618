"""GraniteMoE-shaped transformer whose MoE blocks run through a pluggable router
hook and one MoE backend per layer -- with the HIP path, ``route`` +
``HipMoEBackend`` on every layer.

Follows the reference model (miniep/modeling.py):
  * ``ModelConfig`` fields and ``from_json`` -- modeling.py:25-52;
  * RMSNorm, llama RoPE (rotate-half) -- :55-80;
  * ``Block.forward``: pre-norm attention with GQA and ``attention_multiplier``
    as the score scale, residual scaled by ``residual_multiplier``, post-norm,
    router, MoE backend, scaled residual -- :146-197;
  * model: embeddings x ``embedding_multiplier``, final norm, tied LM head
    divided by ``logits_scaling``, optional last-position-only logits -- :218-254;
  * greedy decoding -- :249-262 (batched here: equal-length prompts decode
    together, one token per sequence per step).
Weights use the checkpoint's key names (weights.py:17-26), so a loaded
checkpoint dict drops in.

Choices made here (not fixed by the reference): the KV cache is preallocated per layer and written in
place (no concatenation per decode step); attention runs in fp32 (batched
bf16 products with transposed operands are avoided on ROCm); the LM head is
computed in fp32 for the positions asked for; router logits are fp32 (the
router hook decides, see ``backend.route``).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Callable, Sequence

import torch
import torch.nn.functional as F


@dataclass
class ModelConfig:
    """Field names and meaning as the reference's ModelConfig (modeling.py:25-47)."""
    hidden_size: int = 1024
    intermediate_size: int = 512
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    num_local_experts: int = 32
    num_experts_per_tok: int = 8
    vocab_size: int = 49155
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    embedding_multiplier: float = 12.0
    attention_multiplier: float = 0.015625
    residual_multiplier: float = 0.22
    logits_scaling: float = 6.0
    max_position_embeddings: int = 4096
    eos_token_id: int = 0
    pad_token_id: int = 0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @staticmethod
    def from_json(path: str | Path) -> "ModelConfig":
        raw = json.loads(Path(path).read_text())
        return ModelConfig(**{f.name: raw[f.name] for f in fields(ModelConfig) if f.name in raw})


def layer_keys(layer: int) -> dict[str, str]:
    p = f"model.layers.{layer}."
    return {
        "input_ln": p + "input_layernorm.weight",
        "post_ln": p + "post_attention_layernorm.weight",
        "wq": p + "self_attn.q_proj.weight",
        "wk": p + "self_attn.k_proj.weight",
        "wv": p + "self_attn.v_proj.weight",
        "wo": p + "self_attn.o_proj.weight",
        "router": p + "block_sparse_moe.router.layer.weight",
        "w_in": p + "block_sparse_moe.input_linear.weight",
        "w_out": p + "block_sparse_moe.output_linear.weight",
    }


def random_weights(cfg: ModelConfig, seed: int = 0, dtype=torch.bfloat16, device="cpu",
                   std: float = 0.02, expert_std: tuple[float, float] | None = None) -> dict[str, torch.Tensor]:
    """Seeded random-init weights, N(0, std) matrices and unit norm weights,
    drawn layer by layer on the CPU generator, then cast and moved.
    ``expert_std`` = (input_linear std, output_linear std) overrides `std` for
    the experts: with N(0, 0.02) everywhere the x12 embedding dominates the
    residual stream of a random model, which then mostly repeats its input
    token whatever its MoE blocks compute."""
    s_in, s_out = expert_std if expert_std is not None else (std, std)
    g = torch.Generator().manual_seed(seed)
    H, I, E = cfg.hidden_size, cfg.intermediate_size, cfg.num_local_experts
    d, hq, hk = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads

    def mat(*shape, sd=std):
        return (torch.randn(*shape, generator=g) * sd).to(dtype).to(device)

    w = {"model.embed_tokens.weight": mat(cfg.vocab_size, H),
         "model.norm.weight": torch.ones(H, dtype=dtype, device=device)}
    for layer in range(cfg.num_hidden_layers):
        k = layer_keys(layer)
        w[k["input_ln"]] = torch.ones(H, dtype=dtype, device=device)
        w[k["post_ln"]] = torch.ones(H, dtype=dtype, device=device)
        w[k["wq"]] = mat(hq * d, H)
        w[k["wk"]] = mat(hk * d, H)
        w[k["wv"]] = mat(hk * d, H)
        w[k["wo"]] = mat(H, hq * d)
        w[k["router"]] = mat(E, H)
        w[k["w_in"]] = mat(E, 2 * I, H, sd=s_in)
        w[k["w_out"]] = mat(E, H, I, sd=s_out)
    return w


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * x / sqrt(mean(x^2) + eps), computed in fp32, returned in x.dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (weight.float() * y).to(x.dtype)


class RotaryTable:
    """cos / sin of llama RoPE for every position, fp32, on the model's device."""

    def __init__(self, cfg: ModelConfig, device):
        d = cfg.head_dim
        inv = cfg.rope_theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
        ang = torch.arange(cfg.max_position_embeddings, dtype=torch.float64)[:, None] * inv[None, :]
        ang = torch.cat([ang, ang], dim=-1)
        self.cos = ang.cos().float().to(device)
        self.sin = ang.sin().float().to(device)

    def rotate(self, t: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """t: (B, heads, T, d) fp32; positions: (B, T)."""
        cos = self.cos[positions][:, None]
        sin = self.sin[positions][:, None]
        half = t.shape[-1] // 2
        rot = torch.cat([-t[..., half:], t[..., :half]], dim=-1)
        return t * cos + rot * sin


class KVCache:
    """Per-layer K/V buffers preallocated for `max_len` positions, (B, Hk, max_len, d)."""

    def __init__(self, cfg: ModelConfig, batch: int, max_len: int, device, dtype=torch.float32):
        shape = (batch, cfg.num_key_value_heads, max_len, cfg.head_dim)
        self.k = [torch.empty(shape, dtype=dtype, device=device) for _ in range(cfg.num_hidden_layers)]
        self.v = [torch.empty(shape, dtype=dtype, device=device) for _ in range(cfg.num_hidden_layers)]
        self.length = 0                  # positions filled (same for every layer after a forward)
        self.max_len = max_len

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        t = k.shape[2]
        if self.length + t > self.max_len:
            raise ValueError(f"KV cache full: {self.length} + {t} > {self.max_len}")
        self.k[layer][:, :, self.length:self.length + t] = k
        self.v[layer][:, :, self.length:self.length + t] = v
        return self.k[layer][:, :, :self.length + t], self.v[layer][:, :, :self.length + t]


Router = Callable[[torch.Tensor, torch.Tensor, int], tuple[torch.Tensor, torch.Tensor]]


class GraniteMoeModel:
    """weights: checkpoint-keyed dict; router: (x_flat, w_router, k) -> (topk_idx,
    topk_gate); moe_backends: one callable per layer with the LocalMoEBackend
    protocol (x_flat, topk_idx, topk_gate, valid_mask) -> (N, H).  With
    ``fuse_router``, a backend that has ``route_and_call`` runs the router
    itself (the fused router + dispatch of HipMoEBackend)."""

    def __init__(self, cfg: ModelConfig, weights: dict, router: Router, moe_backends: Sequence,
                 fuse_router: bool = False):
        if len(moe_backends) != cfg.num_hidden_layers:
            raise ValueError(f"{len(moe_backends)} MoE backends for {cfg.num_hidden_layers} layers")
        self.cfg = cfg
        self.w = weights
        self.router = router
        self.moe = list(moe_backends)
        # backends with route_and_call run the router hook themselves (same results)
        self.fuse_router = fuse_router
        self.embed = weights["model.embed_tokens.weight"]
        self.rope = RotaryTable(cfg, self.embed.device)
        self._head: torch.Tensor | None = None

    def _attention(self, layer: int, x: torch.Tensor, positions: torch.Tensor, cache: KVCache | None,
                   attn_mask: torch.Tensor | None) -> torch.Tensor:
        cfg, k_ = self.cfg, layer_keys(layer)
        B, T, H = x.shape
        d, hq, hk = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
        x2 = x.reshape(B * T, H)
        q = F.linear(x2, self.w[k_["wq"]]).float().view(B, T, hq, d).transpose(1, 2)
        k = F.linear(x2, self.w[k_["wk"]]).float().view(B, T, hk, d).transpose(1, 2)
        v = F.linear(x2, self.w[k_["wv"]]).float().view(B, T, hk, d).transpose(1, 2)
        q = self.rope.rotate(q, positions)
        k = self.rope.rotate(k, positions)
        if cache is not None:
            k, v = cache.write(layer, k, v)
        k = k.repeat_interleave(hq // hk, dim=1)
        v = v.repeat_interleave(hq // hk, dim=1)
        S = k.shape[2]
        if attn_mask is None:
            # queries sit at the last T of the S key positions (causal, bottom-right aligned)
            qpos = torch.arange(S - T, S, device=x.device)[:, None]
            attn_mask = torch.arange(S, device=x.device)[None, :] <= qpos
        o = F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v.contiguous(),
                                           attn_mask=attn_mask, scale=cfg.attention_multiplier)
        o = o.transpose(1, 2).reshape(B * T, hq * d).to(x.dtype)
        return F.linear(o, self.w[k_["wo"]]).view(B, T, H)

    def _block(self, layer: int, h: torch.Tensor, positions, cache, attn_mask, moe_valid) -> torch.Tensor:
        cfg, k_ = self.cfg, layer_keys(layer)
        x = rms_norm(h, self.w[k_["input_ln"]], cfg.rms_norm_eps)
        h = h + self._attention(layer, x, positions, cache, attn_mask) * cfg.residual_multiplier
        x = rms_norm(h, self.w[k_["post_ln"]], cfg.rms_norm_eps)
        B, T, H = x.shape
        x_flat = x.reshape(B * T, H)
        fused = getattr(self.moe[layer], "route_and_call", None) if self.fuse_router else None
        if fused is not None:
            moe_out, _, _ = fused(x_flat, self.w[k_["router"]], cfg.num_experts_per_tok, moe_valid)
        else:
            topk_idx, topk_gate = self.router(x_flat, self.w[k_["router"]], cfg.num_experts_per_tok)
            moe_out = self.moe[layer](x_flat, topk_idx, topk_gate, valid_mask=moe_valid)
        return h + moe_out.view(B, T, H) * cfg.residual_multiplier

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, cache: KVCache | None = None, positions=None,
                attn_mask=None, moe_valid=None, logits_at: torch.Tensor | None = None) -> torch.Tensor:
        """input_ids (B, T) -> fp32 logits (B, T, V), or (B, 1, V) at `logits_at` (B,)."""
        cfg = self.cfg
        B, T = input_ids.shape
        if positions is None:
            start = cache.length if cache is not None else 0
            positions = torch.arange(start, start + T, device=input_ids.device).expand(B, T)
        if moe_valid is not None:
            moe_valid = moe_valid.reshape(-1)
        h = self.embed[input_ids] * cfg.embedding_multiplier
        for layer in range(cfg.num_hidden_layers):
            h = self._block(layer, h, positions, cache, attn_mask, moe_valid)
        if cache is not None:
            cache.length += T
        if logits_at is not None:
            h = h[torch.arange(B, device=h.device), logits_at][:, None]
        h = rms_norm(h, self.w["model.norm.weight"], cfg.rms_norm_eps)
        if self._head is None:
            self._head = self.embed.float()            # tied LM head, fp32 copy made once
        return F.linear(h.float(), self._head) / cfg.logits_scaling

    __call__ = forward


def greedy_generate(model: GraniteMoeModel, prompts: torch.Tensor, new_tokens: int,
                    forced: torch.Tensor | None = None, return_logits: bool = False):
    """Batched greedy decoding of equal-length prompts (B, T).

    Returns (tokens (B, new_tokens), margins (B, new_tokens)): the argmax token
    of every step and the gap between the best and second-best logit there;
    with ``return_logits`` also the last-position logits of every step
    (B, new_tokens, V).  With `forced` (B, new_tokens), those tokens are fed
    back instead of the argmax (teacher forcing), so two models can be
    compared decision by decision on the same inputs.
    """
    B, T = prompts.shape
    cache = KVCache(model.cfg, B, T + new_tokens, prompts.device)
    logits = model(prompts, cache=cache, logits_at=torch.full((B,), T - 1, device=prompts.device))
    toks, margins, steps = [], [], []
    for step in range(new_tokens):
        last = logits[:, -1]
        top2 = last.topk(2, dim=-1)
        toks.append(top2.indices[:, 0])
        margins.append(top2.values[:, 0] - top2.values[:, 1])
        if return_logits:
            steps.append(last.clone())
        nxt = toks[-1] if forced is None else forced[:, step]
        if step + 1 < new_tokens:
            logits = model(nxt[:, None], cache=cache)
    out = (torch.stack(toks, 1), torch.stack(margins, 1))
    return out + (torch.stack(steps, 1),) if return_logits else out


def build_hip_model(cfg: ModelConfig, weights: dict, check: bool = False) -> GraniteMoeModel:
    """The model with every MoE block on the HIP path: ``route`` (fused router
    kernel, fp32 logits) and one ``HipMoEBackend`` per layer, each block's
    router and dispatch run as one fused call (``route_and_call``)."""
    from .backend import HipMoEBackend, route

    backends = []
    for layer in range(cfg.num_hidden_layers):
        k = layer_keys(layer)
        backends.append(HipMoEBackend(weights[k["w_in"]], weights[k["w_out"]], check=check))
    return GraniteMoeModel(cfg, weights, route, backends, fuse_router=True)


__all__ = ["ModelConfig", "layer_keys", "random_weights", "rms_norm", "RotaryTable", "KVCache",
           "GraniteMoeModel", "greedy_generate", "build_hip_model"]
