"""MoE backends on the HIP kernels, with the reference's backend protocol.

The reference's transformer calls one backend per layer as
    backend(x_flat (N,H), topk_idx (N,k) int64, topk_gate (N,k), valid_mask (N,) bool|None) -> (N,H)
(miniep/modeling.py:131-145, called at :196) after the inline router of
Block.forward (:192-195).  This module provides:

  route(x_flat, w_router, k)   the router hook (modeling.py:192-195)
  HipMoEBackend                drop-in for LocalMoEBackend (modeling.py:131-145)
  HipEPShareBackend            the rank-local part of EPMoEBackend
                               (ep.py:186-249): one GPU's share of a batch
                               sent by S source ranks
  EmulatedEPMoEBackend         EPMoEBackend's result for a `world`-rank
                               placement computed on one GPU (every rank's
                               share in turn, one combine); no collectives
  EPStats                      the counters of ep.py:164-183, device-resident
"""
from __future__ import annotations

import torch

from . import ops
from .placement import Placement


def route(x_flat: torch.Tensor, w_router: torch.Tensor, k: int, return_logits: bool = False):
    """Router of Block.forward (modeling.py:193-195) on the fused HIP kernel."""
    return ops.router_topk(x_flat, w_router, k, return_logits=return_logits)


def _world1_tables(n_experts: int, device):
    table = torch.zeros(n_experts, 1, dtype=torch.int32, device=device)
    n_rep = torch.ones(n_experts, dtype=torch.int32, device=device)
    g2l = torch.arange(n_experts, dtype=torch.int32, device=device)
    return table, n_rep, g2l


class HipMoEBackend:
    """All experts resident on this GPU: LocalMoEBackend (modeling.py:131-145).

    w_in (E, 2I, H), w_out (E, H, I) device tensors in the compute dtype.
    ``check`` synchronises after dispatch to raise on out-of-range expert ids
    (the reference raises when it indexes w_in); switch it off in serving
    loops that must not sync."""

    def __init__(self, w_in: torch.Tensor, w_out: torch.Tensor, check: bool = True):
        if not w_in.is_cuda or not w_out.is_cuda:
            raise RuntimeError("HipMoEBackend needs device-resident expert weights")
        self.w_in = w_in.contiguous()
        self.w_out = w_out.contiguous()
        self.num_experts = w_in.shape[0]
        self.check = check
        self._table, self._n_rep, self._g2l = _world1_tables(self.num_experts, w_in.device)
        self.last_dispatch: ops.Dispatch | None = None

    def __call__(self, x_flat, topk_idx, topk_gate, valid_mask=None):
        disp = ops.dispatch(topk_idx, valid_mask, self.num_experts, self._table, self._n_rep,
                            False, None, 0, self._g2l, self.num_experts, check=self.check)
        self.last_dispatch = disp
        y = ops.grouped_swiglu(x_flat.to(self.w_in.dtype), disp, self.w_in, self.w_out)
        return ops.combine(y, topk_gate, disp.row_of_entry, valid_mask)


class EPStats:
    """Per-rank counters (ep.py:164-183), kept on the device so that updating
    them never synchronises; ``snapshot()`` copies them out."""

    def __init__(self, num_layers: int, num_experts: int, device=None):
        device = device if device is not None else ("cuda" if torch.cuda.is_available() else "cpu")
        self.route_counts = torch.zeros(num_layers, num_experts, dtype=torch.long, device=device)
        self.recv_tokens_per_layer = torch.zeros(num_layers, dtype=torch.long, device=device)
        self.steps = 0

    @property
    def recv_tokens(self) -> int:
        return int(self.recv_tokens_per_layer.sum().item())

    def snapshot(self) -> dict:
        return {
            "recv_tokens": self.recv_tokens,
            "recv_tokens_per_layer": self.recv_tokens_per_layer.tolist(),
            "route_counts": self.route_counts.tolist(),
            "steps": self.steps,
        }


class HipEPShareBackend:
    """One rank's share of an expert-parallel MoE layer (ep.py:186-249 without
    the collectives).

    The batch handed to ``share`` is the concatenation of what S source ranks
    send (``seg_tokens`` = S+1 token offsets; default one source).  Each source
    has its own round-robin counters (one Placement per rank), passed as
    ``rr`` (S, E) int64 or zeros, as after reset_rr() at the start of every
    forward (worker.py:100,115,127).  Entries whose destination is this rank
    are grouped by local expert (sorted global ids, ep.py:69), run through the
    local weights and written to their (token, slot) cell of ``y_entries``.
    """

    def __init__(self, layer: int, placement: Placement, my_rank: int, w_in: torch.Tensor,
                 w_out: torch.Tensor, stats: EPStats | None = None, check: bool = True):
        self.layer = layer
        self.placement = placement
        self.my_rank = my_rank
        self.w_in = w_in.contiguous()
        self.w_out = w_out.contiguous()
        self.stats = stats
        self.check = check
        self._update_map(placement.experts_of_rank(my_rank)[layer])

    def _update_map(self, local_experts: list[int]):
        """g2l: global -> local expert id, -1 if not resident (ep.py:203-208)."""
        if len(local_experts) != self.w_in.shape[0]:
            raise ValueError(f"{len(local_experts)} local experts but w_in holds {self.w_in.shape[0]}")
        self.local_experts = list(local_experts)
        g2l = torch.full((self.placement.num_experts,), -1, dtype=torch.int32)
        for i, e in enumerate(local_experts):
            g2l[e] = i
        self.g2l = g2l.to(self.w_in.device)

    def apply_placement(self, placement: Placement, w_in: torch.Tensor, w_out: torch.Tensor):
        """Swap in a new placement and this rank's re-sliced weights
        (the hot swap of server.py:51-62)."""
        self.placement = placement
        self.w_in, self.w_out = w_in.contiguous(), w_out.contiguous()
        self._update_map(placement.experts_of_rank(self.my_rank)[self.layer])

    def dispatch(self, topk_idx, valid_mask=None, seg_tokens=None, rr=None, want_dest=False):
        n = topk_idx.shape[0]
        seg = [0, n] if seg_tokens is None else [int(v) for v in seg_tokens]
        n_seg = len(seg) - 1
        E = self.placement.num_experts
        table, n_rep = self.placement.tables(self.layer, self.w_in.device)
        has_rep = self.placement.has_replicas(self.layer)
        if has_rep and rr is None:
            rr = torch.zeros(n_seg, E, dtype=torch.long, device=self.w_in.device)
        rc = self.stats.route_counts[self.layer] if self.stats is not None else None
        disp = ops.dispatch(topk_idx, valid_mask, E, table, n_rep, has_rep, rr if has_rep else None,
                            self.my_rank, self.g2l, len(self.local_experts), seg_tokens=seg,
                            route_counts=rc, want_dest=want_dest, check=self.check)
        if self.stats is not None:
            self.stats.recv_tokens_per_layer[self.layer] += disp.offsets[-1].to(torch.long)
        return disp

    def share(self, x_flat, topk_idx, valid_mask=None, seg_tokens=None, rr=None, y_entries=None,
              want_dest=False):
        """(Dispatch, y_entries): this rank's rows and their expert outputs."""
        disp = self.dispatch(topk_idx, valid_mask, seg_tokens, rr, want_dest)
        y = ops.grouped_swiglu(x_flat.to(self.w_in.dtype), disp, self.w_in, self.w_out, y_entries)
        return disp, y


class EmulatedEPMoEBackend:
    """EPMoEBackend's output (ep.py:210-249) for a `world`-rank placement,
    computed on one GPU: each rank's share runs with that rank's own weight
    slice (owned experts + replicas, sorted global ids -- weights.py:54-58),
    every share writes the common (token, slot) buffer, then one combine in
    canonical slot order.  Equal to HipMoEBackend bit for bit for any
    placement, which is the reference's placement-invariance property
    (ep.py:1-8)."""

    def __init__(self, layer: int, placement: Placement, world: int, w_in_full: torch.Tensor,
                 w_out_full: torch.Tensor, check: bool = True):
        self.layer, self.placement, self.world = layer, placement, world
        mine = [placement.experts_of_rank(r)[layer] for r in range(world)]
        self.ranks = [HipEPShareBackend(layer, placement, r, w_in_full[ids], w_out_full[ids],
                                        check=check) for r, ids in enumerate(mine)]

    def __call__(self, x_flat, topk_idx, topk_gate, valid_mask=None, seg_tokens=None, rr=None):
        n, k = topk_idx.shape
        dev = x_flat.device
        y = torch.empty((max(n * k, 1), x_flat.shape[1]), dtype=self.ranks[0].w_in.dtype, device=dev)
        present = torch.full((max(n * k, 1),), -1, dtype=torch.int32, device=dev)
        seg = [0, n] if seg_tokens is None else list(seg_tokens)
        rr0 = (torch.zeros(len(seg) - 1, self.placement.num_experts, dtype=torch.long, device=dev)
               if rr is None else rr)
        for be in self.ranks:
            rr_r = rr0.clone()
            disp, _ = be.share(x_flat, topk_idx, valid_mask, seg, rr_r, y_entries=y)
            present = torch.maximum(present, disp.row_of_entry)
        if rr is not None and self.placement.has_replicas(self.layer):
            rr.copy_(rr_r)
        return ops.combine(y, topk_gate, present, valid_mask)
