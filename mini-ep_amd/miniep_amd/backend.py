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

from dataclasses import dataclass

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
    ``check=True`` synchronises after the dispatch and again after the
    experts: it raises on out-of-range expert ids (the reference raises when
    it indexes w_in) and on a kernel wait that gave up (whose outputs are
    NaN).  Off by default, so that a call never synchronises the host."""

    def __init__(self, w_in: torch.Tensor, w_out: torch.Tensor, check: bool = False):
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
        out = ops.grouped_swiglu_combine(x_flat.to(self.w_in.dtype), disp, self.w_in, self.w_out, topk_gate,
                                         valid_mask)
        if self.check:
            ops.experts_check(out.device)
        return out

    def route_and_call(self, x_flat, w_router, k, valid_mask=None):
        """The router hook and this backend in one go (Block.forward,
        modeling.py:193-196) through ops.moe_layer: the router kernel also
        builds the dispatch, and decode batches run router, experts and
        combine as one launch; same results as route() + __call__.  Returns
        (out, topk_idx, topk_gate)."""
        x = x_flat.to(self.w_in.dtype)
        out, idx, gate, disp = ops.moe_layer(x, w_router, k, self.w_in, self.w_out, valid_mask)
        self.last_dispatch = disp
        if self.check:
            ops.dispatch_check(out.device)
            ops.experts_check(out.device)
        return out, idx, gate


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

    def __init__(self, layer: int, placement: Placement, my_rank: int, w_in: torch.Tensor | None = None,
                 w_out: torch.Tensor | None = None, stats: EPStats | None = None, check: bool = True,
                 store=None):
        self.layer = layer
        self.placement = placement
        self.my_rank = my_rank
        self.stats = stats
        self.check = check
        self.w_slot = None
        if store is not None:
            self.use_store(placement, store)
        else:
            if w_in is None or w_out is None:
                raise ValueError("give the rank's expert weights or an ExpertStore")
            self.w_in = w_in.contiguous()
            self.w_out = w_out.contiguous()
            self._update_map(placement.experts_of_rank(my_rank)[layer])

    def _update_map(self, local_experts: list[int]):
        """g2l: global -> local expert id, -1 if not resident (ep.py:203-208)."""
        if self.w_slot is None and len(local_experts) != self.w_in.shape[0]:
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
        self.w_slot = None
        self._update_map(placement.experts_of_rank(self.my_rank)[self.layer])

    def use_store(self, placement: Placement, store) -> None:
        """Read this layer's experts from an ExpertStore's slots (whose resident
        set must be the placement's experts of this rank)."""
        local = placement.experts_of_rank(self.my_rank)[self.layer]
        if store.local_experts[self.layer] != local:
            raise ValueError(f"layer {self.layer}: the store holds {store.local_experts[self.layer]}, "
                             f"the placement gives rank {self.my_rank} {local}")
        self.placement = placement
        self.w_in, self.w_out, self.w_slot = store.layer_weights(self.layer)
        self._update_map(local)

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

    def send(self, x_flat, topk_idx, valid_mask=None, rr=None) -> "SendBatch":
        """Sender half of EPMoEBackend.__call__ (ep.py:216-226) for this rank's
        own tokens: route_counts, destinations with this rank's round-robin
        counters `rr` (1, E) (zeros = after reset_rr), the destination-sorted
        order (stable), the send counts per rank, the inverse order, and the
        send buffer (rows of x and their experts) in that order."""
        n, k = topk_idx.shape
        dev = self.w_in.device
        E = self.placement.num_experts
        world = self.placement.world
        table, n_rep = self.placement.tables(self.layer, dev)
        has_rep = self.placement.has_replicas(self.layer)
        if has_rep and rr is None:
            rr = torch.zeros(1, E, dtype=torch.long, device=dev)
        rc = self.stats.route_counts[self.layer] if self.stats is not None else None
        nobody = torch.full((E,), -1, dtype=torch.int32, device=dev)
        d = ops.dispatch(topk_idx, valid_mask, E, table, n_rep, has_rep, rr if has_rep else None, -1,
                         nobody, 0, route_counts=rc, want_dest=True, check=self.check)
        # the destination-sorted order is the dispatch itself keyed by destination
        key = d.dest[: n * k].clamp(min=0).view(n, k).to(torch.int64)   # masked entries stay masked
        t1, r1, ident = _world1_tables(world, dev)
        srt = ops.dispatch(key, valid_mask, world, t1, r1, False, None, 0, ident, world, check=False)
        m = int(srt.offsets[-1])
        send_x, send_ids = ops.gather_rows(x_flat.to(self.w_in.dtype), srt.perm, m, k, topk_idx)
        return SendBatch(send_x, send_ids, srt.counts, srt.row_of_entry, m)

    def receive(self, recv_x, recv_experts) -> torch.Tensor:
        """Receiver half (ep.py:228-231): the rows that arrived, one expert each,
        through this rank's resident experts; outputs in arrival order.  A row
        for an expert not resident here raises NotResidentError (ep.py:230)."""
        n = recv_x.shape[0]
        dev = self.w_in.device
        if n == 0:
            return torch.empty(0, recv_x.shape[1], dtype=self.w_in.dtype, device=dev)
        E = self.placement.num_experts
        t1, r1, _ = _world1_tables(E, dev)
        d = ops.dispatch(recv_experts.view(n, 1), None, E, t1, r1, False, None, 0, self.g2l,
                         len(self.local_experts), check=self.check)
        if self.stats is not None:
            self.stats.recv_tokens_per_layer[self.layer] += d.offsets[-1].to(torch.long)
        return ops.grouped_swiglu(recv_x.to(self.w_in.dtype), d, self.w_in, self.w_out, w_slot=self.w_slot)

    def share(self, x_flat, topk_idx, valid_mask=None, seg_tokens=None, rr=None, y_entries=None,
              want_dest=False):
        """(Dispatch, y_entries): this rank's rows and their expert outputs."""
        disp = self.dispatch(topk_idx, valid_mask, seg_tokens, rr, want_dest)
        y = ops.grouped_swiglu(x_flat.to(self.w_in.dtype), disp, self.w_in, self.w_out, y_entries,
                               w_slot=self.w_slot)
        return disp, y


@dataclass
class SendBatch:
    """What one rank sends: rows (m, H) and their experts (m,) grouped by
    destination rank, `send_counts` (world,) rows per destination, and `inv`
    (N*k,) the row of each of its entries in the send order (-1 if masked)."""
    x: torch.Tensor
    experts: torch.Tensor
    send_counts: torch.Tensor
    inv: torch.Tensor
    rows: int


class EmulatedEPExchangeBackend:
    """EPMoEBackend.__call__ (ep.py:210-249) end to end for `world` ranks on one
    GPU, each rank with its own weight slice: every rank routes its own tokens
    (source segment r of the batch), builds its send buffer (``send``), the
    two all-to-alls are device copies between the ranks' buffers in rank
    order (what all_to_all_single with these split sizes delivers), each
    rank runs what it received (``receive``), and each sender combines the
    returned rows through its inverse order (ops.combine_rows).  Equal to
    HipMoEBackend bit for bit for any placement (ep.py:1-8)."""

    def __init__(self, layer: int, placement: Placement, world: int, w_in_full: torch.Tensor,
                 w_out_full: torch.Tensor, stats: "EPStats | None" = None, check: bool = True):
        self.layer, self.placement, self.world = layer, placement, world
        self.ranks = [HipEPShareBackend(layer, placement, r, w_in_full[ids], w_out_full[ids], stats=stats,
                                        check=check)
                      for r, ids in ((r, placement.experts_of_rank(r)[layer]) for r in range(world))]

    def __call__(self, x_flat, topk_idx, topk_gate, valid_mask=None, seg_tokens=None, rr=None):
        n = x_flat.shape[0]
        seg = [n * r // self.world for r in range(self.world + 1)] if seg_tokens is None else list(seg_tokens)
        sl = [slice(seg[r], seg[r + 1]) for r in range(self.world)]
        vm = [None if valid_mask is None else valid_mask[s] for s in sl]
        sends = [be.send(x_flat[s], topk_idx[s], vm[r], None if rr is None else rr[r:r + 1])
                 for r, (be, s) in enumerate(zip(self.ranks, sl))]
        # counts exchange (ep.py:120-124): per sender, the row offsets of each destination
        off = [[0] + torch.cumsum(b.send_counts, 0).tolist() for b in sends]
        # all_to_all of rows and experts (ep.py:224-226), then the experts of each rank
        ys = []
        for q, be in enumerate(self.ranks):
            rx = torch.cat([b.x[off[r][q]:off[r][q + 1]] for r, b in enumerate(sends)])
            re = torch.cat([b.experts[off[r][q]:off[r][q + 1]] for r, b in enumerate(sends)])
            ys.append(be.receive(rx, re))
        # the reverse all_to_all (ep.py:233) and each sender's combine (ep.py:237-242)
        recv_off = [[0] + torch.cumsum(torch.tensor([off[r][q + 1] - off[r][q] for r in range(self.world)]),
                                       0).tolist() for q in range(self.world)]
        outs = []
        for r, b in enumerate(sends):
            back = torch.cat([ys[q][recv_off[q][r]:recv_off[q][r + 1]] for q in range(self.world)])
            if back.shape[0] == 0:
                back = torch.zeros(1, x_flat.shape[1], dtype=ys[0].dtype, device=x_flat.device)
            outs.append(ops.combine_rows(back, topk_gate[sl[r]], b.inv, vm[r]))
        return torch.cat(outs)


class EmulatedEPMoEBackend:
    """EPMoEBackend's output (ep.py:210-249) for a `world`-rank placement,
    computed on one GPU: each rank's share runs with that rank's own weight
    slice (owned experts + replicas, sorted global ids -- weights.py:54-58),
    every share writes the common (token, slot) buffer, then one combine in
    canonical slot order.  Equal to HipMoEBackend bit for bit for any
    placement, which is the reference's placement-invariance property
    (ep.py:1-8).  With ``stores`` (one ExpertStore per rank, holding that
    rank's experts of the placement) the ranks read their weights from the
    stores' slots instead of slices of the full weights."""

    def __init__(self, layer: int, placement: Placement, world: int, w_in_full: torch.Tensor | None = None,
                 w_out_full: torch.Tensor | None = None, check: bool = True, stores=None):
        self.layer, self.placement, self.world = layer, placement, world
        if stores is not None:
            # each rank reads its experts from its own ExpertStore's slots
            self.ranks = [HipEPShareBackend(layer, placement, r, check=check, store=stores[r])
                          for r in range(world)]
            return
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
