"""Device-resident expert weights in slots, and the live re-placement of
server.py:51-62 on top of them.

The reference swaps a new placement in by reloading, for every layer, the
rank's owned + replica experts from the checkpoint in sorted id order
(``load_weights(experts_per_layer=my, only_experts=True)``, weights.py:37-61)
and handing the new slices to each backend (server.py:51-62).  Here each rank
keeps, per layer, ``capacity`` expert slots in HBM:

    w_in[l]  (capacity, 2I, H)     w_out[l]  (capacity, H, I)
    slot_of[l]: global expert -> slot        w_slot[l] (n_local,) int32 device

The local experts stay in sorted global-id order (the row grouping of the
dispatch, ep.py:69 / weights.py:54-58); local expert j reads its weights
from slot ``w_slot[l][j]`` (``mep_grouped_swiglu_slots``).  A new placement
keeps every expert that stays resident where it is, frees the slots of the
experts that leave, and copies only the experts that arrive into free slots
(``mep_copy_experts``), from the checkpoint's tensors (device memory: with
288 GB of HBM a rank can keep the whole expert checkpoint, 2.3 GB for
GraniteMoE in bf16, next to its slots).  All layers' slots live in one
tensor per weight, so a re-placement from a checkpoint held as (layers,
experts, ...) tensors is ONE copy launch for every layer, and the slot tables
of all layers one host-to-device copy.  With ``capacity`` >= the number of
experts and every expert loaded, a re-placement copies nothing at all.
"""
from __future__ import annotations

import time

import torch

from . import ops
from .placement import Placement


class ExpertStore:
    """One rank's expert weights in per-layer slots on one device."""

    def __init__(self, num_layers: int, capacity: int, hidden: int, inter: int,
                 dtype=torch.bfloat16, device="cuda"):
        if capacity < 1:
            raise ValueError("capacity must be at least 1")
        self.num_layers, self.capacity = num_layers, capacity
        self.hidden, self.inter, self.dtype = hidden, inter, dtype
        self.device = torch.device(device)
        # every layer's slots in one tensor: layer l's are rows [l * capacity, (l + 1) * capacity)
        self.w_in_all = torch.empty(num_layers * capacity, 2 * inter, hidden, dtype=dtype, device=self.device)
        self.w_out_all = torch.empty(num_layers * capacity, hidden, inter, dtype=dtype, device=self.device)
        self.w_in = [self.w_in_all[l * capacity:(l + 1) * capacity] for l in range(num_layers)]
        self.w_out = [self.w_out_all[l * capacity:(l + 1) * capacity] for l in range(num_layers)]
        self.slot_of: list[dict[int, int]] = [{} for _ in range(num_layers)]
        self.local_experts: list[list[int]] = [[] for _ in range(num_layers)]
        self.w_slot: list[torch.Tensor] = [torch.zeros(0, dtype=torch.int32, device=self.device)
                                           for _ in range(num_layers)]
        self.copied_total = 0
        self.last_pairs: tuple[list[int], list[int]] = ([], [])

    def _plan(self, layer: int, experts, n_experts: int):
        """Bookkeeping of a new resident set for `layer`: (arriving experts,
        their free slots, the slot of every resident expert in id order)."""
        want = sorted(set(int(e) for e in experts))
        if len(want) > self.capacity:
            raise ValueError(f"layer {layer}: {len(want)} resident experts exceed {self.capacity} slots")
        if want and (want[0] < 0 or want[-1] >= n_experts):
            raise ValueError(f"layer {layer}: expert id outside the checkpoint's {n_experts} experts")
        old, wanted = self.slot_of[layer], set(want)
        keep = {e: s for e, s in old.items() if e in wanted}
        free = sorted(set(range(self.capacity)) - set(keep.values()))
        arriving = [e for e in want if e not in keep]
        slots = free[:len(arriving)]
        keep.update(zip(arriving, slots))
        return want, arriving, slots, keep

    def assign(self, layer: int, experts, src_in: torch.Tensor, src_out: torch.Tensor) -> int:
        """Make `experts` (global ids) the resident set of `layer`: experts
        that stay keep their slots, experts that leave free theirs, and
        arriving experts are copied from the checkpoint tensors
        ``src_in`` (E, 2I, H) / ``src_out`` (E, H, I) into free slots.
        Returns the number of experts copied."""
        want, arriving, slots, keep = self._plan(layer, experts, src_in.shape[0])
        ops.copy_experts(src_in.to(self.dtype).contiguous(), src_out.to(self.dtype).contiguous(), arriving,
                         self.w_in[layer], self.w_out[layer], slots)
        self.slot_of[layer] = keep
        self.local_experts[layer] = want
        self.w_slot[layer] = torch.tensor([keep[e] for e in want], dtype=torch.int32, device=self.device)
        self.copied_total += len(arriving)
        return len(arriving)

    def assign_all(self, experts_per_layer, ck_in: torch.Tensor, ck_out: torch.Tensor) -> int:
        """``assign`` for every layer at once from a checkpoint held as
        ``ck_in`` (L, E, 2I, H) / ``ck_out`` (L, E, H, I): one copy launch
        moves every arriving expert of every layer, and the slot tables of
        all layers arrive in one host-to-device copy.  Returns the number of
        experts copied."""
        n_layers, n_experts = ck_in.shape[0], ck_in.shape[1]
        if n_layers != self.num_layers or len(experts_per_layer) != n_layers:
            raise ValueError(f"{n_layers} checkpoint layers for a store of {self.num_layers}")
        plans = [self._plan(l, experts_per_layer[l], n_experts) for l in range(n_layers)]
        src = [l * n_experts + e for l, (_, arriving, _, _) in enumerate(plans) for e in arriving]
        dst = [l * self.capacity + s for l, (_, _, slots, _) in enumerate(plans) for s in slots]
        self.last_pairs = (src, dst)                  # (checkpoint row, slot row) of each copied expert
        ops.copy_experts(ck_in.to(self.dtype).reshape(n_layers * n_experts, *ck_in.shape[2:]),
                         ck_out.to(self.dtype).reshape(n_layers * n_experts, *ck_out.shape[2:]), src,
                         self.w_in_all, self.w_out_all, dst)
        width = max(1, max(len(want) for want, _, _, _ in plans))
        table = torch.zeros(n_layers, width, dtype=torch.int32)
        for l, (want, _, _, keep) in enumerate(plans):
            table[l, :len(want)] = torch.tensor([keep[e] for e in want], dtype=torch.int32)
        table = table.to(self.device)
        for l, (want, _, _, keep) in enumerate(plans):
            self.slot_of[l] = keep
            self.local_experts[l] = want
            self.w_slot[l] = table[l, :len(want)]
        self.copied_total += len(src)
        return len(src)

    def layer_weights(self, layer: int):
        """(w_in slots, w_out slots, w_slot (n_local,) int32) of `layer`."""
        return self.w_in[layer], self.w_out[layer], self.w_slot[layer]


def apply_placement(backends, store: ExpertStore, placement: Placement, rank: int, checkpoint) -> dict:
    """Swap `placement` in live for this rank (server.py:51-62): every layer's
    resident experts become the placement's experts of `rank`, copying only
    the arriving ones from ``checkpoint``: a pair of device tensors (w_in (L,
    E, 2I, H), w_out (L, E, H, I)), which makes the whole swap one copy
    launch, or a callable layer -> (w_in (E, 2I, H), w_out (E, H, I)), one
    launch per layer; every backend then reads its layer's slots.  Returns
    {"copied": experts copied, "seconds": wall time including the device
    work}."""
    t0 = time.perf_counter()
    mine = placement.experts_of_rank(rank)
    if isinstance(checkpoint, tuple):
        copied = store.assign_all(mine, checkpoint[0], checkpoint[1])
    else:
        copied = 0
        for layer in range(store.num_layers):
            src_in, src_out = checkpoint(layer)
            copied += store.assign(layer, mine[layer], src_in, src_out)
    for be in backends:
        be.use_store(placement, store)
    torch.cuda.synchronize(store.device)
    return {"copied": copied, "seconds": time.perf_counter() - t0}
