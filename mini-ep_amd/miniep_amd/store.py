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
(``mep_copy_experts``, one launch per layer), from the checkpoint's tensors
(device memory: with 288 GB of HBM a rank can keep the whole expert
checkpoint, 2.3 GB for GraniteMoE in bf16, next to its slots).  With
``capacity`` >= the number of experts and every expert loaded, a
re-placement copies nothing at all.
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
        self.w_in = [torch.empty(capacity, 2 * inter, hidden, dtype=dtype, device=self.device)
                     for _ in range(num_layers)]
        self.w_out = [torch.empty(capacity, hidden, inter, dtype=dtype, device=self.device)
                      for _ in range(num_layers)]
        self.slot_of: list[dict[int, int]] = [{} for _ in range(num_layers)]
        self.local_experts: list[list[int]] = [[] for _ in range(num_layers)]
        self.w_slot: list[torch.Tensor] = [torch.zeros(0, dtype=torch.int32, device=self.device)
                                           for _ in range(num_layers)]
        self.copied_total = 0

    def assign(self, layer: int, experts, src_in: torch.Tensor, src_out: torch.Tensor) -> int:
        """Make `experts` (global ids) the resident set of `layer`: experts
        that stay keep their slots, experts that leave free theirs, and
        arriving experts are copied from the checkpoint tensors
        ``src_in`` (E, 2I, H) / ``src_out`` (E, H, I) into free slots.
        Returns the number of experts copied."""
        want = sorted(set(int(e) for e in experts))
        if len(want) > self.capacity:
            raise ValueError(f"layer {layer}: {len(want)} resident experts exceed {self.capacity} slots")
        if want and (want[0] < 0 or want[-1] >= src_in.shape[0]):
            raise ValueError(f"layer {layer}: expert id outside the checkpoint's {src_in.shape[0]} experts")
        old, wanted = self.slot_of[layer], set(want)
        keep = {e: s for e, s in old.items() if e in wanted}
        free = sorted(set(range(self.capacity)) - set(keep.values()))
        arriving = [e for e in want if e not in keep]
        slots = free[:len(arriving)]
        ops.copy_experts(src_in.to(self.dtype).contiguous(), src_out.to(self.dtype).contiguous(), arriving,
                         self.w_in[layer], self.w_out[layer], slots)
        keep.update(zip(arriving, slots))
        self.slot_of[layer] = keep
        self.local_experts[layer] = want
        self.w_slot[layer] = torch.tensor([keep[e] for e in want], dtype=torch.int32, device=self.device)
        self.copied_total += len(arriving)
        return len(arriving)

    def layer_weights(self, layer: int):
        """(w_in slots, w_out slots, w_slot (n_local,) int32) of `layer`."""
        return self.w_in[layer], self.w_out[layer], self.w_slot[layer]


def apply_placement(backends, store: ExpertStore, placement: Placement, rank: int, checkpoint) -> dict:
    """Swap `placement` in live for this rank (server.py:51-62): every layer's
    resident experts become the placement's experts of `rank`, copying only
    the arriving ones from ``checkpoint`` (a callable layer -> (w_in (E, 2I, H),
    w_out (E, H, I)) device tensors); every backend then reads its layer's
    slots.  Returns {"copied": experts copied, "seconds": wall time including
    the device work}."""
    t0 = time.perf_counter()
    mine = placement.experts_of_rank(rank)
    copied = 0
    for layer in range(store.num_layers):
        src_in, src_out = checkpoint(layer)
        copied += store.assign(layer, mine[layer], src_in, src_out)
    for be in backends:
        be.use_store(placement, store)
    torch.cuda.synchronize(store.device)
    return {"copied": copied, "seconds": time.perf_counter() - t0}
