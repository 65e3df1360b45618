"""Expert placement with replica round-robin: the interface of miniep/ep.py:20-96.

``owners[layer][expert]`` lists the ranks holding a copy of that expert.  The
host keeps the same plan I/O as the reference (``naive``, ``from_plan``,
``to_plan``, ``experts_of_rank``, ``reset_rr``); the dispatch arithmetic
(``dest_ranks``) runs in the HIP dispatch kernel on device-resident tables:

  table[l]   (E, Rmax) int32   rank of expert e's j-th replica (ep.py:35-45)
  n_rep[l]   (E,) int32        number of replicas
  rr         (L, E) int64      round-robin counters, zeroed by reset_rr()
                               before every forward (worker.py:100,115,127)
"""
from __future__ import annotations

import torch

from . import ops


class Placement:
    """owners[layer][expert] = list of ranks holding that expert (>= 1 each)."""

    def __init__(self, owners: list[list[list[int]]], device=None):
        if not owners or not owners[0]:
            raise ValueError("owners must list at least one layer and one expert")
        for l, layer in enumerate(owners):
            if len(layer) != len(owners[0]):
                raise ValueError(f"layer {l} has {len(layer)} experts, expected {len(owners[0])}")
            for e, o in enumerate(layer):
                if len(o) < 1:
                    raise ValueError(f"layer {l} expert {e} has no owner")
        self.owners = [[list(o) for o in layer] for layer in owners]
        self.num_layers = len(owners)
        self.num_experts = len(owners[0])
        if device is None:
            device = "cuda" if torch.cuda.is_available() else "cpu"
        self.device = torch.device(device)
        self._tables = [self._build_table(self.owners[l]) for l in range(self.num_layers)]
        self._dev_tables: dict = {}
        self._rr = torch.zeros(self.num_layers, self.num_experts, dtype=torch.long, device=self.device)

    @property
    def world(self) -> int:
        """Ranks the placement spans: 1 + the highest rank holding an expert."""
        return 1 + max(r for layer in self.owners for o in layer for r in o)

    @staticmethod
    def _build_table(owners_l):
        """table[e, j] = rank of e's j-th replica, unused cells 0 (ep.py:35-45)."""
        n_exp = len(owners_l)
        rmax = max(len(o) for o in owners_l)
        table = torch.zeros(n_exp, rmax, dtype=torch.int32)
        n_rep = torch.zeros(n_exp, dtype=torch.int32)
        for e, o in enumerate(owners_l):
            table[e, :len(o)] = torch.tensor(o, dtype=torch.int32)
            n_rep[e] = len(o)
        return table, n_rep

    # ---- plan I/O (ep.py:47-71) -----------------------------------------
    @staticmethod
    def naive(num_layers: int, num_experts: int, world: int, device=None) -> "Placement":
        """Contiguous blocks of num_experts/world experts per rank (ep.py:47-52)."""
        if num_experts % world != 0:
            raise ValueError(f"{num_experts} experts do not split over {world} ranks")
        per = num_experts // world
        return Placement([[[e // per] for e in range(num_experts)] for _ in range(num_layers)],
                         device=device)

    @staticmethod
    def from_plan(plan: dict, device=None) -> "Placement":
        """Plan JSON -> placement, owner lists sorted (ep.py:54-60)."""
        layers = plan["owners"]
        owners = [[sorted(int(r) for r in layers[str(l)][str(e)]) for e in range(len(layers[str(l)]))]
                  for l in range(len(layers))]
        return Placement(owners, device=device)

    def to_plan(self) -> dict:
        return {"owners": {str(l): {str(e): list(self.owners[l][e]) for e in range(self.num_experts)}
                           for l in range(self.num_layers)}}

    def experts_of_rank(self, rank: int) -> dict[int, list[int]]:
        """layer -> sorted global ids resident on `rank` (ep.py:67-71)."""
        return {l: sorted(e for e in range(self.num_experts) if rank in self.owners[l][e])
                for l in range(self.num_layers)}

    def reset_rr(self):
        self._rr.zero_()

    # ---- device tables ----------------------------------------------------
    def has_replicas(self, layer: int) -> bool:
        return bool((self._tables[layer][1] != 1).any())

    def tables(self, layer: int, device=None):
        """(table, n_rep) of `layer` as int32 tensors on `device` (cached)."""
        dev = self.device if device is None else torch.device(device)
        key = (layer, str(dev))
        if key not in self._dev_tables:
            t, n = self._tables[layer]
            self._dev_tables[key] = (t.to(dev), n.to(dev))
        return self._dev_tables[key]

    def rr(self, layer: int) -> torch.Tensor:
        """This layer's (1, E) round-robin counter row (a view, updated in place)."""
        return self._rr[layer:layer + 1]

    def dest_ranks(self, layer: int, expert_ids: torch.Tensor) -> torch.Tensor:
        """Destination rank of each entry (ep.py:76-96) computed by the dispatch
        kernel; advances this layer's counters exactly like the reference."""
        ids = expert_ids.reshape(-1, 1).to(device=self.device, dtype=torch.int64)
        table, n_rep = self.tables(layer)
        has_rep = self.has_replicas(layer)
        g2l = torch.full((self.num_experts,), -1, dtype=torch.int32, device=self.device)
        d = ops.dispatch(ids, None, self.num_experts, table, n_rep, has_rep,
                         self.rr(layer) if has_rep else None, -1, g2l, 0,
                         want_dest=True, check=True)
        return d.dest[: ids.shape[0]].to(torch.int64)
