"""Greedy hot-expert replication planner with the interface of miniep/balancer.py.

Input: global per-(layer, expert) routing counts from a profiling window (for
example the dispatch kernel's ``route_counts``).  Output: a Placement that
starts from the naive contiguous placement and adds replicas of hot experts on
under-loaded ranks, one at a time, within a per-rank slot budget, until the
layer's max/mean rank load is within ``target_ratio`` (behaviour of
balancer.py:47-89).

Each step takes the (expert, rank) replica that lowers the busiest rank the
most: candidates are ranked expert by expert, then rank by rank, and a later
candidate wins only with a strictly lower maximum (behaviour of
balancer.py:26-44).  A replicated expert's load is split evenly over its
copies, which is what the round-robin dispatch does (ep.py:76-96).

How the search is organised here: the planner keeps, per rank, the sorted
list of experts it holds and that rank's load.  A candidate replica changes
the loads of the expert's current holders and of the new rank only, so only
those ranks are re-summed; the other ranks' maximum comes from a rank order
sorted once per step.  A rank's load is always summed over its experts in
ascending id order, starting from 0.0, with each term ``count / copies``:
those are the float operations of the reference's per-trial re-summation, so
every comparison -- and therefore the plan -- is the same
(tests/test_host.py checks the plan of results/plan_balanced.json).

This is host-side planning, run once per rebalance; the per-token work it
steers runs in the HIP dispatch kernel.
"""
from __future__ import annotations

import bisect

import torch

from .placement import Placement


class _LayerPlan:
    """Replica state of one layer: holders of each expert, experts of each
    rank, remaining slots per rank, and every rank's load."""

    def __init__(self, counts: list[float], world: int, per_rank: int, slots_per_rank: int):
        self.counts = counts
        self.world = world
        self.holders = [[e // per_rank] for e in range(len(counts))]
        self.members = [[] for _ in range(world)]
        for e, (r,) in enumerate(self.holders):
            self.members[r].append(e)
        self.free = [slots_per_rank] * world
        self.load = [self._sum(r) for r in range(world)]

    def _sum(self, rank: int, extra: int = -1) -> float:
        """Load of `rank`, optionally with one more copy of expert `extra`
        (on this rank if it is not already here): the experts' shares added
        in ascending id order."""
        mine = self.members[rank]
        if extra >= 0 and extra not in mine:
            mine = mine[:]
            bisect.insort(mine, extra)
        total = 0.0
        for e in mine:
            copies = len(self.holders[e]) + (1 if e == extra else 0)
            total += self.counts[e] / copies
        return total

    def peak(self) -> float:
        return max(self.load)

    def trial_peak(self, expert: int, rank: int, by_load: list[int]) -> float:
        """Busiest rank's load if `rank` took a copy of `expert`."""
        touched = self.holders[expert] + [rank]
        peak = max(self._sum(q, expert) for q in touched)
        for q in by_load:                          # busiest rank the trial leaves alone
            if q not in touched:
                return max(peak, self.load[q])
        return peak

    def best_addition(self):
        """(peak, expert, rank) of the in-budget replica that lowers the
        busiest rank the most, or None if none lowers it."""
        now = self.peak()
        by_load = sorted(range(self.world), key=lambda q: -self.load[q])
        best = None
        for e, held_by in enumerate(self.holders):
            if self.counts[e] / len(held_by) == 0:
                continue                           # an idle expert gains nothing from a copy
            for r in range(self.world):
                if self.free[r] <= 0 or r in held_by:
                    continue
                p = self.trial_peak(e, r, by_load)
                if p < now and (best is None or p < best[0]):
                    best = (p, e, r)
        return best

    def add(self, expert: int, rank: int) -> None:
        touched = self.holders[expert] + [rank]
        bisect.insort(self.holders[expert], rank)
        bisect.insort(self.members[rank], expert)
        self.free[rank] -= 1
        for q in touched:
            self.load[q] = self._sum(q)


def plan_layer(counts: list[float], world: int, per_rank: int, slots_per_rank: int,
               target_ratio: float) -> tuple[list[list[int]], list[float], list[float]]:
    """One layer -> (holders of each expert, rank loads before, rank loads after)."""
    st = _LayerPlan(counts, world, per_rank, slots_per_rank)
    before = list(st.load)
    mean = sum(before) / world
    while mean and st.peak() / mean > target_ratio:
        pick = st.best_addition()
        if pick is None:
            break
        st.add(pick[1], pick[2])
    return [list(h) for h in st.holders], before, list(st.load)


def plan_balanced(counts, world: int, slots_per_rank: int = 2, target_ratio: float = 1.05,
                  device=None) -> tuple[Placement, dict]:
    """counts (num_layers, num_experts) global routing counts -> (Placement,
    report): the report holds each layer's predicted max/mean load before and
    after and its replica count, and the replica total (balancer.py:63-89)."""
    counts = torch.as_tensor(counts).to("cpu")
    num_layers, num_experts = counts.shape
    per_rank = num_experts // world
    layers, summary = [], []
    for l in range(num_layers):
        holders, before, after = plan_layer(counts[l].double().tolist(), world, per_rank,
                                            slots_per_rank, target_ratio)
        mean = sum(before) / world
        extra = sum(len(h) for h in holders) - num_experts
        summary.append({
            "layer": l,
            "imbalance_before": max(before) / mean if mean else 1.0,
            "imbalance_after": max(after) / mean if mean else 1.0,
            "replicas": extra,
        })
        layers.append(holders)
    report = {"layers": summary, "replicas_total": sum(s["replicas"] for s in summary)}
    return Placement(layers, device=device), report
