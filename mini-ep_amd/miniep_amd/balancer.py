"""Greedy hot-expert replication planner: the interface of miniep/balancer.py.

Input: global per-(layer, expert) routing counts from a profiling window
(e.g. the dispatch kernel's ``route_counts``).  Output: a Placement that starts
from the naive contiguous placement and adds replicas of hot experts on
under-loaded ranks, one at a time, each time taking the (expert, rank) that
lowers the layer's busiest rank the most, within a per-rank slot budget
(balancer.py:47-60), until max/mean load is within ``target_ratio``.

A replicated expert's load is split evenly over its replicas, which is what
the round-robin dispatch does (ep.py:76-96).  This is host-side planning, run
once per rebalance; the per-token work it steers runs in the HIP dispatch
kernel.
"""
from __future__ import annotations

import torch

from .placement import Placement


def rank_loads(loads: list[float], owners: list[list[int]], world: int) -> list[float]:
    """Expected load per rank when each expert's load is split evenly over its
    owners (balancer.py:17-23)."""
    out = [0.0] * world
    for e, own in enumerate(owners):
        share = loads[e] / len(own)
        for r in own:
            out[r] += share
    return out


def best_replica_addition(loads, owners, world, slots):
    """(new_max, expert, rank) of the in-budget replica that lowers the busiest
    rank the most, or None (balancer.py:26-44).  Candidates are scanned expert
    by expert, rank by rank; a later candidate wins only if strictly better."""
    cur_max = max(rank_loads(loads, owners, world))
    best = None
    for e, own in enumerate(owners):
        if loads[e] / len(own) == 0:
            continue
        for r in range(world):
            if r in own or slots[r] <= 0:
                continue
            trial = list(owners)
            trial[e] = sorted(own + [r])
            new_max = max(rank_loads(loads, trial, world))
            if new_max < cur_max and (best is None or new_max < best[0]):
                best = (new_max, e, r)
    return best


def plan_layer(loads, world, per, slots_per_rank, target_ratio):
    """Greedy replication for one layer -> (owners, loads_before, loads_after)
    (balancer.py:47-60)."""
    owners = [[e // per] for e in range(len(loads))]
    slots = [slots_per_rank] * world
    before = rank_loads(loads, owners, world)
    mean = sum(before) / world
    while mean and max(rank_loads(loads, owners, world)) / mean > target_ratio:
        best = best_replica_addition(loads, owners, world, slots)
        if best is None:
            break
        _, e, r = best
        owners[e] = sorted(owners[e] + [r])
        slots[r] -= 1
    return owners, before, rank_loads(loads, owners, world)


def plan_balanced(counts, world: int, slots_per_rank: int = 2, target_ratio: float = 1.05,
                  device=None) -> tuple[Placement, dict]:
    """counts: (num_layers, num_experts) global routing counts -> (Placement,
    report) with per-layer imbalance before/after and the replica total
    (balancer.py:63-89)."""
    counts = torch.as_tensor(counts).to("cpu")
    num_layers, num_experts = counts.shape
    per = num_experts // world
    all_owners = []
    report = {"layers": [], "replicas_total": 0}
    for l in range(num_layers):
        loads = counts[l].double().tolist()
        owners, before, after = plan_layer(loads, world, per, slots_per_rank, target_ratio)
        mean = sum(before) / world
        replicas = sum(len(o) for o in owners) - num_experts
        report["replicas_total"] += replicas
        report["layers"].append({
            "layer": l,
            "imbalance_before": max(before) / mean if mean else 1.0,
            "imbalance_after": max(after) / mean if mean else 1.0,
            "replicas": replicas,
        })
        all_owners.append(owners)
    return Placement(all_owners, device=device), report
