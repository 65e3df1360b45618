"""The balancer loop on the GPU: statistics -> plan -> new placement -> hot swap.

Reference flow: each rank counts the experts of the entries it routes
(`route_counts`, ep.py:164-183, 216-217), the server sums them over ranks
and re-plans with the balancer (server.py:166-183, balancer.py:63-89), then
every rank swaps in its re-sliced expert weights (server.py:51-62).

Here: four Zipf(1.1)-skewed layers, world 4, naive placement; each emulated
rank dispatches its own quarter of the tokens with the dispatch kernel, which
accumulates `route_counts` on the device; `plan_balanced` re-plans from those
counts; then
  * the GPU counts equal the oracle's bincount, so the plan is the oracle's plan;
  * the rows each rank receives under the new plan (the round-robin of the
    dispatch kernel, all four senders) are balanced to the planner's target;
  * every rank's share under the new plan is bit-exact against the oracle;
  * after `apply_placement` with re-sliced weights, the world-4 output is
    bitwise the all-local output (placement invariance, ep.py:1-8).
"""
import numpy as np
import pytest
import torch

from helpers import banner, to_np
from miniep_amd import (EmulatedEPMoEBackend, EPStats, HipEPShareBackend, HipMoEBackend, Placement,
                        plan_balanced, route, workloads)
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
WORLD, LAYERS, T, E, K = 4, 4, 8192, 32, 8


def _rows_per_rank(p: Placement, layer: int, idx: torch.Tensor, w_in, w_out) -> list[int]:
    """Rows each rank receives from all WORLD senders (one token quarter each)."""
    seg = [T * s // WORLD for s in range(WORLD + 1)]
    rows = []
    for r in range(WORLD):
        ids = p.experts_of_rank(r)[layer]
        be = HipEPShareBackend(layer, p, r, w_in[ids], w_out[ids])
        rows.append(int(be.dispatch(idx, seg_tokens=seg).offsets[-1]))
    return rows


def test_route_counts_plan_and_hot_swap():
    banner("balancer loop: GPU route_counts -> plan_balanced -> new placement")
    layers = [workloads.make_layer(T, seed=20 + l, zipf_s=1.1) for l in range(LAYERS)]
    bf = torch.bfloat16
    xs = [L.x.to(bf).to(DEV) for L in layers]
    w_in = [L.w_in.to(bf).to(DEV) for L in layers]
    w_out = [L.w_out.to(bf).to(DEV) for L in layers]
    idxs, gates = zip(*[route(xs[l], layers[l].w_router.to(bf).to(DEV), K) for l in range(LAYERS)])

    # statistics: every rank routes its own quarter of the tokens on the naive placement
    naive = Placement.naive(LAYERS, E, WORLD, device=DEV)
    stats = EPStats(LAYERS, E, device=DEV)
    quarter = T // WORLD
    for l in range(LAYERS):
        for r in range(WORLD):
            ids = naive.experts_of_rank(r)[l]
            be = HipEPShareBackend(l, naive, r, w_in[l][ids], w_out[l][ids], stats=stats)
            be.dispatch(idxs[l][r * quarter:(r + 1) * quarter])
    counts = stats.route_counts.cpu()
    oracle_counts = np.stack([np.bincount(to_np(i).reshape(-1), minlength=E) for i in idxs])
    assert counts.numpy().tolist() == oracle_counts.tolist()

    p_new, report = plan_balanced(counts, WORLD, slots_per_rank=2, target_ratio=1.05, device=DEV)
    p_ref, _ = plan_balanced(torch.from_numpy(oracle_counts), WORLD, slots_per_rank=2, target_ratio=1.05)
    assert p_new.owners == p_ref.owners
    assert report["replicas_total"] > 0

    for l in range(LAYERS):
        before = _rows_per_rank(naive, l, idxs[l], w_in[l], w_out[l])
        after = _rows_per_rank(p_new, l, idxs[l], w_in[l], w_out[l])
        assert sum(before) == sum(after) == T * K
        imb_b, imb_a = max(before) / (T * K / WORLD), max(after) / (T * K / WORLD)
        print(f"layer {l}: rows per rank naive {before} ({imb_b:.3f}) -> planned {after} ({imb_a:.3f}); "
              f"planner {report['layers'][l]['imbalance_before']:.3f} -> {report['layers'][l]['imbalance_after']:.3f}",
              flush=True)
        assert imb_a < imb_b
        assert imb_a <= report["layers"][l]["imbalance_after"] + 0.02

    # every rank's share under the new plan, bit-exact (layer 0, four senders with their own rr)
    l = 0
    table, n_rep = p_new.tables(l)
    t_ref, n_ref = O.build_table(p_new.owners[l])
    seg = [T * s // WORLD for s in range(WORLD + 1)]
    rr0 = np.zeros((WORLD, E), np.int64)
    seen = np.zeros(T * K, np.int64)
    for r in range(WORLD):
        ids = p_new.experts_of_rank(r)[l]
        g2l = np.full(E, -1)
        g2l[ids] = np.arange(len(ids))
        be = HipEPShareBackend(l, p_new, r, w_in[l][ids], w_out[l][ids])
        rr = torch.zeros(WORLD, E, dtype=torch.long, device=DEV)
        d = be.dispatch(idxs[l], seg_tokens=seg, rr=rr, want_dest=True)
        ref = O.dispatch(to_np(idxs[l]), None, E, t_ref, n_ref, rr0, seg, r, g2l)
        M = int(ref["offsets"][-1])
        assert to_np(d.counts).tolist() == ref["counts"].tolist()
        assert to_np(d.perm)[:M].tolist() == ref["perm"].tolist()
        assert to_np(d.dest).tolist() == ref["dest"].tolist()
        assert to_np(rr).tolist() == ref["rr_after"].tolist()
        seen[ref["perm"]] += 1
    assert (seen == 1).all()

    # hot swap: ranks start on the naive slices, swap in the planned ones
    ep = EmulatedEPMoEBackend(l, naive, WORLD, w_in[l], w_out[l])
    ep.placement = p_new
    for r, be in enumerate(ep.ranks):
        ids = p_new.experts_of_rank(r)[l]
        be.apply_placement(p_new, w_in[l][ids], w_out[l][ids])
    local = HipMoEBackend(w_in[l], w_out[l])(xs[l], idxs[l], gates[l])
    got = ep(xs[l], idxs[l], gates[l], seg_tokens=seg)
    assert torch.equal(local, got)
