"""Dispatch parity on the GPU (mep_dispatch) vs the oracle: bit-exact.

Covers world-1 (LocalMoEBackend) grouping, the replica round-robin of every
layer of the reference's balanced plan, one rank's share with several source
segments, valid masks, empty inputs, error reporting and run-to-run identity.
"""
import json

import numpy as np
import pytest
import torch

from helpers import banner, to_np
from miniep_amd import Placement, _lib, ops, workloads
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _routing(n, k, E, seed, zipf=False):
    g = torch.Generator().manual_seed(seed)
    if zipf:
        w = torch.arange(1, E + 1, dtype=torch.float64) ** -1.2
        lg = torch.log(w)[torch.randperm(E, generator=g)] - torch.log(-torch.log(torch.rand(n, E, generator=g, dtype=torch.float64)))
    else:
        lg = torch.rand(n, E, generator=g)
    return lg.topk(k, dim=-1).indices


def _world1(E):
    return (torch.zeros(E, 1, dtype=torch.int32, device=DEV), torch.ones(E, dtype=torch.int32, device=DEV),
            torch.arange(E, dtype=torch.int32, device=DEV))


def _check(d, ref, n, k, n_local):
    M = int(ref["offsets"][-1])
    assert to_np(d.counts).tolist() == ref["counts"].tolist()
    assert to_np(d.offsets).tolist() == ref["offsets"].tolist()
    assert to_np(d.perm)[:M].tolist() == ref["perm"].tolist()
    assert to_np(d.row_of_entry)[: n * k].tolist() == ref["row_of_entry"].tolist()


@pytest.mark.parametrize("n,k,E,masked,zipf", [(3000, 8, 32, True, False), (16384, 8, 32, False, True),
                                               (1, 8, 32, False, False), (999, 3, 7, True, False),
                                               (5000, 1, 256, False, False), (2048, 32, 64, True, True),
                                               (70000, 8, 32, True, True)])   # > 512 blocks: scanned histograms
def test_world1_grouping(n, k, E, masked, zipf):
    banner(f"dispatch world1 n={n} k={k} E={E}")
    topk = _routing(n, k, E, n + k, zipf)
    valid = (torch.rand(n, generator=torch.Generator().manual_seed(1)) < 0.8) if masked else None
    table, n_rep, g2l = _world1(E)
    rc = torch.zeros(E, dtype=torch.long, device=DEV)
    d = ops.dispatch(topk.to(DEV), None if valid is None else valid.to(DEV), E, table, n_rep, False, None,
                     0, g2l, E, route_counts=rc, want_dest=True)
    ref = O.dispatch(topk.numpy(), None if valid is None else valid.numpy(), E, np.zeros((E, 1), np.int64),
                     np.ones(E, np.int64), np.zeros((1, E), np.int64), [0, n], 0, np.arange(E))
    _check(d, ref, n, k, E)
    assert to_np(d.dest)[: n * k].tolist() == ref["dest"].tolist()
    assert to_np(rc).tolist() == ref["route_counts"].tolist()
    # run-to-run identity (no atomics decide positions)
    d2 = ops.dispatch(topk.to(DEV), None if valid is None else valid.to(DEV), E, table, n_rep, False, None,
                      0, g2l, E)
    M = int(ref["offsets"][-1])          # perm rows past M are not defined
    assert torch.equal(d.perm[:M], d2.perm[:M]) and torch.equal(d.row_of_entry, d2.row_of_entry)


def test_dest_ranks_every_plan_layer(golden_dir):
    """Placement.dest_ranks (ep.py:76-96) on all 24 layers of the reference plan,
    three forwards per layer without reset (counters carry over), then reset."""
    banner("dest_ranks plan layers")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    rng = np.random.default_rng(0)
    for layer in range(24):
        t_ref, n_ref = O.build_table(p.owners[layer])
        rr = np.zeros(32, np.int64)
        for step in range(3):
            ids = rng.integers(0, 32, int(rng.integers(1, 3000)))
            got = p.dest_ranks(layer, torch.from_numpy(ids))
            ref, rr = O.dest_ranks(t_ref, n_ref, rr, ids)
            assert to_np(got).tolist() == ref.tolist(), (layer, step)
            assert to_np(p.rr(layer)[0]).tolist() == rr.tolist()
    p.reset_rr()
    assert int(p._rr.abs().sum()) == 0


@pytest.mark.parametrize("sources,n", [(1, 8192), (4, 8192), (4, 40000)])
def test_rank_share_plan_layer2(golden_dir, sources, n):
    """One rank's share under the reference's balanced plan, layer 2 (8 owned +
    2 replicas per rank), n Zipf(1.1)-routed tokens from `sources` senders
    (n = 40000: 625 blocks, above the threshold for the scanned histograms)."""
    banner(f"rank share layer2 sources={sources} n={n}")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    L = workloads.make_layer(n, seed=3, zipf_s=1.1)
    topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices
    k, E = 8, 32
    seg = [n * s // sources for s in range(sources + 1)]
    table, n_rep = p.tables(2)
    t_ref, n_ref = O.build_table(p.owners[2])
    rr0 = np.random.default_rng(1).integers(0, 6, (sources, E))
    seen = np.zeros(n * k, np.int64)
    for r in range(4):
        local = p.experts_of_rank(r)[2]
        g2l = np.full(E, -1)
        g2l[local] = np.arange(len(local))
        rr = torch.from_numpy(rr0.copy()).to(DEV)
        rc = torch.zeros(E, dtype=torch.long, device=DEV)
        d = ops.dispatch(topk.to(DEV), None, E, table, n_rep, True, rr, r,
                         torch.from_numpy(g2l).int().to(DEV), len(local), seg_tokens=seg,
                         route_counts=rc, want_dest=True)
        ref = O.dispatch(topk.numpy(), None, E, t_ref, n_ref, rr0, seg, r, g2l)
        _check(d, ref, n, k, len(local))
        assert to_np(d.dest).tolist() == ref["dest"].tolist()
        assert to_np(rr).tolist() == ref["rr_after"].tolist()
        assert to_np(rc).tolist() == ref["route_counts"].tolist()
        seen[ref["perm"]] += 1
    assert (seen == 1).all()          # the 4 shares partition the entries


def test_random_placements_every_rank():
    """Seeded random cases: experts with 1-3 owner ranks out of 4 (random
    replica sets), 1-5 source segments of random sizes (empty ones included),
    random masks and round-robin counters, every rank's share bit-exact against
    the oracle, and the 4 shares partition the kept entries."""
    rng = np.random.default_rng(11)
    for case in range(12):
        E = int(rng.choice([8, 16, 32, 64]))
        k = int(rng.integers(1, min(E, 8) + 1))
        n = int(rng.choice([1, 37, 513, 4000, 70000 if case == 11 else 9000]))
        sources = int(rng.integers(1, 6))
        banner(f"random placement case {case}: n={n} k={k} E={E} sources={sources}")
        owners = [sorted(rng.choice(4, int(rng.integers(1, 4)), replace=False).tolist()) for _ in range(E)]
        for r in range(4):                      # every rank owns at least one expert
            if not any(r in o for o in owners):
                e = int(rng.integers(E))
                owners[e] = sorted(set(owners[e]) | {r})
        p = Placement([owners], device=DEV)
        table, n_rep = p.tables(0)
        t_ref, n_ref = O.build_table(owners)
        cuts = np.sort(rng.integers(0, n + 1, sources - 1))
        seg = [0, *cuts.tolist(), n]
        topk = torch.from_numpy(np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int64))
        valid = torch.from_numpy(rng.random(n) < 0.85)
        rr0 = rng.integers(0, 5, (sources, E))
        seen = np.zeros(n * k, np.int64)
        for r in range(4):
            local = p.experts_of_rank(r)[0]
            g2l = np.full(E, -1)
            g2l[local] = np.arange(len(local))
            rr = torch.from_numpy(rr0.copy()).to(DEV)
            d = ops.dispatch(topk.to(DEV), valid.to(DEV), E, table, n_rep, True, rr, r,
                             torch.from_numpy(g2l).int().to(DEV), len(local), seg_tokens=seg, want_dest=True)
            ref = O.dispatch(topk.numpy(), valid.numpy(), E, t_ref, n_ref, rr0, seg, r, g2l)
            _check(d, ref, n, k, len(local))
            assert to_np(d.dest).tolist() == ref["dest"].tolist()
            assert to_np(rr).tolist() == ref["rr_after"].tolist()
            seen[ref["perm"]] += 1
        kept = np.repeat(valid.numpy(), k)
        assert (seen[kept] == 1).all() and (seen[~kept] == 0).all()


def test_empty_and_all_masked():
    banner("dispatch empty")
    E = 32
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(torch.zeros(0, 8, dtype=torch.long, device=DEV), None, E, table, n_rep, False, None,
                     0, g2l, E)
    assert to_np(d.offsets).tolist() == [0] * (E + 1)
    topk = _routing(100, 8, E, 3)
    d = ops.dispatch(topk.to(DEV), torch.zeros(100, dtype=torch.bool, device=DEV), E, table, n_rep, False,
                     None, 0, g2l, E)
    assert to_np(d.offsets).tolist() == [0] * (E + 1)
    assert (to_np(d.row_of_entry)[:800] == -1).all()


def test_errors_are_reported():
    banner("dispatch errors")
    E = 32
    table, n_rep, g2l = _world1(E)
    bad = _routing(64, 8, E, 4)
    bad[5, 3] = 40
    with pytest.raises(_lib.ExpertRangeError):
        ops.dispatch(bad.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E)
    # rank 0 holds experts 0..15 only, naive world-2 placement
    tab2 = (torch.arange(E, dtype=torch.int32) // 16).reshape(E, 1).to(DEV)
    g2l_missing = torch.full((E,), -1, dtype=torch.int32)
    g2l_missing[:8] = torch.arange(8, dtype=torch.int32)
    with pytest.raises(_lib.NotResidentError):
        ops.dispatch(_routing(64, 8, E, 5).to(DEV), None, E, tab2, n_rep, False, None, 0,
                     g2l_missing.to(DEV), 8)
    with pytest.raises(_lib.MepError, match="segments"):
        ops.dispatch(_routing(64, 8, E, 6).to(DEV), None, E, table, n_rep, False, None, 0, g2l, E,
                     seg_tokens=list(range(0, 64, 3)) + [64])
    with pytest.raises(_lib.MepError, match="rr is required"):
        ops.dispatch(_routing(64, 8, E, 6).to(DEV), None, E, table, n_rep, True, None, 0, g2l, E)


def test_zero_replica_count_is_reported():
    """n_rep[e] = 0 (an expert without an owner, which Placement forbids,
    ep.py:21) is reported by mep_dispatch_check instead of being clamped
    silently; the launch itself stays in bounds."""
    banner("dispatch n_rep = 0")
    E, n, k = 32, 512, 8
    topk = _routing(n, k, E, 3)
    table, n_rep, g2l = _world1(E)
    n_rep[5] = 0
    with pytest.raises(_lib.MepError, match="n_rep"):
        ops.dispatch(topk.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E, check=True)
    n_rep[5] = 2                                          # more replicas than the table has columns
    with pytest.raises(_lib.MepError, match="n_rep"):
        ops.dispatch(topk.to(DEV), None, E, table, n_rep, True,
                     torch.zeros(1, E, dtype=torch.long, device=DEV), 0, g2l, E, check=True)
    n_rep[5] = 1
    ops.dispatch(topk.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E, check=True)
