"""Expert parallelism end to end on one GPU: EPMoEBackend.__call__
(ep.py:210-249) for a world of 4 ranks, every rank with its own weight slice.

Each rank routes its own tokens; the send side (destinations with the rank's
own round-robin counters, the destination-sorted order, send counts, inverse
order, the gathered send buffer) runs on the dispatch and gather kernels;
the two all-to-alls are device copies in rank order; each receiver runs the
rows it got (one expert each, k = 1) through the grouped GEMM; each sender
combines the returned rows through its inverse order.  The result must be
bitwise the all-local backend (placement invariance, ep.py:1-8), the send
buffer and counts must match the oracle's destination sort, and a row for a
non-resident expert must raise like ep.py:230.
"""
import json

import numpy as np
import pytest
import torch

from helpers import banner, to_np
from miniep_amd import (EmulatedEPExchangeBackend, EPStats, HipEPShareBackend, HipMoEBackend, Placement, ops,
                        route, workloads)
from miniep_amd._lib import NotResidentError
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("plan_kind,masked", [("balanced", False), ("balanced", True), ("naive", False)])
def test_exchange_equals_local_bitwise(golden_dir, plan_kind, masked):
    banner(f"ep exchange world 4, {plan_kind} placement, masked={masked}")
    if plan_kind == "balanced":
        p = Placement.from_plan(json.loads((golden_dir / "plan_balanced.json").read_text()), device=DEV)
    else:
        p = Placement.naive(24, 32, 4, device=DEV)
    L = workloads.make_layer(8192, seed=6, zipf_s=1.1)
    bf = torch.bfloat16
    x = L.x.to(bf).to(DEV)
    wi, wo = L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
    idx, gate = route(x, L.w_router.to(bf).to(DEV), 8)
    valid = None
    if masked:
        valid = (torch.rand(8192, generator=torch.Generator().manual_seed(2)) < 0.8).to(DEV)
    local = HipMoEBackend(wi, wo)(x, idx, gate, valid)
    stats = EPStats(24, 32, device=DEV)
    ep = EmulatedEPExchangeBackend(2, p, 4, wi, wo, stats=stats)
    got = ep(x, idx, gate, valid)
    assert torch.equal(local, got)
    # every valid entry was computed exactly once, on some rank
    n_valid = 8 * (8192 if valid is None else int(valid.sum()))
    assert int(stats.recv_tokens_per_layer[2]) == n_valid
    assert int(stats.route_counts[2].sum()) == n_valid


def test_send_side_matches_oracle(golden_dir):
    banner("ep send side vs oracle destination sort")
    p = Placement.from_plan(json.loads((golden_dir / "plan_balanced.json").read_text()), device=DEV)
    L = workloads.make_layer(4096, seed=7, zipf_s=1.1)
    bf = torch.bfloat16
    x = L.x.to(bf).to(DEV)
    idx, _ = route(x, L.w_router.to(bf).to(DEV), 8)
    r = 1
    ids = p.experts_of_rank(r)[2]
    be = HipEPShareBackend(2, p, r, L.w_in[ids].to(bf).to(DEV), L.w_out[ids].to(bf).to(DEV))
    rr = torch.zeros(1, 32, dtype=torch.long, device=DEV)
    b = be.send(x, idx, rr=rr)
    t_ref, n_ref = O.build_table(p.owners[2])
    rr0 = np.zeros((1, 32), np.int64)
    ref = O.dispatch(to_np(idx), None, 32, t_ref, n_ref, rr0, [0, 4096], -1, np.full(32, -1))
    dest = ref["dest"]
    order = np.argsort(dest, kind="stable")                         # ep.py:220
    assert to_np(b.send_counts).tolist() == np.bincount(dest, minlength=4).tolist()
    assert to_np(b.experts).tolist() == to_np(idx).reshape(-1)[order].tolist()
    assert torch.equal(b.x, x[torch.from_numpy(order // 8).to(DEV)])
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)                              # ep.py:239
    assert to_np(b.inv)[: 4096 * 8].tolist() == inv.tolist()
    assert to_np(rr).tolist() == ref["rr_after"].tolist()


def test_receiver_rejects_non_resident_expert():
    banner("ep receive: non-resident expert")
    p = Placement.naive(1, 8, 2, device=DEV)
    w_in = torch.randn(4, 256, 256, device=DEV, dtype=torch.bfloat16)
    w_out = torch.randn(4, 256, 128, device=DEV, dtype=torch.bfloat16)
    be = HipEPShareBackend(0, p, 0, w_in, w_out)                    # experts 0..3 live on rank 0
    rx = torch.randn(5, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(NotResidentError):
        be.receive(rx, torch.tensor([0, 1, 5, 2, 3], device=DEV))
    y = be.receive(rx, torch.tensor([0, 1, 3, 2, 3], device=DEV))
    assert y.shape == (5, 256)


def test_gather_rows_and_combine_rows_direct():
    banner("gather_rows / combine_rows")
    g = torch.Generator().manual_seed(3)
    x = torch.randn(37, 1024, generator=g).to(torch.bfloat16).to(DEV)
    perm = torch.randperm(37 * 4, generator=g).to(torch.int32).to(DEV)
    topk = torch.randint(0, 16, (37, 4), generator=g).to(DEV)
    rows, ids = ops.gather_rows(x, perm, 100, 4, topk)
    pr = to_np(perm)[:100]
    assert torch.equal(rows, x[torch.from_numpy(pr // 4).long().to(DEV)])
    assert to_np(ids).tolist() == to_np(topk).reshape(-1)[pr].tolist()
    # combine_rows through an inverse order equals the plain combine on the reordered rows
    y = torch.randn(37 * 4, 1024, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.softmax(torch.randn(37, 4, generator=g), -1).to(torch.bfloat16).to(DEV)
    order = torch.randperm(37 * 4, generator=g)
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel())
    present = torch.ones(37 * 4, dtype=torch.int32)
    present[::7] = -1
    inv_p = torch.where(present >= 0, inv, torch.full_like(inv, -1)).to(torch.int32).to(DEV)
    a = ops.combine_rows(y[order.to(DEV)], gate, inv_p)
    b = ops.combine(y, gate, present.to(DEV))
    assert torch.equal(a, b)
