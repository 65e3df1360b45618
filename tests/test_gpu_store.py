"""Expert weights in slots (ExpertStore) and the live re-placement of
server.py:51-62 on top of them.

- the grouped GEMM reading local expert j from slot w_slot[j] gives the same
  bits as the same experts sliced into a contiguous (sorted-id) array;
- a world-4 re-placement over 24 layers (naive -> the reference's balanced
  plan -> naive) copies exactly the arriving experts (the plan's 71 replicas,
  then none), and after each swap the world-4 emulated expert-parallel output
  of every layer is bitwise the all-local output (the placement invariance of
  ep.py:1-8).
"""
import json

import pytest
import torch

from helpers import banner
from miniep_amd import EmulatedEPMoEBackend, ExpertStore, HipEPShareBackend, HipMoEBackend, Placement, \
    apply_placement, ops, route, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


@pytest.mark.parametrize("n", [4096, 32])
def test_slots_give_the_bits_of_sliced_weights(golden_dir, n):
    """4096 tokens: the rank share runs the tiled kernel; 32 tokens (about 64
    rows per rank): the small-batch one launch, whose GEMM-2 workgroups also
    DMA weight steps into LDS from the slot's weights."""
    banner(f"expert slots vs sliced weights, {n} tokens")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    L = workloads.make_layer(n, seed=8, zipf_s=1.1)
    wi, wo = L.w_in.to(BF).to(DEV), L.w_out.to(BF).to(DEV)
    x = L.x.to(BF).to(DEV)
    idx, _ = route(x, L.w_router.to(BF).to(DEV), 8)
    r = 2
    ids = p.experts_of_rank(r)[2]
    store = ExpertStore(24, 12, 1024, 512, BF, DEV)
    # fill the slots out of order: 8 other experts first, then the rank's set
    # (its experts land in the free slots around the kept ones)
    other = [e for e in range(32) if e not in ids][:8]
    assert store.assign(2, other + ids[:2], wi, wo) == 10
    assert store.assign(2, ids, wi, wo) == len(ids) - 2
    assert store.w_slot[2].tolist() != list(range(len(ids)))
    seg = [n * q // 4 for q in range(5)]
    y_s = torch.full((n * 8, 1024), float("nan"), dtype=BF, device=DEV)
    y_w = y_s.clone()
    d1, _ = HipEPShareBackend(2, p, r, store=store).share(x, idx, seg_tokens=seg, y_entries=y_s)
    d2, _ = HipEPShareBackend(2, p, r, wi[ids], wo[ids]).share(x, idx, seg_tokens=seg, y_entries=y_w)
    M = int(d1.offsets[-1])                      # perm is defined for the first M rows
    assert M > 0
    rows = d1.perm[:M].long()
    assert torch.equal(d1.perm[:M], d2.perm[:M]) and torch.equal(y_s[rows], y_w[rows])
    assert not torch.isnan(y_s[rows].float()).any()


def test_live_replacement_copies_only_arriving_experts(golden_dir):
    banner("live re-placement over 24 layers, world 4")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    balanced = Placement.from_plan(plan, device=DEV)
    naive = Placement.naive(24, 32, 4, device=DEV)
    g = torch.Generator().manual_seed(21)
    ck_in = (torch.randn(24, 32, 1024, 1024, generator=g) * 0.02).to(BF).to(DEV)
    ck_out = (torch.randn(24, 32, 1024, 512, generator=g) * 0.02).to(BF).to(DEV)
    checkpoint = (ck_in, ck_out)                 # all layers in one launch per rank
    stores = [ExpertStore(24, 10, 1024, 512, BF, DEV) for _ in range(4)]
    for r, st in enumerate(stores):
        for l in range(24):
            st.assign(l, naive.experts_of_rank(r)[l], ck_in[l], ck_out[l])
    lay = workloads.make_layer(2048, seed=22, zipf_s=1.1)
    x = lay.x.to(BF).to(DEV)
    idx, gate = route(x, lay.w_router.to(BF).to(DEV), 8)
    seg = [0, 512, 1024, 1536, 2048]

    def check_all_layers(placement):
        for l in range(24):
            local = HipMoEBackend(ck_in[l], ck_out[l])(x, idx, gate)
            ep = EmulatedEPMoEBackend(l, placement, 4, stores=stores)
            assert torch.equal(ep(x, idx, gate, seg_tokens=seg), local), f"layer {l}"

    check_all_layers(naive)
    copied, secs = 0, 0.0
    for r, st in enumerate(stores):
        res = apply_placement([], st, balanced, r, checkpoint)
        copied += res["copied"]
        secs += res["seconds"]
    replicas = sum(len(o) - 1 for layer in balanced.owners for o in layer)
    print(f"naive -> balanced: {copied} experts copied ({replicas} replicas in the plan), "
          f"{1e3 * secs:.2f} ms over 4 ranks x 24 layers", flush=True)
    assert copied == replicas == 71
    check_all_layers(balanced)
    # back to the naive placement, one layer per launch this time (the callable checkpoint)
    back = sum(apply_placement([], st, naive, r, lambda l: (ck_in[l], ck_out[l]))["copied"]
               for r, st in enumerate(stores))
    assert back == 0                              # the owned experts never left their slots
    check_all_layers(naive)


def test_store_rejects_overflow_and_bad_ids():
    banner("expert store limits")
    store = ExpertStore(1, 4, 256, 128, BF, DEV)
    wi = torch.zeros(8, 256, 256, dtype=BF, device=DEV)
    wo = torch.zeros(8, 256, 128, dtype=BF, device=DEV)
    with pytest.raises(ValueError):
        store.assign(0, [0, 1, 2, 3, 4], wi, wo)
    with pytest.raises(ValueError):
        store.assign(0, [9], wi, wo)
    with pytest.raises(Exception):
        ops.copy_experts(wi, wo, [0, 1], store.w_in[0], store.w_out[0], [2, 2])   # one slot twice
