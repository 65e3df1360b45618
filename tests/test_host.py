"""Host-side tests that need no GPU: the C-ABI library, plan I/O and the balancer.

The balancer KAT is the one reference-held golden vector of the path:
results/plan_balanced.json is the reference's plan_balanced() output for the
summed routing counts of results/bench_naive.json at world 4 with 2 replica
slots per rank (scripts/make_plan.py:24-29).
"""
import ctypes
import json

import numpy as np
import pytest
import torch

from miniep_amd import Placement, _lib, plan_balanced
from oracle import moe_oracle as O


def test_library_exports_every_header_function():
    L = _lib.lib()
    names = _lib.header_functions()
    assert len(names) == 25
    for n in names:
        assert hasattr(L, n), n
    assert L.mep_abi_version() == 5
    assert _lib.last_error() == ""


def test_dispatch_rejects_missing_outputs_before_launch():
    """mep_dispatch validates its arguments on the host before anything is
    enqueued: an output the kernels would write may not be NULL.  (The
    pointers below are placeholders that are never dereferenced.)"""
    L = _lib.lib()
    fake = 4096
    seg = (ctypes.c_int64 * 2)(0, 64)

    def call(n_tokens, n_local, counts, perm, row):
        seg[1] = n_tokens
        return L.mep_dispatch(fake, None, n_tokens, 8, 32, fake, fake, 1, 0, None, seg, 1, 0, fake, n_local,
                              counts, fake, perm, row, None, None, fake, 1 << 20, None)

    # sender mode (n_local = 0): row_of_entry is still written for every entry
    assert call(64, 0, None, None, None) == _lib.ERR_INVALID_ARG
    assert b"row_of_entry" in L.mep_last_error()
    # no tokens but local experts: counts are still written
    assert call(0, 4, None, fake, fake) == _lib.ERR_INVALID_ARG
    assert b"counts" in L.mep_last_error()
    # tokens and local experts: perm receives the kept rows
    assert call(64, 4, fake, None, fake) == _lib.ERR_INVALID_ARG
    assert b"perm" in L.mep_last_error()
    assert call(64, 4, fake, fake, None) == _lib.ERR_INVALID_ARG


def test_experts_combine_rejects_bad_arguments_before_launch():
    """mep_grouped_swiglu_combine checks on the host that y_entries covers
    every (token, slot) cell (max_rows = n_tokens * top_k) and that the
    combine's inputs and output are given, before anything is enqueued.
    (Placeholder pointers, never dereferenced.)"""
    L = _lib.lib()
    fake = 4096
    BF16 = 1

    def call(n, max_rows, row, gate, out):
        return L.mep_grouped_swiglu_combine(fake, n, 8, fake, fake, row, gate, None, 32, max_rows, fake, fake,
                                            1024, 512, BF16, fake, fake, 1 << 30, fake, 1 << 20, out, None)

    assert call(32, 255, fake, fake, fake) == _lib.ERR_INVALID_ARG
    assert b"max_rows" in L.mep_last_error()
    for row, gate, out in ((None, fake, fake), (fake, None, fake), (fake, fake, None)):
        assert call(32, 256, row, gate, out) == _lib.ERR_INVALID_ARG
        assert b"null" in L.mep_last_error()
    assert call(0, 0, None, None, None) == 0          # nothing to do: no pointer is needed


def test_workspace_size_queries():
    L = _lib.lib()
    seg = (ctypes.c_int64 * 2)(0, 16384)
    ws = L.mep_dispatch_workspace_size(16384, 8, 32, 1, seg)
    # header + 2 flag words per block + rr snapshot + per-block histograms (128 blocks)
    assert ws >= 256 + 8 * 128 + 8 * 32 + 4 * 128 * 32
    seg4 = (ctypes.c_int64 * 5)(0, 2048, 4096, 6144, 8192)
    assert L.mep_dispatch_workspace_size(8192, 8, 32, 4, seg4) >= 4 * 32 * 8
    assert L.mep_dispatch_workspace_size(10, 8, 32, 17, None) >= 0
    assert L.mep_experts_workspace_size(131072, 512, _lib.DTYPE_BF16) >= 131072 * 512 * 2
    assert L.mep_experts_workspace_size(4096, 512, _lib.DTYPE_F32) >= 4096 * 512 * 4
    assert L.mep_experts_workspace_size(4096, 512, 7) == 0


def test_plan_balanced_reproduces_reference_plan(golden_dir):
    rc = json.loads((golden_dir / "route_counts_bench_naive.json").read_text())
    ref = json.loads((golden_dir / "plan_balanced.json").read_text())
    placement, report = plan_balanced(torch.tensor(rc["counts"]), rc["world"],
                                      slots_per_rank=rc["slots_per_rank"],
                                      target_ratio=rc["target_ratio"], device="cpu")
    assert placement.to_plan() == ref
    # README.md of the reference: 71 replicas in the balanced plan
    assert report["replicas_total"] == 71
    assert all(l["imbalance_after"] <= l["imbalance_before"] for l in report["layers"])


def _plan_by_full_resum(counts, world, per, slots_per_rank, target):
    """A second statement of the planner for the cross-check below: every
    trial re-sums every rank from scratch, in expert order."""
    owners = [[e // per] for e in range(len(counts))]
    slots = [slots_per_rank] * world

    def loads(own):
        out = [0.0] * world
        for e, o in enumerate(own):
            for r in o:
                out[r] += counts[e] / len(o)
        return out

    mean = sum(loads(owners)) / world
    while mean and max(loads(owners)) / mean > target:
        cur, best = max(loads(owners)), None
        for e in range(len(counts)):
            if counts[e] / len(owners[e]) == 0:
                continue
            for r in range(world):
                if r in owners[e] or slots[r] <= 0:
                    continue
                trial = [list(o) for o in owners]
                trial[e] = sorted(trial[e] + [r])
                m = max(loads(trial))
                if m < cur and (best is None or m < best[0]):
                    best = (m, e, r)
        if best is None:
            break
        owners[best[1]] = sorted(owners[best[1]] + [best[2]])
        slots[best[2]] -= 1
    return owners


@pytest.mark.parametrize("world", [2, 4, 8])
def test_plan_balanced_matches_full_resummation(world):
    """The planner re-sums only the ranks a candidate touches; on skewed,
    tie-heavy random counts its plans equal those of re-summing every rank
    for every trial."""
    rng = np.random.default_rng(world)
    E = 32
    counts = np.zeros((40, E), dtype=np.int64)
    for l in range(40):
        p = np.arange(1, E + 1, dtype=np.float64) ** -rng.uniform(0.3, 1.6)
        rng.shuffle(p)
        counts[l] = rng.multinomial(int(rng.integers(50, 5000)), p / p.sum())
        if l % 5 == 0:
            counts[l] = (counts[l] // 100) * 100          # many exact ties
        if l % 7 == 0:
            counts[l, rng.integers(0, E, 6)] = 0          # idle experts
    slots, target = (2, 1.05) if world < 8 else (1, 1.02)
    placement, report = plan_balanced(torch.tensor(counts), world, slots_per_rank=slots,
                                      target_ratio=target, device="cpu")
    for l in range(counts.shape[0]):
        ref = _plan_by_full_resum(counts[l].astype(float).tolist(), world, E // world, slots, target)
        assert placement.owners[l] == ref, f"layer {l}"
    assert report["replicas_total"] == sum(len(o) for lay in placement.owners for o in lay) - 40 * E


def test_placement_plan_io_and_tables(golden_dir):
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device="cpu")
    assert p.to_plan() == plan
    assert p.num_layers == 24 and p.num_experts == 32
    # layer 2: 8 owned + 2 replica experts on every rank
    for r in range(4):
        assert len(p.experts_of_rank(r)[2]) == 10
    for l in range(24):
        t_ref, n_ref = O.build_table(p.owners[l])
        t, n = p.tables(l)
        assert np.array_equal(t.numpy(), t_ref) and np.array_equal(n.numpy(), n_ref)
        assert p.has_replicas(l) == bool((n_ref != 1).any())
    naive = Placement.naive(24, 32, 4, device="cpu")
    assert naive.experts_of_rank(3)[0] == list(range(24, 32))
    assert not naive.has_replicas(0)
    with pytest.raises(ValueError):
        Placement.naive(1, 30, 4, device="cpu")
    with pytest.raises(ValueError):
        Placement([[[0], []]], device="cpu")


def test_ops_reject_cpu_tensors():
    from miniep_amd import ops
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.router_topk(torch.zeros(4, 256), torch.zeros(32, 256), 8)


def test_dispatch_noalloc_rejects_calls_beyond_its_scratch():
    """The allocation-free dispatch checks its size limit on the host, before
    it touches the device: 2^22 entries with 256 experts need more than the
    2 MiB static scratch."""
    L = _lib.lib()
    fake = 4096
    n = 1 << 19
    seg = (ctypes.c_int64 * 2)(0, n)
    assert L.mep_dispatch_workspace_size(n, 8, 256, 1, seg) > (2 << 20)
    rc = L.mep_dispatch_noalloc(fake, None, n, 8, 256, fake, fake, 1, 0, None, seg, 1, 0, fake, 256,
                                fake, fake, fake, fake, None, None, None, None)
    assert rc == _lib.ERR_UNSUPPORTED and b"static scratch" in L.mep_last_error()
