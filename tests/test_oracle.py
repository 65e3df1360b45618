"""Pins of the CPU oracle (runs without a GPU).

Every oracle function is checked against something that does not share its
code: torch's own ops (the routines the reference calls), brute-force Python
loops over tiny inputs, hand-derived known answers, or closed forms.  The
``test_mutant_*`` tests plant plausible mistakes in copies of oracle functions
and show that these pins fail on them.
"""
import itertools
import math

import numpy as np
import pytest
import torch

from helpers import tie_free
from oracle import moe_oracle as O


# ---------------------------------------------------------------- bf16 ------
def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 10000).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, -1.0, 3.3895314e38, 1e-45, np.inf, -np.inf], np.float32)])
    v = v.astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    got = O.bf16_round(v)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_bf16_ties_round_to_even():
    # 1 + 2^-8 lies exactly between bf16 neighbours 1 and 1 + 2^-7 -> even (1.0)
    assert O.bf16_round(np.float32(1 + 2 ** -8)) == np.float32(1.0)
    assert O.bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)


# ---------------------------------------------------------------- router ----
def test_router_logits_brute_force():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 16)).astype(np.float32)
    w = rng.standard_normal((5, 16)).astype(np.float32)
    got = O.router_logits(x, w)
    for t in range(3):
        for e in range(5):
            ref = math.fsum(float(x[t, i]) * float(w[e, i]) for i in range(16))
            assert got[t, e] == np.float32(ref)


def test_topk_softmax_matches_torch_on_tie_free_rows():
    """torch.topk / torch.softmax are the ops the reference calls (modeling.py:194-195)."""
    g = torch.Generator().manual_seed(2)
    lg = torch.randn(512, 32, generator=g)
    s = lg.sort(dim=-1, descending=True).values
    assert not (s[:, :-1] == s[:, 1:]).any()
    ref_v, ref_i = lg.topk(8, dim=-1)
    ref_g = torch.softmax(ref_v.float(), dim=-1)
    idx, gate = O.topk_softmax(lg.numpy(), 8)
    assert np.array_equal(idx, ref_i.numpy())
    np.testing.assert_allclose(gate, ref_g.numpy(), rtol=2e-6, atol=1e-7)
    _, gate_b = O.topk_softmax(lg.numpy(), 8, gate_bf16=True)
    ref_b = ref_g.to(torch.bfloat16).float().numpy()
    assert np.abs(gate_b - ref_b).max() <= 2 ** -8 * ref_b.max()


def test_topk_tie_rule_brute_force():
    """Equal logits: lower expert id first (the kernels' documented rule)."""
    rng = np.random.default_rng(3)
    lg = rng.integers(-3, 4, size=(200, 12)).astype(np.float32)   # many ties
    idx, gate = O.topk_softmax(lg, 5)
    for t in range(200):
        order = sorted(range(12), key=lambda e: (-float(lg[t, e]), e))[:5]
        assert list(idx[t]) == order
        ex = [math.exp(float(lg[t, e]) - float(lg[t, order[0]])) for e in order]
        np.testing.assert_allclose(gate[t], np.array(ex) / sum(ex), rtol=1e-6)


def test_topk_gate_invariants():
    rng = np.random.default_rng(4)
    lg = (rng.standard_normal((100, 32)) * 3).astype(np.float32)
    idx, gate = O.topk_softmax(lg, 8)
    np.testing.assert_allclose(gate.sum(1), 1.0, rtol=1e-6)
    assert (np.diff(gate, axis=1) <= 0).all()                       # descending
    sel = np.take_along_axis(lg, idx, 1)
    np.testing.assert_allclose(np.log(gate[:, 1] / gate[:, 0]), sel[:, 1] - sel[:, 0], atol=1e-5)


# -------------------------------------------------------- flatten / order ---
def test_flatten_topk_loops():
    rng = np.random.default_rng(5)
    for n, k in [(0, 8), (1, 1), (7, 3), (13, 8)]:
        mask = rng.random(n) < 0.6
        tok, slot, keep_e = O.flatten_topk(n, k, mask)
        ref = [(t, s) for t in range(n) for s in range(k) if mask[t]]
        assert list(zip(tok.tolist(), slot.tolist())) == ref
        assert keep_e.tolist() == [bool(mask[t]) for t in range(n) for _ in range(k)]
        tok, slot, _ = O.flatten_topk(n, k, None)
        assert list(zip(tok.tolist(), slot.tolist())) == [(t, s) for t in range(n) for s in range(k)]


def test_stable_expert_order_brute_force():
    rng = np.random.default_rng(6)
    for m in [0, 1, 10, 300]:
        ids = rng.integers(0, 6, m)
        order, counts = O.stable_expert_order(ids, 6)
        assert order.tolist() == sorted(range(m), key=lambda f: (ids[f], f))
        assert counts.tolist() == [int((ids == e).sum()) for e in range(6)]


# ------------------------------------------------------------ dest_ranks ----
def test_dest_ranks_hand_kats():
    # expert 24 of plan_balanced layer 2 is held by ranks [0, 1, 3]
    table, n_rep = O.build_table([[0], [0, 1, 3]])
    d, rr = O.dest_ranks(table, n_rep, np.array([0, 0]), np.array([1] * 7))
    assert d.tolist() == [0, 1, 3, 0, 1, 3, 0] and rr.tolist() == [0, 7]
    d, rr = O.dest_ranks(table, n_rep, np.array([0, 2]), np.array([1] * 7))
    assert d.tolist() == [3, 0, 1, 3, 0, 1, 3] and rr.tolist() == [0, 9]
    # interleaved experts: each expert's own occurrence index drives its slot
    d, rr = O.dest_ranks(table, n_rep, np.array([5, 0]), np.array([1, 0, 1, 0, 1]))
    assert d.tolist() == [0, 0, 1, 0, 3] and rr.tolist() == [7, 3]
    # no replicas in the layer: table[e, 0], counters untouched (ep.py:84-85)
    t1, n1 = O.build_table([[2], [1]])
    d, rr = O.dest_ranks(t1, n1, np.array([4, 4]), np.array([0, 1, 1]))
    assert d.tolist() == [2, 1, 1] and rr.tolist() == [4, 4]


def _random_owners(rng, n_exp, world):
    return [sorted(rng.choice(world, size=rng.integers(1, world + 1), replace=False).tolist())
            for _ in range(n_exp)]


def test_dest_ranks_vectorised_equals_entry_loop():
    rng = np.random.default_rng(7)
    for _ in range(300):
        world = int(rng.integers(1, 5))
        n_exp = int(rng.integers(1, 7))
        table, n_rep = O.build_table(_random_owners(rng, n_exp, world))
        rr = rng.integers(0, 20, n_exp)
        ids = rng.integers(0, n_exp, int(rng.integers(0, 40)))
        d1, r1 = O.dest_ranks(table, n_rep, rr, ids)
        d2, r2 = O.dest_ranks_loop(table, n_rep, rr, ids)
        assert d1.tolist() == d2.tolist() and r1.tolist() == r2.tolist()


# --------------------------------------------------------------- dispatch ---
def _brute_share(topk_idx, valid, table, n_rep, rr, seg_tokens, my_rank, local_experts):
    """Per-source simulation with Python loops: each source computes dest with
    the per-entry loop and sends its entries for my_rank in flat order; the
    receiver concatenates by source and sorts stably by local id."""
    n, k = topk_idx.shape
    recv = []
    for s in range(len(seg_tokens) - 1):
        entries = [(t * k + j, int(topk_idx[t, j])) for t in range(seg_tokens[s], seg_tokens[s + 1])
                   for j in range(k) if valid[t]]
        dest, _ = O.dest_ranks_loop(table, n_rep, rr[s], [e for _, e in entries])
        recv += [(f, e) for (f, e), d in zip(entries, dest) if d == my_rank]
    pos = {e: i for i, e in enumerate(local_experts)}
    recv = [(f, e) for f, e in recv if e in pos]
    ordered = sorted(range(len(recv)), key=lambda i: (pos[recv[i][1]], i))
    return [recv[i][0] for i in ordered], [sum(1 for _, e in recv if e == le) for le in local_experts]


def test_dispatch_brute_force_multi_source():
    rng = np.random.default_rng(8)
    for trial in range(60):
        world = int(rng.integers(1, 5))
        E = int(rng.integers(world, 9))
        owners = _random_owners(rng, E, world)
        table, n_rep = O.build_table(owners)
        n, k = int(rng.integers(0, 12)), int(rng.integers(1, min(E, 4) + 1))
        topk = np.stack([rng.permutation(E)[:k] for _ in range(n)]) if n else np.zeros((0, k), np.int64)
        valid = rng.random(n) < 0.8
        S = int(rng.integers(1, 4))
        cuts = sorted(rng.integers(0, n + 1, S - 1).tolist())
        seg = [0] + cuts + [n]
        rr = rng.integers(0, 5, (S, E))
        for r in range(world):
            local = [e for e in range(E) if r in owners[e]]
            g2l = np.full(E, -1)
            g2l[local] = np.arange(len(local))
            res = O.dispatch(topk, valid, E, table, n_rep, rr, seg, r, g2l)
            perm, counts = _brute_share(topk, valid, table, n_rep, rr, seg, r, local)
            assert res["perm"].tolist() == perm, (trial, r)
            assert res["counts"].tolist() == counts
            assert not res["not_resident"]


def test_dispatch_shares_partition_and_world1_filter():
    rng = np.random.default_rng(9)
    plan_owners = [[0, 2], [1], [0, 1, 3], [2, 3], [3], [1, 2], [0], [2]]
    table, n_rep = O.build_table(plan_owners)
    n, k, E, world = 50, 3, 8, 4
    topk = np.stack([rng.permutation(E)[:k] for _ in range(n)])
    valid = rng.random(n) < 0.9
    rr = np.zeros((1, E), np.int64)
    ident = np.arange(E)
    w1 = O.dispatch(topk, valid, E, np.zeros((E, 1), np.int64), np.ones(E, np.int64), rr, [0, n], 0, ident)
    seen = []
    for r in range(world):
        local = [e for e in range(E) if r in plan_owners[e]]
        g2l = np.full(E, -1)
        g2l[local] = np.arange(len(local))
        res = O.dispatch(topk, valid, E, table, n_rep, rr, [0, n], r, g2l)
        dest = res["dest"]
        # single source: rank r's rows = world-1 stable order filtered to dest == r
        assert res["perm"].tolist() == [f for f in w1["perm"].tolist() if dest[f] == r]
        seen += res["perm"].tolist()
    valid_entries = [t * k + s for t in range(n) for s in range(k) if valid[t]]
    assert sorted(seen) == valid_entries                                 # a partition
    assert w1["route_counts"].tolist() == np.bincount(topk[valid].reshape(-1), minlength=E).tolist()


def test_dispatch_flags_non_resident():
    table, n_rep = O.build_table([[0], [0]])
    res = O.dispatch(np.array([[0, 1]]), None, 2, table, n_rep, np.zeros((1, 2)), [0, 1], 0,
                     np.array([0, -1]))
    assert res["not_resident"] and res["perm"].tolist() == [0]


# ---------------------------------------------------------------- experts ---
def _silu(v):
    return v / (1.0 + math.exp(-v))


def test_experts_brute_force_float64():
    rng = np.random.default_rng(10)
    E, H, I = 3, 8, 4
    w_in = rng.standard_normal((E, 2 * I, H)).astype(np.float32)
    w_out = rng.standard_normal((E, H, I)).astype(np.float32)
    x = rng.standard_normal((7, H)).astype(np.float32)
    ids = np.array([2, 0, 2, 1, 0, 2, 1])
    got = O.experts(x, ids, w_in, w_out)
    for r in range(7):
        e = ids[r]
        a = [_silu(sum(float(w_in[e, j, i]) * float(x[r, i]) for i in range(H))) *
             sum(float(w_in[e, I + j, i]) * float(x[r, i]) for i in range(H)) for j in range(I)]
        y = [sum(float(w_out[e, o, j]) * a[j] for j in range(I)) for o in range(H)]
        np.testing.assert_allclose(got[r], y, rtol=1e-5, atol=1e-5)


def test_combine_closed_form():
    rng = np.random.default_rng(11)
    n, k, H = 5, 3, 4
    y = rng.standard_normal((n * k, H)).astype(np.float32)
    g = rng.random((n, k)).astype(np.float32)
    present = rng.random(n * k) < 0.7
    got = O.combine(y, g, present, n, k)
    for t in range(n):
        ref = sum(g[t, s] * y[t * k + s].astype(np.float64) for s in range(k) if present[t * k + s])
        np.testing.assert_allclose(got[t], ref if np.ndim(ref) else np.zeros(H), rtol=1e-6, atol=1e-7)


def test_moe_layer_per_token_loop():
    rng = np.random.default_rng(12)
    n, E, k, H, I = 6, 4, 2, 8, 4
    x = rng.standard_normal((n, H)).astype(np.float32)
    w_r = rng.standard_normal((E, H)).astype(np.float32)
    w_in = rng.standard_normal((E, 2 * I, H)).astype(np.float32)
    w_out = rng.standard_normal((E, H, I)).astype(np.float32)
    valid = np.array([1, 1, 0, 1, 1, 0], bool)
    idx, gate = O.topk_softmax(O.router_logits(x, w_r), k)
    got = O.moe_layer_local(x, idx, gate, w_in, w_out, valid)
    for t in range(n):
        ref = np.zeros(H)
        if valid[t]:
            for s in range(k):
                e = idx[t, s]
                h = w_in[e].astype(np.float64) @ x[t].astype(np.float64)
                a = h[:I] / (1 + np.exp(-h[:I])) * h[I:]
                ref += gate[t, s] * (w_out[e].astype(np.float64) @ a)
        np.testing.assert_allclose(got[t], ref, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------- mutants ------
def test_mutant_dest_off_by_one_is_caught():
    def bad(table, n_rep, rr, ids):
        d, r = O.dest_ranks(table, n_rep, np.asarray(rr) + 1, ids)
        return d, r - 1
    table, n_rep = O.build_table([[0, 1, 3]])
    assert bad(table, n_rep, [0], [0] * 4)[0].tolist() != O.dest_ranks_loop(table, n_rep, [0], [0] * 4)[0].tolist()


def test_mutant_tie_break_is_caught():
    lg = np.array([[1.0, 2.0, 2.0, 0.0]], np.float32)
    bad = np.argsort(-lg[:, ::-1], axis=1, kind="stable")[:, :2]
    bad = lg.shape[1] - 1 - bad
    good = sorted(range(4), key=lambda e: (-float(lg[0, e]), e))[:2]
    assert O.topk_softmax(lg, 2)[0][0].tolist() == good and bad[0].tolist() != good


def test_mutant_swapped_gate_up_is_caught():
    rng = np.random.default_rng(13)
    w_in = rng.standard_normal((1, 8, 4)).astype(np.float32)
    w_out = rng.standard_normal((1, 4, 4)).astype(np.float32)
    x = rng.standard_normal((3, 4)).astype(np.float32)
    swapped = np.concatenate([w_in[:, 4:], w_in[:, :4]], axis=1)
    assert not np.allclose(O.experts(x, np.zeros(3, int), swapped, w_out),
                           O.experts(x, np.zeros(3, int), w_in, w_out), rtol=1e-3)


def test_torch_cpu_restatement_matches_numpy_oracle():
    """The PyTorch-CPU restatement that bench.py times as the CPU baseline
    computes the same layer as the numpy oracle (tie-free routing, masks)."""
    from oracle import torch_cpu as TC
    g = torch.Generator().manual_seed(4)
    n, H, E, I, k = 300, 256, 16, 128, 4
    x = torch.randn(n, H, generator=g)
    wr = torch.randn(E, H, generator=g) * 0.05
    wi = torch.randn(E, 2 * I, H, generator=g) * 0.05
    wo = torch.randn(E, H, I, generator=g) * 0.05
    valid = torch.rand(n, generator=g) < 0.8
    lg = O.router_logits(x.numpy(), wr.numpy())
    assert tie_free(lg, k)
    idx, gate = TC.route(x, wr, k)
    ridx, rgate = O.topk_softmax(lg, k)
    assert np.array_equal(idx.numpy(), ridx)
    np.testing.assert_allclose(gate.numpy(), rgate, rtol=1e-5, atol=1e-6)
    out = TC.moe_local(x, idx, gate, wi, wo, valid).numpy()
    ref = O.moe_layer_local(x.numpy(), ridx, rgate, wi.numpy(), wo.numpy(), valid.numpy())
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()
    assert (out[~valid.numpy()] == 0).all()
    # a planted mistake (gate and up halves swapped) is caught by the same check
    bad = TC.moe_local(x, idx, gate, torch.cat([wi[:, I:], wi[:, :I]], 1), wo, valid).numpy()
    assert np.abs(bad - ref).max() > 1e-2 * np.abs(ref).max()
