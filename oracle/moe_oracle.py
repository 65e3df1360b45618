"""CPU oracle for the GraniteMoE MoE-block hot path (numpy only).

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only
to compute expected results or the timed CPU baseline.  The HIP path never
calls into it.

Each function restates one piece of the reference algorithm (mini-EP,
``miniep/modeling.py`` and ``miniep/ep.py``) in plain numpy so that the GPU
kernels can be compared against it on identical inputs:

=====================  ==========================================  =============
function               follows (reference file:line)               pinned by
=====================  ==========================================  =============
router_logits          modeling.py:193 (x_flat @ W_r.T)            float64 dot
topk_softmax           modeling.py:194-195 (topk, fp32 softmax)    torch.topk /
                                                                   brute force
flatten_topk           modeling.py:107-117                         python loops
stable_expert_order    modeling.py:94-96 (argsort stable,          brute force
                       unique_consecutive)
build_table            ep.py:35-45 (_build_table)                  plan KAT
dest_ranks             ep.py:76-96 (vectorised round-robin)        per-entry loop
dest_ranks_loop        ep.py:79-82 (the per-entry loop it states)  hand KATs
dispatch               ep.py:210-231 + modeling.py:94-96           brute force,
                       (rank-local share, g2l, stable order)       world-1 filter
experts                modeling.py:83-104 (run_experts)            float64 loop
combine                modeling.py:120-128,144 (gate, scatter,     closed form
                       slot-order sum)
moe_layer_local        modeling.py:131-145 (LocalMoEBackend)       per-token
                                                                   float64 loop
=====================  ==========================================  =============

The tie rule of ``topk_softmax`` is "larger logit first, lower expert index
first among equal logits".  torch's CPU ``topk`` orders tied values in an
implementation-defined way, so the rule is pinned against torch only on
tie-free rows; tied rows are pinned by brute force against the stated rule.

bf16 is represented as float32 arrays whose values are exactly representable
in bf16 (``bf16_round``), or as raw uint16 bit patterns (``bf16_bits``).
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round", "bf16_bits", "bf16_from_bits",
    "router_logits", "topk_softmax", "flatten_topk", "stable_expert_order",
    "build_table", "dest_ranks", "dest_ranks_loop", "dispatch", "experts",
    "combine", "moe_layer_local", "silu",
]


# ----------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, the rounding torch uses for .to(bf16))
# ----------------------------------------------------------------------------
def bf16_bits(a) -> np.ndarray:
    """float32 array -> uint16 bf16 bit patterns, round-to-nearest-even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(a, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_from_bits(b) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(a) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return bf16_from_bits(bf16_bits(a))


def silu(v):
    return v / (1.0 + np.exp(-v))


# ----------------------------------------------------------------------------
# a1: router  (modeling.py:192-195)
# ----------------------------------------------------------------------------
def router_logits(x, w_router) -> np.ndarray:
    """logits = x_flat @ W_r.T (modeling.py:193), accumulated in float64 and
    rounded once to float32.  x: (N, H), w_router: (E, H) -> (N, E) float32."""
    return (np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T).astype(np.float32)


def topk_softmax(logits, k, gate_bf16=False):
    """topk(k) sorted descending + float32 softmax over the k selected logits
    (modeling.py:194-195).  Returns (idx int64 (N,k), gate float32 (N,k)); with
    ``gate_bf16`` the gate is rounded to bf16 as ``.to(x.dtype)`` does for a
    bf16 model.  Equal logits: lower expert index first."""
    lg = np.asarray(logits, np.float32)
    n, e = lg.shape
    if n == 0:
        return np.zeros((0, k), np.int64), np.zeros((0, k), np.float32)
    # stable sort of the negated values: descending, ties keep index order
    idx = np.argsort(-lg, axis=1, kind="stable")[:, :k].astype(np.int64)
    tl = np.take_along_axis(lg, idx, axis=1)
    ex = np.exp(tl - tl[:, :1]).astype(np.float32)
    gate = (ex / ex.sum(axis=1, dtype=np.float32, keepdims=True)).astype(np.float32)
    if gate_bf16:
        gate = bf16_round(gate)
    return idx, gate


# ----------------------------------------------------------------------------
# a2/a3: flatten + stable order by expert  (modeling.py:107-117, :94-96)
# ----------------------------------------------------------------------------
def flatten_topk(n, k, valid_mask=None):
    """(token_ids, slot_ids, keep_e) exactly as modeling.py:107-117:
    entries f = t*k + s in token-major, slot-minor order, invalid tokens
    dropped."""
    keep = np.ones(n, bool) if valid_mask is None else np.asarray(valid_mask, bool)
    keep_e = np.repeat(keep, k)
    token_ids = np.repeat(np.arange(n, dtype=np.int64), k)[keep_e]
    slot_ids = np.tile(np.arange(k, dtype=np.int64), n)[keep_e]
    return token_ids, slot_ids, keep_e


def stable_expert_order(expert_ids, n_experts):
    """order = argsort(expert_ids, stable=True); counts = bincount
    (modeling.py:94-96; unique_consecutive keeps only the non-empty experts,
    which are the nonzero entries of the full bincount)."""
    ids = np.asarray(expert_ids, np.int64)
    order = np.argsort(ids, kind="stable").astype(np.int64)
    counts = np.bincount(ids, minlength=n_experts).astype(np.int64)
    return order, counts


# ----------------------------------------------------------------------------
# a4: replica round-robin  (ep.py:35-45, :76-96)
# ----------------------------------------------------------------------------
def build_table(owners_l):
    """table[e, j] = rank of expert e's j-th replica, n_rep[e] = #replicas
    (ep.py:35-45).  Unused cells are 0, as in the reference."""
    n_exp = len(owners_l)
    rmax = max(len(o) for o in owners_l)
    table = np.zeros((n_exp, rmax), np.int64)
    n_rep = np.zeros(n_exp, np.int64)
    for e, o in enumerate(owners_l):
        table[e, :len(o)] = o
        n_rep[e] = len(o)
    return table, n_rep


def dest_ranks(table, n_rep, rr_layer, expert_ids):
    """Vectorised round-robin of ep.py:76-96.

    Returns (dest, rr_after).  When no expert of the layer is replicated the
    reference returns ``table[e, 0]`` and leaves the counters untouched
    (ep.py:84-85); otherwise the i-th occurrence (flat order) of expert e goes
    to replica (rr[e] + i) % n_rep[e] and rr[e] += count[e] (ep.py:86-96).
    """
    ids = np.asarray(expert_ids, np.int64)
    rr = np.array(rr_layer, np.int64, copy=True)
    if (np.asarray(n_rep) == 1).all():
        return table[ids, 0].astype(np.int64), rr
    m = ids.size
    n_exp = table.shape[0]
    counts = np.bincount(ids, minlength=n_exp).astype(np.int64)
    order = np.argsort(ids, kind="stable")
    srt = ids[order]
    starts = np.cumsum(counts) - counts
    within_sorted = np.arange(m, dtype=np.int64) - starts[srt]
    within = np.empty_like(within_sorted)
    within[order] = within_sorted
    slot = (rr[ids] + within) % n_rep[ids]
    rr += counts
    return table[ids, slot].astype(np.int64), rr


def dest_ranks_loop(table, n_rep, rr_layer, expert_ids):
    """The per-entry loop whose assignment ep.py:79-82 says the vectorised
    version reproduces: entry after entry, expert e goes to replica
    rr[e] % n_rep[e], then rr[e] += 1.  (Small inputs only.)"""
    rr = [int(v) for v in rr_layer]
    any_rep = any(int(r) != 1 for r in n_rep)
    out = []
    for e in (int(v) for v in expert_ids):
        if not any_rep:
            out.append(int(table[e][0]))
            continue
        out.append(int(table[e][rr[e] % int(n_rep[e])]))
        rr[e] += 1
    rr_after = np.array(rr if any_rep else list(rr_layer), np.int64)
    return np.array(out, np.int64), rr_after


# ----------------------------------------------------------------------------
# a5: one GPU's share of the EP dispatch  (ep.py:210-231 with run_experts' sort)
# ----------------------------------------------------------------------------
def dispatch(topk_idx, valid_mask, n_experts, table, n_rep, rr, seg_tokens,
             my_rank, g2l):
    """Rank ``my_rank``'s share of the entries, in the order its experts see them.

    topk_idx (N,k); valid_mask (N,) bool or None; table/n_rep from
    ``build_table``; rr (S, E) round-robin counters, one row per source
    segment; seg_tokens: S+1 token offsets, segment s = tokens
    [seg_tokens[s], seg_tokens[s+1]) is what source rank s sends (each source
    owns its own Placement counters, ep.py:27-33); g2l (E,) global -> local
    expert id or -1 (ep.py:203-208).

    Per source segment: flatten (ep.py:211-213), route_counts (ep.py:216-217),
    dest_ranks (ep.py:219), stable sort by destination (ep.py:220) keeping the
    part for ``my_rank``; receive order is by source (all_to_all splits,
    ep.py:225-226); g2l + residency check (ep.py:229-230); run_experts then
    stable-sorts by local expert (modeling.py:94-96).

    Returns dict with counts (n_local,), offsets (n_local+1,), perm (M,) =
    flat entry id t*k+s of each row in local expert order, row_of_entry (N*k,)
    (-1 if not here), dest (N*k,) (-1 for dropped entries), route_counts (E,),
    rr_after (S,E), not_resident (bool).
    """
    topk_idx = np.asarray(topk_idx, np.int64)
    n, k = topk_idx.shape
    g2l = np.asarray(g2l, np.int64)
    n_local = int((g2l >= 0).sum())
    rr = np.array(rr, np.int64, copy=True).reshape(len(seg_tokens) - 1, n_experts)
    valid = np.ones(n, bool) if valid_mask is None else np.asarray(valid_mask, bool)
    dest_all = np.full(n * k, -1, np.int64)
    route_counts = np.zeros(n_experts, np.int64)
    recv_entries, recv_experts = [], []
    for s in range(len(seg_tokens) - 1):
        t0, t1 = int(seg_tokens[s]), int(seg_tokens[s + 1])
        tok, slot, keep_e = flatten_topk(t1 - t0, k, valid[t0:t1])
        flat_e = topk_idx[t0:t1].reshape(-1)[keep_e]
        fid = (tok + t0) * k + slot                      # global flat entry id
        route_counts += np.bincount(flat_e, minlength=n_experts)
        dest, rr[s] = dest_ranks(table, n_rep, rr[s], flat_e)
        dest_all[fid] = dest
        order = np.argsort(dest, kind="stable")
        mine = order[dest[order] == my_rank]
        recv_entries.append(fid[mine])
        recv_experts.append(flat_e[mine])
    recv_entries = np.concatenate(recv_entries) if recv_entries else np.zeros(0, np.int64)
    recv_experts = np.concatenate(recv_experts) if recv_experts else np.zeros(0, np.int64)
    local = g2l[recv_experts]
    not_resident = bool((local < 0).any())
    keep = local >= 0
    recv_entries, local = recv_entries[keep], local[keep]
    order, counts = stable_expert_order(local, n_local)
    perm = recv_entries[order]
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    row_of_entry = np.full(n * k, -1, np.int64)
    row_of_entry[perm] = np.arange(perm.size, dtype=np.int64)
    return dict(counts=counts, offsets=offsets, perm=perm, row_of_entry=row_of_entry,
                dest=dest_all, route_counts=route_counts, rr_after=rr,
                not_resident=not_resident)


# ----------------------------------------------------------------------------
# a6/a7: gathered rows through the SwiGLU experts  (modeling.py:83-104)
# ----------------------------------------------------------------------------
def experts(x_rows, local_expert_of_row, w_in, w_out, act_bf16=False, out_bf16=False):
    """run_experts (modeling.py:83-104) in float32 (numpy sgemm):
    h = X_e @ W_in[e].T; gate, up = h[:, :I], h[:, I:]; y = (silu(gate)*up) @ W_out[e].T.
    ``act_bf16``/``out_bf16`` round the activation / output to bf16 where a bf16
    model stores them.  Output keeps input row order."""
    x_rows = np.asarray(x_rows, np.float32)
    ids = np.asarray(local_expert_of_row, np.int64)
    inter = w_in.shape[1] // 2
    out = np.zeros((x_rows.shape[0], w_out.shape[1]), np.float32)
    for e in np.unique(ids):
        rows = np.nonzero(ids == e)[0]
        h = x_rows[rows] @ np.asarray(w_in[e], np.float32).T
        a = (silu(h[:, :inter]) * h[:, inter:]).astype(np.float32)
        if act_bf16:
            a = bf16_round(a)
        y = a @ np.asarray(w_out[e], np.float32).T
        out[rows] = bf16_round(y) if out_bf16 else y
    return out


# ----------------------------------------------------------------------------
# a8/a9: gate weighting + slot-order combine  (modeling.py:120-128, :144)
# ----------------------------------------------------------------------------
def combine(y_entries, topk_gate, present, n, k):
    """out[t] = sum_s gate[t,s] * y[t*k+s] over present entries, slot order
    (modeling.py:144 gates, :126-128 unique-cell scatter then sum over the slot
    axis).  y_entries: (n*k, H) in flat entry order; present: (n*k,) bool."""
    y = np.asarray(y_entries, np.float32).reshape(n, k, -1)
    g = np.asarray(topk_gate, np.float32).reshape(n, k) * np.asarray(present, bool).reshape(n, k)
    return (y * g[:, :, None]).sum(axis=1, dtype=np.float32).astype(np.float32)


def moe_layer_local(x, topk_idx, topk_gate, w_in, w_out, valid_mask=None,
                    act_bf16=False, out_bf16=False):
    """LocalMoEBackend.__call__ (modeling.py:138-145): flatten, gather rows,
    run_experts, gate, scatter_combine.  Returns (N, H) float32."""
    x = np.asarray(x, np.float32)
    n, k = topk_idx.shape
    tok, slot, keep_e = flatten_topk(n, k, valid_mask)
    ids = np.asarray(topk_idx, np.int64).reshape(-1)[keep_e]
    ys = experts(x[tok], ids, w_in, w_out, act_bf16=act_bf16, out_bf16=out_bf16)
    y_entries = np.zeros((n * k, w_out.shape[1]), np.float32)
    y_entries[tok * k + slot] = ys
    return combine(y_entries, topk_gate, keep_e, n, k)
