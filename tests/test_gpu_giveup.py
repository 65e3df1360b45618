"""The bounded waits of the one-launch kernels, driven to give up from the host.

Four kernels wait on other workgroups of the same launch: the fused router +
dispatch and the one-launch dispatch (each workgroup waits for every other's
per-expert counts), the tiled experts launch (a GEMM-2 tile waits for its row
tile's GEMM-1 counts), the small-batch experts launch (GEMM-2 workgroups wait
for their chunk's GEMM-1 counts) and the small-batch launch that ends with the
combine (combine workgroups wait for every GEMM-2 workgroup).  A wait that
gives up must not be silent: ``mep_test_force_giveup`` makes one wait of each
kind give up after a few polls, and every case asserts that

  * every kernel exits (the calls return and the stream synchronises),
  * the give-up is reported (mep_dispatch_check / mep_experts_check),
  * what the caller consumes is poisoned (row_of_entry -2 and offsets[-1] -1
    for a dispatch, NaN for the expert rows or outputs that depended on the
    wait), and the rest equals the normal call's bits,
  * the workspace words return to zero, and
  * the next call on the same workspace gives the normal call's bits.

The reference fails loudly rather than silently (ep.py:230 asserts); these
waits have no counterpart there (its dispatch is a host-synchronised torch
sequence).
"""
import contextlib

import numpy as np
import pytest
import torch

from helpers import banner
from miniep_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
POLLS = 2000
HEADER_BYTES = 512 + 64 * 128                                 # dispatch workspace header: 4 lines + 64 group lines


@contextlib.contextmanager
def force_giveup(site):
    L = _lib.lib()
    _lib.check(L.mep_test_force_giveup(site, POLLS), "mep_test_force_giveup")
    try:
        yield
    finally:
        _lib.check(L.mep_test_force_giveup(_lib.GIVEUP_NONE, 0), "mep_test_force_giveup")


def _world1(E):
    return (torch.zeros(E, 1, dtype=torch.int32, device=DEV), torch.ones(E, dtype=torch.int32, device=DEV),
            torch.arange(E, dtype=torch.int32, device=DEV))


def _dispatch_ws():
    dev = torch.device(DEV, torch.cuda.current_device())
    return ops._DISPATCH_WS[(dev.index, ops._stream(dev))]


def _queue_words_zero():
    for q in ops._QUEUES.values():
        assert int(q.abs().sum()) == 0


def _raises_hip(fn, what):
    with pytest.raises(_lib.MepError) as ei:
        fn()
    assert ei.value.code == _lib.ERR_HIP, ei.value
    assert what in ei.value.message, ei.value.message


def test_route_dispatch_giveup():
    """Fused router + dispatch (64 workgroups): the last workgroup withholds
    its counts, every workgroup gives up, the call is poisoned; the experts
    launch on that dispatch runs no tile and is flagged, the combine gives NaN;
    the header words return to zero and the next call is exact."""
    banner("give-up: route_dispatch (T=4096)")
    bf = torch.bfloat16
    L = workloads.make_layer(4096, seed=31, zipf_s=1.2)
    x, w = L.x.to(bf).to(DEV), L.w_router.to(bf).to(DEV)
    wi, wo = L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
    idx0, gate0, d0 = ops.route_dispatch(x, w, 8, check=True)
    out0 = ops.grouped_swiglu_combine(x, d0, wi, wo, gate0)
    ops.experts_check()
    ws = _dispatch_ws()
    words = ws[:512].view(torch.int32)
    epoch = int(words[32])
    with force_giveup(_lib.GIVEUP_DISPATCH):
        idx1, gate1, d1 = ops.route_dispatch(x, w, 8, check=False)
        torch.cuda.synchronize()
    _raises_hip(lambda: _lib.check(_lib.lib().mep_dispatch_check(ws.data_ptr(), ops._stream(x.device)),
                                   "mep_route_dispatch"), "gave up")
    assert int(d1.offsets[-1]) == -1
    assert bool((d1.row_of_entry == -2).all())
    assert int(words[64]) == 0 and int(words[96]) == 0      # finished-group counter, give-up word
    assert int(ws[512:HEADER_BYTES].view(torch.int32).abs().sum()) == 0   # per-group finished counters
    assert int(words[32]) == epoch + 1                      # advanced once, by the last workgroup
    assert torch.equal(idx1, idx0) and torch.equal(gate1, gate0)   # the router part is unaffected
    # downstream: no tile runs on the poisoned offsets, every output is NaN
    out1 = ops.grouped_swiglu_combine(x, d1, wi, wo, gate1)
    _raises_hip(ops.experts_check, "dispatch gave up")
    assert bool(torch.isnan(out1.float()).all())
    _queue_words_zero()
    # the same workspace and queue serve the next call exactly
    idx2, gate2, d2 = ops.route_dispatch(x, w, 8, check=True)
    out2 = ops.grouped_swiglu_combine(x, d2, wi, wo, gate2)
    ops.experts_check()
    assert torch.equal(d2.offsets, d0.offsets) and torch.equal(d2.perm, d0.perm)
    assert torch.equal(d2.row_of_entry, d0.row_of_entry)
    assert torch.equal(out2, out0)
    assert int(words[32]) == epoch + 2


def test_dispatch_giveup_ep_share():
    """One-launch dispatch of a rank share (4 source segments, replicas, 128
    blocks): every block gives up, the call is poisoned, the round-robin
    counters are left as they were; the next call equals the normal one."""
    banner("give-up: one-launch dispatch, rank share with replicas")
    g = torch.Generator().manual_seed(32)
    E, k, n, world = 32, 8, 8192, 4
    topk = torch.rand(n, E, generator=g).topk(k, -1).indices.to(DEV)
    table = torch.tensor([[e // 8, (e // 8 + 1) % world] for e in range(E)], dtype=torch.int32, device=DEV)
    n_rep = torch.tensor([2 if e % 3 == 0 else 1 for e in range(E)], dtype=torch.int32, device=DEV)
    mine = [e for e in range(E) if 1 in table[e, : int(n_rep[e])].tolist()]
    g2l = torch.full((E,), -1, dtype=torch.int32)
    for j, e in enumerate(mine):
        g2l[e] = j
    g2l = g2l.to(DEV)
    seg = [0, 2048, 4096, 6144, 8192]
    rr_init = torch.randint(0, 5, (4, E), generator=g).to(DEV)

    def run(check):
        rr = rr_init.clone()
        d = ops.dispatch(topk, None, E, table, n_rep, True, rr, 1, g2l, len(mine), seg_tokens=seg,
                         want_dest=True, check=check)
        return d, rr

    d0, rr0 = run(True)
    ws = _dispatch_ws()
    words = ws[:512].view(torch.int32)
    with force_giveup(_lib.GIVEUP_DISPATCH):
        d1, rr1 = run(False)
        torch.cuda.synchronize()
    _raises_hip(lambda: _lib.check(_lib.lib().mep_dispatch_check(ws.data_ptr(), ops._stream(topk.device)),
                                   "mep_dispatch"), "gave up")
    assert int(d1.offsets[-1]) == -1
    assert bool((d1.row_of_entry[: n * k] == -2).all())
    assert torch.equal(rr1, rr_init)                          # no block applied the counter update
    assert int(words[64]) == 0 and int(words[96]) == 0
    assert int(ws[512:HEADER_BYTES].view(torch.int32).abs().sum()) == 0
    d2, rr2 = run(True)
    assert torch.equal(d2.offsets, d0.offsets) and torch.equal(d2.counts, d0.counts)
    m = int(d0.offsets[-1])
    assert torch.equal(d2.perm[:m], d0.perm[:m]) and torch.equal(d2.row_of_entry, d0.row_of_entry)
    assert torch.equal(d2.dest, d0.dest) and torch.equal(rr2, rr0)


def _first_rows(d, rows_per_unit):
    """Rows of the first row tile / chunk: the first expert with rows."""
    counts = d.counts.cpu().numpy()
    e0 = int(np.nonzero(counts)[0][0])
    return np.arange(min(rows_per_unit, int(counts[e0])))    # offsets[e0] == 0


def _cells(d, rows):
    return d.perm.cpu().numpy()[rows]


@pytest.mark.parametrize("case", ["tiled_t4096", "small_t32"])
def test_experts_giveup(case):
    """A GEMM-2 wait that gives up (the tiled launch: row tile 0's four GEMM-2
    tiles; the small-batch launch: chunk 0's GEMM-2 workgroups) writes NaN
    into exactly those rows' (token, slot) cells, is flagged, leaves the
    schedule words at zero, and the next call gives the normal bits."""
    banner(f"give-up: experts GEMM-2 wait ({case})")
    bf = torch.bfloat16
    n = int(case.split("_t")[1])
    L = workloads.make_layer(n, seed=33, zipf_s=1.2)
    topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices.to(DEV)
    E = L.w_in.shape[0]
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(topk, None, E, table, n_rep, False, None, 0, g2l, E)
    x, wi, wo = L.x.to(bf).to(DEV), L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
    y0 = torch.full((n * 8, 1024), 7.0, dtype=bf, device=DEV)
    ops.grouped_swiglu(x, d, wi, wo, y0)
    ops.experts_check()
    site, unit = (_lib.GIVEUP_ROWS, 256) if case.startswith("tiled") else (_lib.GIVEUP_CHUNK, 32)
    y1 = torch.full_like(y0, 7.0)
    with force_giveup(site):
        ops.grouped_swiglu(x, d, wi, wo, y1)
        torch.cuda.synchronize()
    _raises_hip(ops.experts_check, "gave up waiting")
    cells = _cells(d, _first_rows(d, unit))
    assert len(cells) > 0
    bad = np.zeros(n * 8, bool)
    bad[cells] = True
    bad_t = torch.from_numpy(bad).to(DEV)
    assert bool(torch.isnan(y1[bad_t].float()).all())
    assert torch.equal(y1[~bad_t], y0[~bad_t])
    _queue_words_zero()
    y2 = torch.full_like(y0, 7.0)
    ops.grouped_swiglu(x, d, wi, wo, y2)
    ops.experts_check()
    assert torch.equal(y2, y0)
    _queue_words_zero()


def test_small_batch_combine_giveup():
    """The small-batch launch that ends with the combine: combine workgroup 0
    gives up waiting for GEMM-2, its tokens' outputs (tokens 0 and 1 at hidden
    1024) are NaN, the others are exact; flagged, words back to zero, and the
    next call is exact."""
    banner("give-up: small-batch combine wait")
    bf = torch.bfloat16
    n = 32
    L = workloads.make_layer(n, seed=34)
    x, w = L.x.to(bf).to(DEV), L.w_router.to(bf).to(DEV)
    wi, wo = L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
    idx, gate, d = ops.route_dispatch(x, w, 8, check=True)
    out0 = ops.grouped_swiglu_combine(x, d, wi, wo, gate)
    ops.experts_check()
    with force_giveup(_lib.GIVEUP_COMBINE):
        out1 = ops.grouped_swiglu_combine(x, d, wi, wo, gate)
        torch.cuda.synchronize()
    _raises_hip(ops.experts_check, "gave up waiting")
    per_wg = 256 // (1024 // 8)                               # tokens of one combine workgroup
    assert bool(torch.isnan(out1[:per_wg].float()).all())
    assert torch.equal(out1[per_wg:], out0[per_wg:])
    _queue_words_zero()
    out2 = ops.grouped_swiglu_combine(x, d, wi, wo, gate)
    ops.experts_check()
    assert torch.equal(out2, out0)
    _queue_words_zero()


def test_giveup_hook_rejects_bad_arguments():
    L = _lib.lib()
    assert L.mep_test_force_giveup(9, 10) == _lib.ERR_INVALID_ARG
    assert L.mep_test_force_giveup(_lib.GIVEUP_ROWS, 0) == _lib.ERR_INVALID_ARG
    assert L.mep_test_force_giveup(_lib.GIVEUP_NONE, 0) == 0
