"""mep_dispatch_noalloc (the allocation-free form of mep_dispatch, workspace
in a static device array) against mep_dispatch through the raw C ABI: the
same outputs bit for bit on two calls in a row, the second with a smaller
input, on a replicated multi-source share and on a world-1 batch, and the
status word against mep_dispatch_check."""
import ctypes
import json

import pytest
import torch

from helpers import banner
from miniep_amd import Placement, _lib, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outputs(n, k, n_local, E):
    i32 = dict(dtype=torch.int32, device=DEV)
    return dict(counts=torch.full((max(n_local, 1),), -7, **i32), offsets=torch.full((n_local + 1,), -7, **i32),
                perm=torch.full((n * k,), -7, **i32), row=torch.full((n * k,), -7, **i32),
                dest=torch.full((n * k,), -7, **i32),
                route_counts=torch.arange(E, dtype=torch.int64, device=DEV))


def _call(L, noalloc, idx, table, n_rep, has_rep, rr, seg, my_rank, g2l, n_local, out, status=None):
    n, k = idx.shape
    E = table.shape[0]
    segs = (ctypes.c_int64 * len(seg))(*seg)
    s = torch.cuda.current_stream().cuda_stream
    common = (idx.data_ptr(), None, n, k, E, table.data_ptr(), n_rep.data_ptr(), table.shape[1], int(has_rep),
              None if rr is None else rr.data_ptr(), segs, len(seg) - 1, my_rank, g2l.data_ptr(), n_local,
              out["counts"].data_ptr(), out["offsets"].data_ptr(), out["perm"].data_ptr(), out["row"].data_ptr(),
              out["dest"].data_ptr(), out["route_counts"].data_ptr())
    if noalloc:
        rc = L.mep_dispatch_noalloc(*common, None if status is None else status.data_ptr(), s)
        assert rc == 0, L.mep_last_error()
        return None
    ws = torch.zeros(L.mep_dispatch_workspace_size(n, k, E, len(seg) - 1, segs), dtype=torch.uint8, device=DEV)
    rc = L.mep_dispatch(*common, ws.data_ptr(), ws.numel(), s)
    assert rc == 0, L.mep_last_error()
    return ws


def _same(a, b, M, nk):
    assert torch.equal(a["counts"], b["counts"]) and torch.equal(a["offsets"], b["offsets"])
    assert torch.equal(a["perm"][:M], b["perm"][:M])
    assert torch.equal(a["row"][:nk], b["row"][:nk]) and torch.equal(a["dest"][:nk], b["dest"][:nk])
    assert torch.equal(a["route_counts"], b["route_counts"])


def test_noalloc_matches_dispatch_on_consecutive_calls(golden_dir):
    banner("mep_dispatch_noalloc vs mep_dispatch")
    L = _lib.lib()
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    table, n_rep = p.tables(2, DEV)
    E = 32
    for r in (1, 3):                                       # two ranks' shares, consecutive calls
        ids = p.experts_of_rank(r)[2]
        g2l = torch.full((E,), -1, dtype=torch.int32, device=DEV)
        g2l[torch.tensor(ids)] = torch.arange(len(ids), dtype=torch.int32, device=DEV)
        for T, seed in ((8192, 5), (3000, 6)):              # the second call is smaller
            lay = workloads.make_layer(T, seed=seed, zipf_s=1.1)
            idx = lay.x.to(DEV) @ lay.w_router.to(DEV).T
            idx = idx.topk(8, dim=-1).indices.contiguous()
            seg = [T * s // 4 for s in range(5)]
            rr0 = torch.randint(0, 5, (4, E), generator=torch.Generator().manual_seed(T), dtype=torch.int64).to(DEV)
            a, b = _outputs(T, 8, len(ids), E), _outputs(T, 8, len(ids), E)
            rr_a, rr_b = rr0.clone(), rr0.clone()
            status = torch.full((1,), 0xFF, dtype=torch.int32, device=DEV)
            ws = _call(L, False, idx, table, n_rep, True, rr_a, seg, r, g2l, len(ids), a)
            _call(L, True, idx, table, n_rep, True, rr_b, seg, r, g2l, len(ids), b, status)
            torch.cuda.synchronize()
            M = int(a["offsets"][-1])
            _same(a, b, M, T * 8)
            assert torch.equal(rr_a, rr_b)
            assert int(status.item()) == 0 and L.mep_dispatch_check(ws.data_ptr(), None) == 0
    # world 1 (LocalMoEBackend) after the shares: the scratch keeps the last call's data
    for T in (16384, 700):
        lay = workloads.make_layer(T, seed=T, zipf_s=1.2)
        idx = (lay.x.to(DEV) @ lay.w_router.to(DEV).T).topk(8, dim=-1).indices.contiguous()
        t1 = torch.zeros(E, 1, dtype=torch.int32, device=DEV)
        r1 = torch.ones(E, dtype=torch.int32, device=DEV)
        ident = torch.arange(E, dtype=torch.int32, device=DEV)
        a, b = _outputs(T, 8, E, E), _outputs(T, 8, E, E)
        _call(L, False, idx, t1, r1, False, None, [0, T], 0, ident, E, a)
        _call(L, True, idx, t1, r1, False, None, [0, T], 0, ident, E, b)
        torch.cuda.synchronize()
        _same(a, b, T * 8, T * 8)


def test_noalloc_status_reports_dropped_entries():
    banner("mep_dispatch_noalloc status")
    L = _lib.lib()
    E, n, k = 32, 600, 8
    idx = torch.randint(0, E, (n, k), generator=torch.Generator().manual_seed(2)).to(DEV)
    idx[5, 3] = E + 4                                      # out of range
    t1 = torch.zeros(E, 1, dtype=torch.int32, device=DEV)
    r1 = torch.ones(E, dtype=torch.int32, device=DEV)
    g2l = torch.arange(E, dtype=torch.int32, device=DEV)
    g2l[7] = -1                                            # expert 7 not resident here
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = _outputs(n, k, E, E)
    _call(L, True, idx, t1, r1, False, None, [0, n], 0, g2l, E, out, status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.DISPATCH_STATUS_RANGE | _lib.DISPATCH_STATUS_NOT_RESIDENT
    # the next call on clean input clears it
    idx[5, 3] = 0
    g2l[7] = 7
    _call(L, True, idx, t1, r1, False, None, [0, n], 0, g2l, E, out, status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
