"""The raw C ABI through ctypes, exactly as a binding would call it (no
miniep_amd wrapper): must give the same bits as the HipMoEBackend path."""
import ctypes

import pytest
import torch

from helpers import banner
from miniep_amd import HipMoEBackend, _lib, ops, route, workloads

pytestmark = pytest.mark.gpu


def _moe_layer_raw(L, x, w_r, w_in, w_out, k=8, one_call=False):
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    N, H = x.shape
    E = w_r.shape[0]
    I = w_out.shape[2]
    BF16 = 1
    s = torch.cuda.current_stream().cuda_stream

    def ok(rc):
        if rc != 0:
            raise RuntimeError(L.mep_last_error().decode())

    idx = torch.empty(N, k, dtype=torch.int64, device="cuda")
    gate = torch.empty(N, k, dtype=x.dtype, device="cuda")
    ok(L.mep_router_topk(x.data_ptr(), w_r.data_ptr(), N, H, E, k, BF16, idx.data_ptr(), gate.data_ptr(),
                         None, s))
    seg = (i64 * 2)(0, N)
    ws = torch.zeros(L.mep_dispatch_workspace_size(N, k, E, 1, seg), dtype=torch.uint8, device="cuda")
    table = torch.zeros(E, 1, dtype=torch.int32, device="cuda")
    n_rep = torch.ones(E, dtype=torch.int32, device="cuda")
    g2l = torch.arange(E, dtype=torch.int32, device="cuda")
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(N * k, dtype=torch.int32, device="cuda")
    row = torch.empty(N * k, dtype=torch.int32, device="cuda")
    ok(L.mep_dispatch(idx.data_ptr(), None, N, k, E, table.data_ptr(), n_rep.data_ptr(), 1, 0, None, seg, 1, 0,
                      g2l.data_ptr(), E, counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(), row.data_ptr(),
                      None, None, ws.data_ptr(), ws.numel(), s))
    ok(L.mep_dispatch_check(ws.data_ptr(), s))
    act = torch.empty(L.mep_experts_workspace_size(N * k, I, BF16), dtype=torch.uint8, device="cuda")
    y = torch.empty(N * k, H, dtype=x.dtype, device="cuda")
    queue = torch.zeros(L.mep_experts_queue_ints(N * k, E), dtype=torch.int32, device="cuda")
    out = torch.empty(N, H, dtype=x.dtype, device="cuda")
    if one_call:
        ok(L.mep_grouped_swiglu_combine(x.data_ptr(), N, k, perm.data_ptr(), offsets.data_ptr(), row.data_ptr(),
                                        gate.data_ptr(), None, E, N * k, w_in.data_ptr(), w_out.data_ptr(), H, I,
                                        BF16, y.data_ptr(), act.data_ptr(), act.numel(), queue.data_ptr(),
                                        queue.numel(), out.data_ptr(), s))
    else:
        ok(L.mep_grouped_swiglu(x.data_ptr(), N, k, perm.data_ptr(), offsets.data_ptr(), E, N * k,
                                w_in.data_ptr(), w_out.data_ptr(), H, I, BF16, y.data_ptr(), act.data_ptr(),
                                act.numel(), queue.data_ptr(), queue.numel(), s))
    ok(L.mep_experts_check(queue.data_ptr(), s))
    assert int(queue.abs().sum()) == 0                   # every launch leaves the schedule words at zero
    if not one_call:
        ok(L.mep_combine(y.data_ptr(), gate.data_ptr(), row.data_ptr(), None, N, k, H, BF16, out.data_ptr(), s))
    return out, idx, gate


@pytest.mark.parametrize("n", [2048, 32])
def test_raw_ctypes_layer_matches_backend(n):
    """2048 tokens: the tiled experts launch; 32 tokens: the small-batch
    launch, which mep_grouped_swiglu_combine ends with the combine.  The raw
    calls (experts + combine as two calls, and as one) give the backend's
    bits."""
    banner(f"raw C ABI layer, {n} tokens")
    L = _lib.lib()          # signatures are registered by the loader
    layer = workloads.make_layer(n, seed=9, zipf_s=1.2 if n > 1000 else 0.0)
    bf = torch.bfloat16
    x = layer.x.to(bf).cuda()
    w_r = layer.w_router.to(bf).cuda()
    w_in = layer.w_in.to(bf).cuda()
    w_out = layer.w_out.to(bf).cuda()
    out, idx, gate = _moe_layer_raw(L, x, w_r, w_in, w_out)
    out1, _, _ = _moe_layer_raw(L, x, w_r, w_in, w_out, one_call=True)
    idx2, gate2 = route(x, w_r, 8)
    ref = HipMoEBackend(w_in, w_out)(x, idx2, gate2)
    assert torch.equal(idx, idx2) and torch.equal(gate, gate2)
    assert torch.equal(out, ref) and torch.equal(out1, ref)


class _RawBlock:
    """The whole block through the raw C ABI (mep_moe_layer), with argtypes
    of its own on a separate handle of the library, as a binding would
    declare them; the dispatch workspace grows (zero-filled) with the batch
    and the schedule buffer is kept per size, left zero by every call."""

    def __init__(self):
        vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
        L = ctypes.CDLL(_lib.lib()._name)
        L.mep_last_error.restype = ctypes.c_char_p
        L.mep_route_dispatch_workspace_size.restype = sz
        L.mep_route_dispatch_workspace_size.argtypes = [i64, i32]
        L.mep_moe_layer_queue_ints.restype = sz
        L.mep_moe_layer_queue_ints.argtypes = [i64, i32, i32]
        L.mep_experts_workspace_size.restype = sz
        L.mep_experts_workspace_size.argtypes = [i64, i32, i32]
        L.mep_moe_layer.restype = ctypes.c_int
        L.mep_moe_layer.argtypes = [vp, vp, vp, i64, i32, i32, i32, i32, vp, vp, i32, vp, vp, vp,
                                    vp, vp, vp, vp, vp, vp, vp, sz, vp, sz, vp, sz, vp, vp]
        self.L, self.dws, self.queues = L, None, {}

    def __call__(self, x, w_r, w_in, w_out, k=8):
        L = self.L
        N, H = x.shape
        E, I = w_r.shape[0], w_out.shape[2]
        s = torch.cuda.current_stream().cuda_stream
        e = lambda *shape, dt=torch.int32: torch.empty(*shape, dtype=dt, device="cuda")
        idx, gate = e(N, k, dt=torch.int64), e(N, k, dt=x.dtype)
        counts, offsets, perm, row = e(E), e(E + 1), e(N * k), e(N * k)
        y, out = e(N * k, H, dt=x.dtype), e(N, H, dt=x.dtype)
        need = L.mep_route_dispatch_workspace_size(N, E)
        if self.dws is None or self.dws.numel() < need:
            self.dws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        act = e(L.mep_experts_workspace_size(N * k, I, 1), dt=torch.uint8)
        nq = L.mep_moe_layer_queue_ints(N, E, H)
        queue = self.queues.setdefault(nq, torch.zeros(nq, dtype=torch.int32, device="cuda"))
        rc = L.mep_moe_layer(x.data_ptr(), w_r.data_ptr(), None, N, H, E, k, 1, w_in.data_ptr(), w_out.data_ptr(), I,
                             idx.data_ptr(), gate.data_ptr(), None, counts.data_ptr(), offsets.data_ptr(),
                             perm.data_ptr(), row.data_ptr(), None, y.data_ptr(), self.dws.data_ptr(),
                             self.dws.numel(), act.data_ptr(), act.numel(), queue.data_ptr(), queue.numel(),
                             out.data_ptr(), s)
        if rc != 0:
            raise RuntimeError(L.mep_last_error().decode())
        torch.cuda.synchronize()
        assert int(queue.abs().sum()) == 0
        return out, idx, gate


def test_raw_ctypes_moe_block_matches_ops():
    """mep_moe_layer through raw ctypes at 32 tokens (one launch), then 7
    (one launch), then 100 (router + dispatch, then the experts launch; the
    dispatch workspace grows): each the bits of ops.moe_layer."""
    raw = _RawBlock()
    bf = torch.bfloat16
    for n in (32, 7, 100):
        banner(f"raw C ABI block (mep_moe_layer), {n} tokens")
        layer = workloads.make_layer(n, seed=11 + n)
        x, w_r, w_in, w_out = (t.to(bf).cuda() for t in (layer.x, layer.w_router, layer.w_in, layer.w_out))
        out, idx, gate = raw(x, w_r, w_in, w_out)
        ref, idx2, gate2, _ = ops.moe_layer(x, w_r, 8, w_in, w_out)
        ops.experts_check()
        assert torch.equal(idx, idx2) and torch.equal(gate, gate2)
        assert torch.equal(out, ref)


def test_error_codes_and_messages():
    banner("C ABI errors")
    L = _lib.lib()
    x = torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda")
    rc = L.mep_router_topk(x.data_ptr(), x.data_ptr(), 4, 1000, 32, 8, 1, x.data_ptr(), x.data_ptr(), None, None)
    assert rc == _lib.ERR_UNSUPPORTED and b"multiple of 256" in L.mep_last_error()
    rc = L.mep_router_topk(x.data_ptr(), x.data_ptr(), 4, 1024, 32, 8, 7, x.data_ptr(), x.data_ptr(), None, None)
    assert rc == _lib.ERR_INVALID_ARG
    rc = L.mep_combine(None, None, None, None, 4, 8, 1024, 1, None, None)
    assert rc == _lib.ERR_INVALID_ARG
    rc = L.mep_grouped_swiglu(x.data_ptr(), 4, 8, x.data_ptr(), x.data_ptr(), 4, 32, x.data_ptr(), x.data_ptr(),
                              1024, 512, 1, x.data_ptr(), x.data_ptr(), 16, x.data_ptr(), 64, None)
    assert rc == _lib.ERR_WORKSPACE
    # a tiled launch needs mep_experts_queue_ints words of schedule (checked before anything is enqueued)
    big = torch.zeros(9 << 20, dtype=torch.int32, device="cuda")     # 36 MiB: covers act of 32768 rows
    need = L.mep_experts_queue_ints(4096 * 8, 32)
    assert need == (16 + 4096 * 8 // 256 + 32) * 32      # one 128-byte line per counter
    rc = L.mep_grouped_swiglu(big.data_ptr(), 4096, 8, big.data_ptr(), big.data_ptr(), 32, 4096 * 8, big.data_ptr(),
                              big.data_ptr(), 1024, 512, 1, big.data_ptr(), big.data_ptr(), big.numel() * 4,
                              big.data_ptr(), need - 1, None)
    assert rc == _lib.ERR_WORKSPACE and b"tile_queue" in L.mep_last_error()
    rc = L.mep_grouped_swiglu(big.data_ptr(), 4096, 8, big.data_ptr(), big.data_ptr(), 32, 4096 * 8, big.data_ptr(),
                              big.data_ptr(), 1024, 512, 1, big.data_ptr(), big.data_ptr(), big.numel() * 4,
                              None, need, None)
    assert rc == _lib.ERR_INVALID_ARG
    assert L.mep_abi_version() == 5
