"""Tensor-level wrappers of the HIP kernels (device tensors in, device tensors out).

Every function here enqueues work on torch's current HIP stream through the
C ABI and returns without synchronising (except ``dispatch(check=True)``,
which mirrors the residency assert of miniep/ep.py:230).  There is no CPU
path: CPU tensors are rejected.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; the kernels take float32 or bfloat16") from None


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("the MoE kernels run on the GPU only; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


_QUEUES: dict[tuple[int, int], torch.Tensor] = {}
_DISPATCH_WS: dict[tuple[int, int], torch.Tensor] = {}


def _tile_queue(dev: torch.device, max_rows: int, n_local: int) -> torch.Tensor:
    """Schedule buffer of the tiled grouped GEMMs for the current stream of
    ``dev`` (mep_experts_queue_ints words): zeroed here, left at zero by
    every launch (but for its sticky error word, see ``experts_check``), one
    per stream so that launches on different streams never share it, and
    replaced by a larger zeroed one when a launch needs more words."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    need = int(_lib.lib().mep_experts_queue_ints(max_rows, n_local))
    q = _QUEUES.get(key)
    if q is None or q.numel() < need:
        q = _QUEUES[key] = torch.zeros(max(need, 64), dtype=torch.int32, device=dev)
    return q


def _dispatch_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Workspace of mep_dispatch / mep_route_dispatch for the current stream
    of ``dev``: zero-filled once here (the one-launch kernels keep the epoch
    that tags the per-block counts they exchange in it), then reused as is by
    every call on that stream, one per stream so that calls on different
    streams never share it, and replaced by a larger zeroed one when a call
    needs more bytes."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    ws = _DISPATCH_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = _DISPATCH_WS[key] = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
    return ws


def dispatch_check(dev: torch.device | None = None) -> None:
    """Synchronise and raise MepError if the last dispatch on the current
    stream of ``dev`` (its workspace) dropped entries or gave up waiting."""
    dev = dev or torch.device("cuda", torch.cuda.current_device())
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    ws = _DISPATCH_WS.get(key)
    if ws is not None:
        _lib.check(_lib.lib().mep_dispatch_check(ws.data_ptr(), _stream(dev)), "mep_dispatch_check")


def experts_check(dev: torch.device | None = None) -> None:
    """Synchronise and raise MepError if a grouped-GEMM launch on the current
    stream of ``dev`` flagged its results invalid (a GEMM-2 tile that gave
    up waiting for its GEMM-1 rows, or a tile queue nobody drained)."""
    dev = dev or torch.device("cuda", torch.cuda.current_device())
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    q = _QUEUES.get(key)
    if q is not None:
        _lib.check(_lib.lib().mep_experts_check(q.data_ptr(), _stream(dev)), "mep_experts_check")


def _mask_u8(valid_mask: torch.Tensor | None, n: int) -> torch.Tensor | None:
    if valid_mask is None:
        return None
    vm = valid_mask.reshape(-1)
    if vm.numel() != n:
        raise ValueError(f"valid_mask has {vm.numel()} entries, expected {n}")
    return vm.to(torch.uint8).contiguous()


# ----------------------------------------------------------------------------
# router (modeling.py:192-195)
# ----------------------------------------------------------------------------
def router_topk(x_flat: torch.Tensor, w_router: torch.Tensor, k: int, return_logits: bool = False):
    """topk_idx (N,k) int64, topk_gate (N,k) x.dtype [, logits (N,E) fp32].

    logits = x_flat @ w_router.T accumulated in fp32; topk descending with
    equal logits resolved to the lower expert id; gate = fp32 softmax of the
    k selected logits stored in x.dtype (modeling.py:193-195)."""
    dev = _require_device(x_flat, w_router)
    x = x_flat.contiguous()
    w = w_router.to(x.dtype).contiguous()
    n, h = x.shape
    e = w.shape[0]
    if w.shape[1] != h:
        raise ValueError(f"router weight {tuple(w.shape)} does not match hidden {h}")
    idx = torch.empty((n, k), dtype=torch.int64, device=dev)
    gate = torch.empty((n, k), dtype=x.dtype, device=dev)
    logits = torch.empty((n, e), dtype=torch.float32, device=dev) if return_logits else None
    rc = _lib.lib().mep_router_topk(x.data_ptr(), w.data_ptr(), n, h, e, k, _dtype_code(x),
                                    idx.data_ptr(), gate.data_ptr(), _ptr(logits), _stream(dev))
    _lib.check(rc, "mep_router_topk")
    return (idx, gate, logits) if return_logits else (idx, gate)


def topk_softmax(logits: torch.Tensor, k: int, gate_dtype: torch.dtype = torch.float32):
    """Top-k + fp32 softmax of precomputed fp32 logits (modeling.py:194-195)."""
    dev = _require_device(logits)
    lg = logits.to(torch.float32).contiguous()
    n, e = lg.shape
    idx = torch.empty((n, k), dtype=torch.int64, device=dev)
    gate = torch.empty((n, k), dtype=gate_dtype, device=dev)
    code = _DTYPES[gate_dtype]
    rc = _lib.lib().mep_topk_softmax(lg.data_ptr(), n, e, k, code, idx.data_ptr(), gate.data_ptr(),
                                     _stream(dev))
    _lib.check(rc, "mep_topk_softmax")
    return idx, gate


# ----------------------------------------------------------------------------
# dispatch (modeling.py:94-96,107-117; ep.py:76-96,216-231)
# ----------------------------------------------------------------------------
@dataclass
class Dispatch:
    """One GPU's share of a routed batch, grouped by local expert.

    counts (n_local,) / offsets (n_local+1,) int32 rows per local expert;
    perm (N*k,) int32 flat entry id of each row (first offsets[-1] valid);
    row_of_entry (N*k,) int32 row of each entry here or -1; dest (N*k,) int32
    destination rank or -1 (only when requested)."""
    counts: torch.Tensor
    offsets: torch.Tensor
    perm: torch.Tensor
    row_of_entry: torch.Tensor
    dest: torch.Tensor | None
    n_tokens: int
    top_k: int
    n_local: int

    @property
    def max_rows(self) -> int:
        return self.n_tokens * self.top_k


def dispatch(topk_idx: torch.Tensor, valid_mask: torch.Tensor | None, n_experts: int,
             table: torch.Tensor, n_rep: torch.Tensor, has_replicas: bool,
             rr: torch.Tensor | None, my_rank: int, g2l: torch.Tensor, n_local: int,
             seg_tokens=None, route_counts: torch.Tensor | None = None,
             want_dest: bool = False, check: bool = True) -> Dispatch:
    """Run mep_dispatch.  ``table`` (E,Rmax) / ``n_rep`` (E,) / ``g2l`` (E,) are
    int32 device tensors; ``rr`` is the (S,E) int64 device counter block
    (updated in place when ``has_replicas``); ``seg_tokens`` the S+1 token
    offsets of the source segments (default: one segment)."""
    dev = _require_device(topk_idx, table, n_rep, g2l, rr, route_counts)
    idx = topk_idx.to(torch.int64).contiguous()
    n, k = idx.shape
    if seg_tokens is None:
        seg_tokens = [0, n]
    seg = [int(v) for v in seg_tokens]
    n_seg = len(seg) - 1
    seg_arr = (ctypes.c_int64 * len(seg))(*seg)
    vm = _mask_u8(valid_mask, n)
    for name, t, dt in (("table", table, torch.int32), ("n_rep", n_rep, torch.int32),
                        ("g2l", g2l, torch.int32)):
        if t.dtype != dt or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous {dt} tensor")
    if rr is not None and (rr.dtype != torch.int64 or not rr.is_contiguous() or rr.numel() != n_seg * n_experts):
        raise TypeError(f"rr must be a contiguous int64 tensor of {n_seg}x{n_experts}")
    if route_counts is not None and (route_counts.dtype != torch.int64 or route_counts.numel() != n_experts):
        raise TypeError("route_counts must be an int64 tensor of n_experts")
    L = _lib.lib()
    ws = _dispatch_workspace(dev, int(L.mep_dispatch_workspace_size(n, k, n_experts, n_seg, seg_arr)))
    nk = max(n * k, 1)
    counts = torch.empty(max(n_local, 1), dtype=torch.int32, device=dev)
    offsets = torch.empty(n_local + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(nk, dtype=torch.int32, device=dev)
    row_of_entry = torch.empty(nk, dtype=torch.int32, device=dev)
    dest = torch.empty(nk, dtype=torch.int32, device=dev) if want_dest else None
    st = _stream(dev)
    rc = L.mep_dispatch(_ptr(idx), _ptr(vm), n, k, n_experts, table.data_ptr(), n_rep.data_ptr(),
                        table.shape[1], 1 if has_replicas else 0, _ptr(rr), seg_arr, n_seg,
                        my_rank, g2l.data_ptr(), n_local, counts.data_ptr(), offsets.data_ptr(),
                        perm.data_ptr(), row_of_entry.data_ptr(), _ptr(dest), _ptr(route_counts),
                        ws.data_ptr(), ws.numel(), st)
    _lib.check(rc, "mep_dispatch")
    if check:
        _lib.check(L.mep_dispatch_check(ws.data_ptr(), st), "mep_dispatch")
    return Dispatch(counts[:n_local], offsets, perm, row_of_entry, dest, n, k, n_local)


def route_dispatch(x_flat: torch.Tensor, w_router: torch.Tensor, k: int, valid_mask: torch.Tensor | None = None,
                   route_counts: torch.Tensor | None = None, check: bool = True, return_logits: bool = False):
    """Router + all-local dispatch in one call (mep_route_dispatch, top_k = 8):
    (topk_idx, topk_gate, Dispatch[, logits]) equal to router_topk followed by
    dispatch with world-1 tables, one launch fewer.  For other k it makes
    those two calls."""
    dev = _require_device(x_flat, w_router, valid_mask, route_counts)
    x = x_flat.contiguous()
    w = w_router.to(x.dtype).contiguous()
    n, h = x.shape
    e = w.shape[0]
    if k != 8:
        out = router_topk(x, w, k, return_logits=return_logits)
        table = torch.zeros(e, 1, dtype=torch.int32, device=dev)
        n_rep = torch.ones(e, dtype=torch.int32, device=dev)
        g2l = torch.arange(e, dtype=torch.int32, device=dev)
        d = dispatch(out[0], valid_mask, e, table, n_rep, False, None, 0, g2l, e, route_counts=route_counts,
                     check=check)
        return (out[0], out[1], d) + ((out[2],) if return_logits else ())
    if w.shape[1] != h:
        raise ValueError(f"router weight {tuple(w.shape)} does not match hidden {h}")
    if route_counts is not None and (route_counts.dtype != torch.int64 or route_counts.numel() != e):
        raise TypeError("route_counts must be an int64 tensor of n_experts")
    vm = _mask_u8(valid_mask, n)
    L = _lib.lib()
    idx = torch.empty((n, k), dtype=torch.int64, device=dev)
    gate = torch.empty((n, k), dtype=x.dtype, device=dev)
    logits = torch.empty((n, e), dtype=torch.float32, device=dev) if return_logits else None
    ws = _dispatch_workspace(dev, int(L.mep_route_dispatch_workspace_size(n, e)))
    nk = max(n * k, 1)
    counts = torch.empty(e, dtype=torch.int32, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(nk, dtype=torch.int32, device=dev)
    row_of_entry = torch.empty(nk, dtype=torch.int32, device=dev)
    st = _stream(dev)
    rc = L.mep_route_dispatch(x.data_ptr(), w.data_ptr(), _ptr(vm), n, h, e, k, _dtype_code(x), idx.data_ptr(),
                              gate.data_ptr(), _ptr(logits), counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(),
                              row_of_entry.data_ptr(), _ptr(route_counts), ws.data_ptr(), ws.numel(), st)
    _lib.check(rc, "mep_route_dispatch")
    if check:
        _lib.check(L.mep_dispatch_check(ws.data_ptr(), st), "mep_route_dispatch")
    d = Dispatch(counts, offsets, perm, row_of_entry, None, n, k, e)
    return (idx, gate, d) + ((logits,) if return_logits else ())


# ----------------------------------------------------------------------------
# grouped SwiGLU experts (modeling.py:83-104) and combine (modeling.py:120-128,144)
# ----------------------------------------------------------------------------
def grouped_swiglu(x_flat: torch.Tensor, disp: Dispatch, w_in: torch.Tensor, w_out: torch.Tensor,
                   y_entries: torch.Tensor | None = None, w_slot: torch.Tensor | None = None) -> torch.Tensor:
    """Expert outputs for every dispatched row, written to the row's
    (token, slot) cell of ``y_entries`` (N*k, H) (allocated if not given).
    With ``w_slot`` (n_local,) int32, local expert j's weights are slot
    w_slot[j] of w_in (n_slots, 2I, H) / w_out (n_slots, H, I)."""
    dev = _require_device(x_flat, w_in, w_out, y_entries, w_slot)
    x = x_flat.contiguous()
    n, h = x.shape
    if w_in.dim() != 3 or w_out.dim() != 3:
        raise ValueError("w_in must be (E, 2I, H) and w_out (E, H, I)")
    e_loc, two_i, h_in = w_in.shape
    inter = two_i // 2
    n_w = disp.n_local if w_slot is None else e_loc
    if w_slot is not None and (w_slot.dtype != torch.int32 or w_slot.numel() != disp.n_local):
        raise ValueError(f"w_slot must hold {disp.n_local} int32 slots")
    if h_in != h or tuple(w_out.shape) != (e_loc, h, inter) or e_loc != n_w:
        raise ValueError(f"weight shapes {tuple(w_in.shape)} / {tuple(w_out.shape)} do not match "
                         f"hidden {h} and {disp.n_local} local experts")
    wi = w_in.to(x.dtype).contiguous()
    wo = w_out.to(x.dtype).contiguous()
    if y_entries is None:
        y_entries = torch.empty((max(n * disp.top_k, 1), h), dtype=x.dtype, device=dev)
    code = _dtype_code(x)
    L = _lib.lib()
    max_rows = n * disp.top_k
    ws_bytes = L.mep_experts_workspace_size(max_rows, inter, code)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    tq = _tile_queue(dev, max_rows, disp.n_local)
    if w_slot is None:
        rc = L.mep_grouped_swiglu(x.data_ptr(), n, disp.top_k, disp.perm.data_ptr(), disp.offsets.data_ptr(),
                                  disp.n_local, max_rows, wi.data_ptr(), wo.data_ptr(), h, inter, code,
                                  y_entries.data_ptr(), ws.data_ptr(), ws.numel(), tq.data_ptr(), tq.numel(),
                                  _stream(dev))
        _lib.check(rc, "mep_grouped_swiglu")
    else:
        rc = L.mep_grouped_swiglu_slots(x.data_ptr(), n, disp.top_k, disp.perm.data_ptr(),
                                        disp.offsets.data_ptr(), disp.n_local, max_rows, wi.data_ptr(),
                                        wo.data_ptr(), w_slot.contiguous().data_ptr(), h, inter, code,
                                        y_entries.data_ptr(), ws.data_ptr(), ws.numel(),
                                        tq.data_ptr(), tq.numel(), _stream(dev))
        _lib.check(rc, "mep_grouped_swiglu_slots")
    return y_entries


def grouped_swiglu_combine(x_flat: torch.Tensor, disp: Dispatch, w_in: torch.Tensor, w_out: torch.Tensor,
                           topk_gate: torch.Tensor, valid_mask: torch.Tensor | None = None,
                           y_entries: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """grouped_swiglu followed by combine (mep_grouped_swiglu_combine): the
    (n, H) layer output, the same bits as the two calls; for small bf16 top-8
    batches the experts' launch ends with the combine (one launch fewer).
    The dispatch must cover every (token, slot) cell (world 1)."""
    dev = _require_device(x_flat, w_in, w_out, topk_gate, y_entries, out)
    x = x_flat.contiguous()
    n, h = x.shape
    if w_in.dim() != 3 or w_out.dim() != 3:
        raise ValueError("w_in must be (E, 2I, H) and w_out (E, H, I)")
    e_loc, two_i, h_in = w_in.shape
    inter = two_i // 2
    if h_in != h or tuple(w_out.shape) != (e_loc, h, inter) or e_loc != disp.n_local:
        raise ValueError(f"weight shapes {tuple(w_in.shape)} / {tuple(w_out.shape)} do not match "
                         f"hidden {h} and {disp.n_local} local experts")
    if tuple(topk_gate.shape) != (n, disp.top_k):
        raise ValueError(f"topk_gate {tuple(topk_gate.shape)} does not match {n} tokens x top-{disp.top_k}")
    wi = w_in.to(x.dtype).contiguous()
    wo = w_out.to(x.dtype).contiguous()
    gate = topk_gate.to(x.dtype).contiguous()
    vm = _mask_u8(valid_mask, n)
    max_rows = n * disp.top_k
    if y_entries is None:
        y_entries = torch.empty((max(max_rows, 1), h), dtype=x.dtype, device=dev)
    if out is None:
        out = torch.empty((n, h), dtype=x.dtype, device=dev)
    code = _dtype_code(x)
    L = _lib.lib()
    ws_bytes = L.mep_experts_workspace_size(max_rows, inter, code)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    tq = _tile_queue(dev, max_rows, disp.n_local)
    rc = L.mep_grouped_swiglu_combine(x.data_ptr(), n, disp.top_k, disp.perm.data_ptr(), disp.offsets.data_ptr(),
                                      disp.row_of_entry.data_ptr(), gate.data_ptr(), _ptr(vm), disp.n_local,
                                      max_rows, wi.data_ptr(), wo.data_ptr(), h, inter, code,
                                      y_entries.data_ptr(), ws.data_ptr(), ws.numel(), tq.data_ptr(), tq.numel(),
                                      out.data_ptr(), _stream(dev))
    _lib.check(rc, "mep_grouped_swiglu_combine")
    return out


def moe_layer(x_flat: torch.Tensor, w_router: torch.Tensor, k: int, w_in: torch.Tensor, w_out: torch.Tensor,
              valid_mask: torch.Tensor | None = None, route_counts: torch.Tensor | None = None,
              return_logits: bool = False):
    """The MoE block of the all-local backend in one call (mep_moe_layer):
    route_dispatch followed by grouped_swiglu_combine, the same bits;
    returns (out, topk_idx, topk_gate, Dispatch[, logits]).  Decode batches of
    GraniteMoE's shape (bf16, 32 experts, top-8, at most 32 tokens) run as one
    launch."""
    dev = _require_device(x_flat, w_router, w_in, w_out, valid_mask, route_counts)
    x = x_flat.contiguous()
    n, h = x.shape
    w = w_router.to(x.dtype).contiguous()
    e = w.shape[0]
    if w.shape[1] != h or w_in.dim() != 3 or w_out.dim() != 3:
        raise ValueError("w_router must be (E, H), w_in (E, 2I, H) and w_out (E, H, I)")
    e_loc, two_i, h_in = w_in.shape
    inter = two_i // 2
    if e_loc != e or h_in != h or tuple(w_out.shape) != (e, h, inter):
        raise ValueError(f"weight shapes {tuple(w_in.shape)} / {tuple(w_out.shape)} do not match "
                         f"hidden {h} and {e} experts")
    if route_counts is not None and (route_counts.dtype != torch.int64 or route_counts.numel() != e):
        raise TypeError("route_counts must be an int64 tensor of n_experts")
    wi = w_in.to(x.dtype).contiguous()
    wo = w_out.to(x.dtype).contiguous()
    vm = _mask_u8(valid_mask, n)
    L = _lib.lib()
    code = _dtype_code(x)
    idx = torch.empty((n, k), dtype=torch.int64, device=dev)
    gate = torch.empty((n, k), dtype=x.dtype, device=dev)
    logits = torch.empty((n, e), dtype=torch.float32, device=dev) if return_logits else None
    nk = max(n * k, 1)
    counts = torch.empty(e, dtype=torch.int32, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(nk, dtype=torch.int32, device=dev)
    row_of_entry = torch.empty(nk, dtype=torch.int32, device=dev)
    y = torch.empty((nk, h), dtype=x.dtype, device=dev)
    out = torch.empty((n, h), dtype=x.dtype, device=dev)
    dws = _dispatch_workspace(dev, int(L.mep_route_dispatch_workspace_size(n, e)))
    max_rows = n * k
    ews = torch.empty(max(int(L.mep_experts_workspace_size(max_rows, inter, code)), 256), dtype=torch.uint8,
                      device=dev)
    need = int(L.mep_moe_layer_queue_ints(n, e, h))
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream(dev))
    tq = _QUEUES.get(key)
    if tq is None or tq.numel() < need:
        tq = _QUEUES[key] = torch.zeros(max(need, 64), dtype=torch.int32, device=dev)
    rc = L.mep_moe_layer(x.data_ptr(), w.data_ptr(), _ptr(vm), n, h, e, k, code, wi.data_ptr(), wo.data_ptr(), inter,
                         idx.data_ptr(), gate.data_ptr(), _ptr(logits), counts.data_ptr(), offsets.data_ptr(),
                         perm.data_ptr(), row_of_entry.data_ptr(), _ptr(route_counts), y.data_ptr(), dws.data_ptr(),
                         dws.numel(), ews.data_ptr(), ews.numel(), tq.data_ptr(), tq.numel(), out.data_ptr(),
                         _stream(dev))
    _lib.check(rc, "mep_moe_layer")
    d = Dispatch(counts, offsets, perm, row_of_entry, None, n, k, e)
    return (out, idx, gate, d) + ((logits,) if return_logits else ())


def copy_experts(src_in: torch.Tensor, src_out: torch.Tensor, src_index: list[int], dst_in: torch.Tensor,
                 dst_out: torch.Tensor, dst_slot: list[int]) -> None:
    """Slot dst_slot[i] of (dst_in, dst_out) = expert src_index[i] of
    (src_in, src_out), one launch (mep_copy_experts); all four are device
    tensors in the checkpoint layout (E, 2I, H) / (E, H, I)."""
    dev = _require_device(src_in, src_out, dst_in, dst_out)
    n = len(src_index)
    if n != len(dst_slot):
        raise ValueError("src_index and dst_slot differ in length")
    if n == 0:
        return
    for t in (src_in, src_out, dst_in, dst_out):
        if not t.is_contiguous() or t.dtype != dst_in.dtype:
            raise TypeError("expert tensors must be contiguous and of one dtype")
    e_src, two_i, h = src_in.shape
    arr_s = (ctypes.c_int32 * n)(*[int(v) for v in src_index])
    arr_d = (ctypes.c_int32 * n)(*[int(v) for v in dst_slot])
    rc = _lib.lib().mep_copy_experts(src_in.data_ptr(), src_out.data_ptr(), e_src, dst_in.data_ptr(),
                                     dst_out.data_ptr(), dst_in.shape[0], arr_s, arr_d, n, h, two_i // 2,
                                     _dtype_code(dst_in), _stream(dev))
    _lib.check(rc, "mep_copy_experts")


def _expert_shapes(x, disp, w_in=None, w_out=None):
    n, h = x.shape
    if w_in is not None:
        e_loc, two_i, h_in = w_in.shape
        if h_in != h or e_loc != disp.n_local:
            raise ValueError(f"w_in {tuple(w_in.shape)} does not match hidden {h} / {disp.n_local} experts")
        return n, h, two_i // 2
    e_loc, h_out, inter = w_out.shape
    if h_out != h or e_loc != disp.n_local:
        raise ValueError(f"w_out {tuple(w_out.shape)} does not match hidden {h} / {disp.n_local} experts")
    return n, h, inter


def swiglu_gate_up(x_flat: torch.Tensor, disp: Dispatch, w_in: torch.Tensor,
                   act: torch.Tensor | None = None) -> torch.Tensor:
    """GEMM-1 + SwiGLU only: act (N*k, I) rows in dispatch order (modeling.py:101-102)."""
    dev = _require_device(x_flat, w_in, act)
    x = x_flat.contiguous()
    n, h, inter = _expert_shapes(x, disp, w_in=w_in)
    if act is None:
        act = torch.empty((max(n * disp.top_k, 1), inter), dtype=x.dtype, device=dev)
    wi = w_in.to(x.dtype).contiguous()
    tq = _tile_queue(dev, n * disp.top_k, disp.n_local)
    rc = _lib.lib().mep_swiglu_gate_up(x.data_ptr(), n, disp.top_k, disp.perm.data_ptr(),
                                       disp.offsets.data_ptr(), disp.n_local, n * disp.top_k,
                                       wi.data_ptr(), h, inter, _dtype_code(x), act.data_ptr(),
                                       act.numel() * act.element_size(), tq.data_ptr(), tq.numel(),
                                       _stream(dev))
    _lib.check(rc, "mep_swiglu_gate_up")
    return act


def swiglu_down(act: torch.Tensor, x_flat: torch.Tensor, disp: Dispatch, w_out: torch.Tensor,
                y_entries: torch.Tensor | None = None) -> torch.Tensor:
    """GEMM-2 + scatter to (token, slot) cells (modeling.py:103)."""
    dev = _require_device(act, x_flat, w_out, y_entries)
    n, h, inter = _expert_shapes(x_flat, disp, w_out=w_out)
    if y_entries is None:
        y_entries = torch.empty((max(n * disp.top_k, 1), h), dtype=act.dtype, device=dev)
    wo = w_out.to(act.dtype).contiguous()
    tq = _tile_queue(dev, n * disp.top_k, disp.n_local)
    rc = _lib.lib().mep_swiglu_down(act.data_ptr(), n, disp.top_k, disp.perm.data_ptr(),
                                    disp.offsets.data_ptr(), disp.n_local, n * disp.top_k, wo.data_ptr(),
                                    h, inter, _dtype_code(act), y_entries.data_ptr(),
                                    tq.data_ptr(), tq.numel(), _stream(dev))
    _lib.check(rc, "mep_swiglu_down")
    return y_entries


def combine(y_entries: torch.Tensor, topk_gate: torch.Tensor, row_of_entry: torch.Tensor,
            valid_mask: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = sum over present slots s (slot order) of gate[t,s] * y[t*k+s]."""
    dev = _require_device(y_entries, topk_gate, row_of_entry, out)
    n, k = topk_gate.shape
    h = y_entries.shape[1]
    gate = topk_gate.to(y_entries.dtype).contiguous()
    vm = _mask_u8(valid_mask, n)
    if out is None:
        out = torch.empty((n, h), dtype=y_entries.dtype, device=dev)
    rc = _lib.lib().mep_combine(y_entries.data_ptr(), gate.data_ptr(), row_of_entry.data_ptr(), _ptr(vm),
                                n, k, h, _dtype_code(y_entries), out.data_ptr(), _stream(dev))
    _lib.check(rc, "mep_combine")
    return out


def combine_rows(y_rows: torch.Tensor, topk_gate: torch.Tensor, row_of_entry: torch.Tensor,
                 valid_mask: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Expert-parallel return path (ep.py:237-242): out[t] = sum over present
    slots s (slot order) of gate[t,s] * y_rows[row_of_entry[t*k+s]]."""
    dev = _require_device(y_rows, topk_gate, row_of_entry, out)
    n, k = topk_gate.shape
    h = y_rows.shape[1]
    gate = topk_gate.to(y_rows.dtype).contiguous()
    vm = _mask_u8(valid_mask, n)
    if out is None:
        out = torch.empty((n, h), dtype=y_rows.dtype, device=dev)
    rc = _lib.lib().mep_combine_rows(y_rows.data_ptr(), gate.data_ptr(), row_of_entry.data_ptr(), _ptr(vm),
                                     n, k, h, _dtype_code(y_rows), out.data_ptr(), _stream(dev))
    _lib.check(rc, "mep_combine_rows")
    return out


def gather_rows(x: torch.Tensor, perm: torch.Tensor, n_rows: int, top_k: int,
                topk_idx: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Send buffer of expert parallelism (ep.py:225-226): rows x[perm[i] // top_k]
    for i < n_rows, and with `topk_idx` the expert of each row."""
    dev = _require_device(x, perm, topk_idx)
    x = x.contiguous()
    n, h = x.shape
    out = torch.empty((n_rows, h), dtype=x.dtype, device=dev)
    ids = None
    flat = None
    if topk_idx is not None:
        flat = topk_idx.reshape(-1).to(torch.int64).contiguous()
        ids = torch.empty(n_rows, dtype=torch.int64, device=dev)
    rc = _lib.lib().mep_gather_rows(x.data_ptr(), n, top_k, perm.data_ptr(), n_rows, h, _dtype_code(x),
                                    _ptr(flat), _ptr(ids), out.data_ptr(), _stream(dev))
    _lib.check(rc, "mep_gather_rows")
    return out, ids
