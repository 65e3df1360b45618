"""The whole MoE block of a decode batch in one launch (mep_moe_layer).

Router + dispatch (one workgroup), GEMM-1 + SwiGLU, GEMM-2 and the combine run
as one launch for bf16, 32 experts, top-8 and at most 32 tokens.  Every
output must equal mep_route_dispatch followed by mep_grouped_swiglu_combine
bit for bit -- indices, gates, logits, counts, offsets, perm, row_of_entry,
route_counts and the layer output -- on consecutive inputs through the same
buffers, with masked tokens and with every token masked; the schedule words
return to zero; a captured graph replays it exactly; and each of its bounded
waits, forced to give up from the host, is reported and poisons the output
(Block.forward's router + backend call, modeling.py:192-196).
"""
import contextlib

import numpy as np
import pytest
import torch

from helpers import TOL_BF16, banner, rel_err, row_rel_err, to_np
from miniep_amd import _lib, ops, workloads
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _two_calls(x, w_r, w_in, w_out, valid=None, route_counts=None):
    idx, gate, d, logits = ops.route_dispatch(x, w_r, 8, valid, route_counts=route_counts, check=True,
                                              return_logits=True)
    out = ops.grouped_swiglu_combine(x, d, w_in, w_out, gate, valid)
    return out, idx, gate, d, logits


def _queue_words_zero():
    for q in ops._QUEUES.values():
        assert int(q.abs().sum()) == 0


def _layer(n, seed, hidden=1024, inter=512):
    L = workloads.make_layer(n, seed=seed, hidden=hidden, inter=inter)
    return (L.x.to(BF).to(DEV), L.w_router.to(BF).to(DEV), L.w_in.to(BF).to(DEV), L.w_out.to(BF).to(DEV), L)


@pytest.mark.parametrize("case", ["t1", "t7", "t16", "t32", "masked_t32", "h2048_t24", "h4096_t8", "i1024_t32", "t33"])
def test_moe_layer_equals_two_calls(case):
    """Shapes: hidden 1024 / 2048 / 4096 (GEMM-1's K loop of 4 / 8 / 16
    blocks of x through the LDS ring), intermediate 1024 (GEMM-2 has K-steps
    past the 16 it stages), masks, and 33 tokens (the two calls)."""
    banner(f"moe_layer one launch vs two calls: {case}")
    n = int(case.split("_t")[-1].lstrip("t"))
    hidden = {"h2048": 2048, "h4096": 4096}.get(case.split("_")[0], 1024)
    inter = 1024 if case.startswith("i1024") else 512
    x, w_r, wi, wo, L = _layer(n, 61 + n, hidden, inter)
    g = torch.Generator().manual_seed(n)
    valid = (torch.rand(n, generator=g) < 0.6).to(DEV) if case.startswith("masked") else None
    rc1 = torch.zeros(32, dtype=torch.int64, device=DEV)
    rc2 = torch.zeros(32, dtype=torch.int64, device=DEV)
    for rep in range(2):                                     # a second input through the same buffers
        xr = x if rep == 0 else torch.randn(tuple(x.shape), generator=g).to(BF).to(DEV)
        got = ops.moe_layer(xr, w_r, 8, wi, wo, valid, route_counts=rc1, return_logits=True)
        ops.experts_check()
        ops.dispatch_check()
        want = _two_calls(xr, w_r, wi, wo, valid, route_counts=rc2)
        ops.experts_check()
        out, idx, gate, d, logits = got
        out2, idx2, gate2, d2, logits2 = want
        assert torch.equal(idx, idx2) and torch.equal(gate, gate2) and torch.equal(logits, logits2), rep
        assert torch.equal(d.counts, d2.counts) and torch.equal(d.offsets, d2.offsets), rep
        m = int(d2.offsets[-1])
        assert torch.equal(d.perm[:m], d2.perm[:m]) and torch.equal(d.row_of_entry, d2.row_of_entry), rep
        assert torch.equal(out, out2), rep
        assert torch.equal(rc1, rc2), rep
        _queue_words_zero()
    # and the oracle: routing bit-exact given the kernel's fp32 logits, the output within the bf16 bar
    lg = to_np(logits)
    ridx, rgate = O.topk_softmax(lg, 8, gate_bf16=True)
    assert np.array_equal(to_np(idx), ridx)
    v = None if valid is None else valid.cpu().numpy()
    ref = O.moe_layer_local(xr.float().cpu().numpy(), ridx, rgate, wi.float().cpu().numpy(), wo.float().cpu().numpy(),
                            v, act_bf16=True, out_bf16=True)
    o = to_np(out)
    assert rel_err(o, ref) <= TOL_BF16
    assert row_rel_err(o, ref, floor=1e-3 * float(np.abs(ref).max())) <= TOL_BF16
    if v is not None:
        assert (o[~v] == 0).all()


def test_moe_layer_interleaved_with_large_dispatch():
    """The decode launch and the one-launch router + dispatch of a large
    batch share the stream's dispatch workspace (header, status words, the
    epoch that tags the exchange) and schedule buffer: interleaved, each
    gives the bits it gives alone."""
    banner("moe_layer one launch interleaved with a 4096-token route_dispatch")
    x, w_r, wi, wo, _ = _layer(32, 74)
    L = workloads.make_layer(4096, seed=75, zipf_s=1.2)
    xb, wb = L.x.to(BF).to(DEV), L.w_router.to(BF).to(DEV)
    out0 = ops.moe_layer(x, w_r, 8, wi, wo)[0].clone()
    idx0, gate0, d0 = ops.route_dispatch(xb, wb, 8, check=True)
    ref = (idx0.clone(), d0.offsets.clone(), d0.perm.clone(), d0.row_of_entry.clone())
    for _ in range(3):
        out = ops.moe_layer(x, w_r, 8, wi, wo)[0]
        idx, gate, d = ops.route_dispatch(xb, wb, 8, check=True)
        ops.experts_check()
        assert torch.equal(out, out0)
        assert torch.equal(idx, ref[0]) and torch.equal(d.offsets, ref[1])
        assert torch.equal(d.perm, ref[2]) and torch.equal(d.row_of_entry, ref[3])
    _queue_words_zero()


def test_moe_layer_every_token_masked():
    banner("moe_layer one launch: every token masked")
    x, w_r, wi, wo, _ = _layer(16, 71)
    valid = torch.zeros(16, dtype=torch.bool, device=DEV)
    out, idx, gate, d = ops.moe_layer(x, w_r, 8, wi, wo, valid)
    ops.experts_check()
    assert bool((out == 0).all())
    assert int(d.offsets[-1]) == 0 and bool((d.row_of_entry == -1).all())
    _queue_words_zero()


def test_moe_layer_graph_replay():
    """Captured in a HIP graph, every replay equals the eager call on the same
    input, with eager calls on other inputs in between."""
    banner("moe_layer one launch: graph replay")
    g = torch.Generator().manual_seed(72)
    _, w_r, wi, wo, _ = _layer(32, 72)
    xs = [torch.randn(32, 1024, generator=g).to(BF).to(DEV) for _ in range(2)]
    x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.moe_layer(x, w_r, 8, wi, wo)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            got = ops.moe_layer(x, w_r, 8, wi, wo)
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(4):
        x.copy_(xs[rep % 2])
        want = ops.moe_layer(x, w_r, 8, wi, wo)[0].clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got[0], want), rep
        ops.moe_layer(xs[(rep + 1) % 2], w_r, 8, wi, wo)
        torch.cuda.synchronize()
    ops.experts_check()
    _queue_words_zero()


@contextlib.contextmanager
def _force_giveup(site):
    L = _lib.lib()
    _lib.check(L.mep_test_force_giveup(site, 2000), "mep_test_force_giveup")
    try:
        yield
    finally:
        _lib.check(L.mep_test_force_giveup(_lib.GIVEUP_NONE, 0), "mep_test_force_giveup")


@pytest.mark.parametrize("site", ["routed", "chunk"])
def test_moe_layer_giveup(site):
    """routed: the first GEMM-1 workgroup's wait for the routing gives up --
    flagged, and the whole output is NaN (the launch is poisoned); chunk: the
    GEMM-2 workgroups of expert 0 give up waiting for act -- flagged, NaN for
    the tokens that use expert 0, the others exact.  The schedule words return
    to zero and the next call is exact either way."""
    banner(f"moe_layer one launch: give-up ({site})")
    x, w_r, wi, wo, _ = _layer(32, 73)
    out0, idx0, gate0, d0 = ops.moe_layer(x, w_r, 8, wi, wo)
    ops.experts_check()
    assert int(d0.counts[0]) > 0                              # expert 0 has rows
    with _force_giveup(_lib.GIVEUP_ROUTED if site == "routed" else _lib.GIVEUP_CHUNK):
        out1 = ops.moe_layer(x, w_r, 8, wi, wo)[0]
        torch.cuda.synchronize()
    with pytest.raises(_lib.MepError) as ei:
        ops.experts_check()
    assert "gave up" in ei.value.message
    if site == "routed":
        assert bool(torch.isnan(out1.float()).all())
    else:
        uses0 = (idx0 == 0).any(dim=1)
        assert bool(torch.isnan(out1[uses0].float()).all())
        assert torch.equal(out1[~uses0], out0[~uses0])
    _queue_words_zero()
    out2 = ops.moe_layer(x, w_r, 8, wi, wo)[0]
    ops.experts_check()
    assert torch.equal(out2, out0)
    _queue_words_zero()
