"""End-to-end MoE layer on the GPU vs the oracle: router hook + backend.

The layer is what Block.forward does after its post-attention RMSNorm
(modeling.py:190-196): route, then the backend returns the combined (N, H)
expert output.  Configurations: fp32 T=512 (bar 1e-5), decode bf16 T=32,
skewed bf16 T=16384 (bar 2e-2), one rank's share under the balanced plan.
"""
import json

import numpy as np
import pytest
import torch

from helpers import TOL_BF16, TOL_F32, banner, rel_err, row_rel_err, to_np
from miniep_amd import EmulatedEPMoEBackend, HipEPShareBackend, HipMoEBackend, Placement, ops, route, workloads
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer_on_gpu(L, dtype, valid=None, check=True):
    x = L.x.to(dtype).to(DEV)
    backend = HipMoEBackend(L.w_in.to(dtype).to(DEV), L.w_out.to(dtype).to(DEV), check=check)
    idx, gate, logits = route(x, L.w_router.to(dtype).to(DEV), L.top_k, return_logits=True)
    out = backend(x, idx, gate, None if valid is None else valid.to(DEV))
    return out, idx, gate, logits, backend


def _oracle_layer(L, dtype, logits, valid=None, tokens=None):
    """Oracle layer on the kernel's fp32 logits (routing bit-exact given them)."""
    bf = dtype == torch.bfloat16
    xr = L.x.to(dtype).float().numpy()
    idx, gate = O.topk_softmax(logits, L.top_k, gate_bf16=bf)
    sel = slice(None) if tokens is None else tokens
    v = None if valid is None else valid.numpy()[sel]
    return O.moe_layer_local(xr[sel], idx[sel], gate[sel], L.w_in.to(dtype).float().numpy(),
                             L.w_out.to(dtype).float().numpy(), v, act_bf16=bf, out_bf16=bf), idx, gate


def test_fp32_layer_t512():
    banner("layer fp32 t=512")
    L = workloads.make_layer(512, seed=0)
    out, idx, gate, logits, _ = _layer_on_gpu(L, torch.float32)
    ref, ridx, _ = _oracle_layer(L, torch.float32, to_np(logits))
    assert np.array_equal(to_np(idx), ridx)
    err = rel_err(to_np(out), ref)
    print(f"rel err {err:.3e}")
    assert err <= TOL_F32


def test_decode_bf16_t32():
    banner("layer bf16 t=32")
    L = workloads.make_layer(32, seed=1)
    out, idx, gate, logits, be = _layer_on_gpu(L, torch.bfloat16)
    ref, ridx, _ = _oracle_layer(L, torch.bfloat16, to_np(logits))
    assert np.array_equal(to_np(idx), ridx)
    assert rel_err(to_np(out), ref) <= TOL_BF16
    assert row_rel_err(to_np(out), ref, floor=1e-3 * float(np.abs(ref).max())) <= TOL_BF16
    assert int(to_np(be.last_dispatch.counts).sum()) == 32 * 8


def test_masked_tokens_and_dummy_prefill():
    banner("layer masks")
    L = workloads.make_layer(700, seed=2)
    valid = torch.rand(700, generator=torch.Generator().manual_seed(0)) < 0.7
    out, idx, gate, logits, _ = _layer_on_gpu(L, torch.bfloat16, valid)
    ref, _, _ = _oracle_layer(L, torch.bfloat16, to_np(logits), valid)
    o = to_np(out)
    assert (o[~valid.numpy()] == 0).all()
    assert rel_err(o, ref) <= TOL_BF16
    # dummy prefill: zero expert load (worker.py:112-122)
    out0, *_ = _layer_on_gpu(L, torch.bfloat16, torch.zeros(700, dtype=torch.bool))
    assert (to_np(out0) == 0).all()


def test_skewed_bf16_t16384():
    banner("layer bf16 t=16384 zipf 1.2")
    L = workloads.make_layer(16384, seed=0, zipf_s=1.2)
    out, idx, gate, logits, be = _layer_on_gpu(L, torch.bfloat16, check=False)
    lg = to_np(logits)
    ridx, _ = O.topk_softmax(lg, 8, gate_bf16=True)
    assert np.array_equal(to_np(idx), ridx)
    counts = np.bincount(ridx.reshape(-1), minlength=32)
    assert to_np(be.last_dispatch.counts).tolist() == counts.tolist()
    # every one of the 16384 output rows against the oracle: normwise, and row
    # by row (each row against its own largest value, floored at 1e-3 of the
    # tensor's) so that no low-norm token hides under the largest rows
    ref, _, _ = _oracle_layer(L, torch.bfloat16, lg)
    o = to_np(out)
    err = rel_err(o, ref)
    rerr = row_rel_err(o, ref, floor=1e-3 * float(np.abs(ref).max()))
    print(f"rel err {err:.3e}, worst row {rerr:.3e} over all {ref.shape[0]} tokens")
    assert err <= TOL_BF16
    assert rerr <= TOL_BF16
    # bitwise identical on a second run
    out2 = be(L.x.to(torch.bfloat16).to(DEV), idx, gate)
    assert torch.equal(out, out2)


def test_largest_bf16_t262144():
    """2^18 tokens: act is 2 GiB and y_entries 4 GiB, the sizes where the
    kernels' 32-bit DMA offsets and int32 entry ids are closest to their
    limits.  Routing bit-exact, counts equal the bincount, the first, last
    and 512 random tokens against the oracle."""
    banner("layer bf16 t=262144")
    T = 262144
    L = workloads.make_layer(T, seed=3, zipf_s=1.2)
    out, idx, gate, logits, be = _layer_on_gpu(L, torch.bfloat16, check=False)
    lg = to_np(logits)
    ridx, _ = O.topk_softmax(lg, 8, gate_bf16=True)
    assert np.array_equal(to_np(idx), ridx)
    assert to_np(be.last_dispatch.counts).tolist() == np.bincount(ridx.reshape(-1), minlength=32).tolist()
    toks = np.concatenate([np.arange(256), np.arange(T - 256, T),
                           np.random.default_rng(1).choice(T, 512, replace=False)])
    ref, _, _ = _oracle_layer(L, torch.bfloat16, lg, tokens=toks)
    o = to_np(out[torch.from_numpy(toks).to(DEV)])
    err = rel_err(o, ref)
    rerr = row_rel_err(o, ref, floor=1e-3 * float(np.abs(ref).max()))
    print(f"rel err {err:.3e}, worst row {rerr:.3e}")
    assert err <= TOL_BF16
    assert rerr <= TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_emulated_ep_equals_local_bitwise(golden_dir, dtype):
    """Placement invariance (ep.py:1-8): world-4 balanced plan, 4 sources, every
    layer-2 rank share on its own weight slice, then one combine -- identical
    bits to the all-local backend."""
    banner(f"emulated ep4 {dtype}")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    L = workloads.make_layer(8192 if dtype == torch.bfloat16 else 1024, seed=4, zipf_s=1.1)
    x = L.x.to(dtype).to(DEV)
    wi, wo = L.w_in.to(dtype).to(DEV), L.w_out.to(dtype).to(DEV)
    idx, gate = route(x, L.w_router.to(dtype).to(DEV), 8)
    n = x.shape[0]
    local = HipMoEBackend(wi, wo)(x, idx, gate)
    ep = EmulatedEPMoEBackend(2, p, 4, wi, wo)
    got = ep(x, idx, gate, seg_tokens=[n * s // 4 for s in range(5)])
    assert torch.equal(local, got)


def test_rank_share_rows_match_oracle(golden_dir):
    """Every row of every rank's share (plan layer 2, 4 sources, T=8192)
    against the oracle's experts on that rank's weight slice."""
    banner("rank share rows, all ranks")
    plan = json.loads((golden_dir / "plan_balanced.json").read_text())
    p = Placement.from_plan(plan, device=DEV)
    L = workloads.make_layer(8192, seed=5, zipf_s=1.1)
    x = L.x.to(torch.bfloat16).to(DEV)
    idx, _ = route(x, L.w_router.to(torch.bfloat16).to(DEV), 8)
    xr = L.x.to(torch.bfloat16).float().numpy()
    flat_e = to_np(idx).reshape(-1)
    total = 0
    for r in range(4):
        ids = p.experts_of_rank(r)[2]
        be = HipEPShareBackend(2, p, r, L.w_in[ids].to(torch.bfloat16).to(DEV),
                               L.w_out[ids].to(torch.bfloat16).to(DEV))
        disp, y = be.share(x, idx, seg_tokens=[0, 2048, 4096, 6144, 8192])
        M = int(disp.offsets[-1])
        rows = to_np(disp.perm)[:M]
        g2l = {e: i for i, e in enumerate(ids)}
        eids = np.array([g2l[int(e)] for e in flat_e[rows]])
        ref = O.experts(xr[rows // 8], eids, L.w_in[ids].to(torch.bfloat16).float().numpy(),
                        L.w_out[ids].to(torch.bfloat16).float().numpy(), act_bf16=True, out_bf16=True)
        err = rel_err(to_np(y)[rows], ref)
        print(f"rank {r}: {M} rows, rel err {err:.3e}", flush=True)
        assert err <= TOL_BF16
        total += M
    # the shares partition the 65536 entries (every entry has exactly one destination)
    assert total == 8192 * 8


@pytest.mark.parametrize("H,I,E,k,n,dtype", [
    (2048, 256, 64, 4, 300, torch.bfloat16),
    (512, 384, 16, 2, 1000, torch.bfloat16),
    (512, 256, 64, 6, 700, torch.float32),
    (256, 128, 16, 1, 1, torch.bfloat16),       # one token, k = 1, I not a multiple of 256
    (256, 256, 16, 1, 37, torch.float32),
    (1024, 512, 32, 8, 1, torch.bfloat16),      # one token through the small-batch kernels
    (1024, 512, 64, 8, 3000, torch.bfloat16),   # 64 experts, tiled kernels
    (1536, 256, 32, 8, 500, torch.bfloat16),    # hidden not a power of two
    (2048, 256, 16, 4, 300, torch.float32),     # fp32 rows of 8 KiB
])
def test_layer_other_shapes(H, I, E, k, n, dtype):
    """Router (E = 16 / 64), dispatch, experts and combine at other shapes."""
    banner(f"layer shape H={H} I={I} E={E} k={k} n={n} {dtype}")
    L = workloads.make_layer(n, seed=E + k, zipf_s=1.1, hidden=H, n_experts=E, top_k=k, inter=I)
    valid = torch.rand(n, generator=torch.Generator().manual_seed(7)) < 0.9
    out, idx, gate, logits, _ = _layer_on_gpu(L, dtype, valid)
    ref, ridx, _ = _oracle_layer(L, dtype, to_np(logits), valid)
    assert np.array_equal(to_np(idx), ridx)
    err = rel_err(to_np(out), ref)
    print(f"rel err {err:.3e}")
    assert err <= (TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)
    assert (to_np(out)[~valid.numpy()] == 0).all()
