"""Router parity on the GPU (mep_router_topk, mep_topk_softmax) vs the oracle.

Bar: indices bit-exact given the same fp32 logits (including tied logits,
resolved lower-id-first on both sides); gates within 1 ulp-scale tolerance;
fused-router logits within fp32 accumulation noise of the float64 oracle.
"""
import numpy as np
import pytest
import torch

from helpers import banner, rel_err, to_np
from miniep_amd import ops, workloads
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("n,e,k", [(4096, 32, 8), (1001, 32, 8), (77, 16, 4), (300, 64, 8),
                                   (129, 256, 8), (50, 8, 8), (33, 32, 1)])
@pytest.mark.parametrize("gate_dtype", [torch.float32, torch.bfloat16])
def test_topk_softmax_bit_exact(n, e, k, gate_dtype):
    banner(f"topk_softmax n={n} e={e} k={k} gate={gate_dtype}")
    g = torch.Generator().manual_seed(n * 7 + e)
    lg = torch.randn(n, e, generator=g) * 2
    idx, gate = ops.topk_softmax(lg.to(DEV), k, gate_dtype)
    ridx, rgate = O.topk_softmax(lg.numpy(), k, gate_bf16=gate_dtype == torch.bfloat16)
    assert np.array_equal(to_np(idx), ridx)
    tol = 2 ** -8 if gate_dtype == torch.bfloat16 else 2e-6
    assert np.abs(to_np(gate) - rgate).max() <= tol


def test_topk_softmax_ties_lower_id_first():
    banner("topk_softmax ties")
    g = torch.Generator().manual_seed(5)
    lg = torch.randint(-2, 3, (2000, 32), generator=g).float()
    lg[0] = 0.0                                     # all equal
    lg[1, :] = -0.0
    lg[1, 7] = 0.0                                  # -0.0 == +0.0
    idx, gate = ops.topk_softmax(lg.to(DEV), 8)
    ridx, rgate = O.topk_softmax(lg.numpy(), 8)
    assert np.array_equal(to_np(idx), ridx)
    assert to_np(idx)[0].tolist() == list(range(8))
    np.testing.assert_allclose(to_np(gate), rgate, rtol=2e-6)


def test_topk_matches_torch_on_tie_free_rows():
    banner("topk vs torch.topk")
    g = torch.Generator().manual_seed(6)
    lg = torch.randn(4096, 32, generator=g)
    ref_v, ref_i = lg.topk(8, dim=-1)
    idx, gate = ops.topk_softmax(lg.to(DEV), 8)
    assert torch.equal(idx.cpu(), ref_i)
    torch.testing.assert_close(gate.cpu(), torch.softmax(ref_v, -1), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,e", [(512, 32), (1000, 32), (16384, 32), (100, 16), (100, 64), (1, 32)])
def test_router_fused(dtype, n, e):
    banner(f"router n={n} e={e} dtype={dtype}")
    g = torch.Generator().manual_seed(11 + n)
    x = torch.randn(n, 1024, generator=g).to(dtype)
    w = (torch.randn(e, 1024, generator=g) * 0.02).to(dtype)
    k = 8
    idx, gate, logits = ops.router_topk(x.to(DEV), w.to(DEV), k, return_logits=True)
    xr, wr = x.float().numpy(), w.float().numpy()
    ref_logits = O.router_logits(xr, wr)
    lg = to_np(logits)
    # fp32 accumulation of 1024 exact products vs the float64 sum
    assert np.abs(lg - ref_logits).max() <= 1e-5 * np.abs(ref_logits).max() + 1e-6
    # selection + softmax bit-exact given the kernel's own fp32 logits
    ridx, rgate = O.topk_softmax(lg, k, gate_bf16=dtype == torch.bfloat16)
    assert np.array_equal(to_np(idx), ridx)
    tol = 2 ** -8 if dtype == torch.bfloat16 else 2e-6
    assert np.abs(to_np(gate) - rgate).max() <= tol
    # and equal to the oracle's own routing wherever its top-9 gaps exceed the logit noise
    oidx, _ = O.topk_softmax(ref_logits, k)
    s = -np.sort(-ref_logits, axis=1)
    clear = (np.diff(-s[:, : k + 1], axis=1) > 1e-4).all(axis=1)
    assert clear.mean() > 0.9
    assert np.array_equal(to_np(idx)[clear], oidx[clear])


def test_router_skewed_layer_routing_counts():
    """Full-size skewed layer: per-expert counts from the kernel's routing equal
    the oracle's selection on the kernel logits (bit-exact)."""
    banner("router skewed t=16384")
    L = workloads.make_layer(16384, seed=0, zipf_s=1.2)
    x = L.x.to(torch.bfloat16).to(DEV)
    w = L.w_router.to(torch.bfloat16).to(DEV)
    idx, gate, logits = ops.router_topk(x, w, 8, return_logits=True)
    ridx, _ = O.topk_softmax(to_np(logits), 8)
    assert np.array_equal(to_np(idx), ridx)
    counts = np.bincount(ridx.reshape(-1), minlength=32)
    assert counts.max() / counts.mean() > 3.5


def test_router_rejects_bad_shapes():
    banner("router errors")
    x = torch.randn(4, 1000, device=DEV)
    w = torch.randn(32, 1000, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 256"):
        ops.router_topk(x, w, 8)
    with pytest.raises(RuntimeError, match="n_experts"):
        ops.router_topk(torch.randn(4, 256, device=DEV), torch.randn(48, 256, device=DEV), 8)
    idx, gate = ops.router_topk(torch.randn(0, 256, device=DEV), torch.randn(32, 256, device=DEV), 8)
    assert idx.shape == (0, 8)


@pytest.mark.parametrize("k", [1, 4, 6])
def test_router_fused_runtime_k(k):
    """top-k other than 8 takes the router's runtime-k selection path."""
    banner(f"router runtime k={k}")
    g = torch.Generator().manual_seed(40 + k)
    x = torch.randn(700, 1024, generator=g).to(torch.bfloat16)
    w = (torch.randn(32, 1024, generator=g) * 0.02).to(torch.bfloat16)
    idx, gate, logits = ops.router_topk(x.to(DEV), w.to(DEV), k, return_logits=True)
    ridx, rgate = O.topk_softmax(to_np(logits), k, gate_bf16=True)
    assert np.array_equal(to_np(idx), ridx)
    assert np.abs(to_np(gate) - rgate).max() <= 2 ** -8


@pytest.mark.parametrize("e", [16, 32, 64])
def test_router_fused_tied_logits(e):
    """Exactly tied logits inside the router kernel (duplicated router rows,
    all-zero tokens): lower expert id first, as the oracle's rule says."""
    banner(f"router tied logits e={e}")
    g = torch.Generator().manual_seed(70 + e)
    x = torch.randn(640, 1024, generator=g).to(torch.bfloat16)
    x[::7] = 0                                           # every logit 0: experts 0..7
    w = (torch.randn(e, 1024, generator=g) * 0.02).to(torch.bfloat16)
    w[e // 2] = w[3]                                     # tied pairs and a triple in every row
    w[e - 1] = w[1]
    w[e - 2] = w[1]
    idx, gate, logits = ops.router_topk(x.to(DEV), w.to(DEV), 8, return_logits=True)
    lg = to_np(logits)
    assert (lg[:, e // 2] == lg[:, 3]).all() and (lg[:, e - 1] == lg[:, 1]).all()
    ridx, rgate = O.topk_softmax(lg, 8, gate_bf16=True)
    assert np.array_equal(to_np(idx), ridx)
    assert to_np(idx)[0].tolist() == list(range(8))
    assert np.abs(to_np(gate) - rgate).max() <= 2 ** -8


@pytest.mark.parametrize("n,e,dtype,masked", [(16384, 32, torch.bfloat16, False), (700, 32, torch.bfloat16, True),
                                              (63, 16, torch.float32, True), (1, 64, torch.bfloat16, False),
                                              (32, 32, torch.bfloat16, True),      # one workgroup
                                              (32768, 32, torch.bfloat16, True),   # 512 workgroups, 2 per CU
                                              (32769, 32, torch.bfloat16, False),  # one more: two launches
                                              (40000, 32, torch.bfloat16, True),   # > 512 blocks: scanned
                                              (0, 32, torch.bfloat16, False)])
def test_route_dispatch_equals_two_calls(n, e, dtype, masked):
    """mep_route_dispatch (bf16 with 32 experts: one cooperative launch while
    its workgroups fit on the GPU at once; otherwise the router kernel with
    histogram output + scatter) gives the bits of mep_router_topk followed by
    mep_dispatch."""
    banner(f"route_dispatch n={n} e={e} {dtype} masked={masked}")
    L = workloads.make_layer(max(n, 1), seed=n + e, zipf_s=1.2 if e == 32 else 0.0, n_experts=e)
    x = L.x[:n].to(dtype).to(DEV)
    w = L.w_router.to(dtype).to(DEV)
    valid = (torch.rand(n, generator=torch.Generator().manual_seed(3)) < 0.8).to(DEV) if masked else None
    rc1 = torch.zeros(e, dtype=torch.int64, device=DEV)
    rc2 = torch.zeros(e, dtype=torch.int64, device=DEV)
    idx, gate, d = ops.route_dispatch(x, w, 8, valid, route_counts=rc1)
    idx2, gate2 = ops.router_topk(x, w, 8)
    table = torch.zeros(e, 1, dtype=torch.int32, device=DEV)
    n_rep = torch.ones(e, dtype=torch.int32, device=DEV)
    g2l = torch.arange(e, dtype=torch.int32, device=DEV)
    d2 = ops.dispatch(idx2, valid, e, table, n_rep, False, None, 0, g2l, e, route_counts=rc2)
    M = int(d2.offsets[-1])
    assert torch.equal(idx, idx2) and torch.equal(gate, gate2)
    assert torch.equal(d.counts, d2.counts) and torch.equal(d.offsets, d2.offsets)
    assert torch.equal(d.perm[:M], d2.perm[:M]) and torch.equal(d.row_of_entry[: n * 8], d2.row_of_entry[: n * 8])
    assert torch.equal(rc1, rc2)


def _route_vs_two_calls(x, w, valid):
    e = w.shape[0]
    n = x.shape[0]
    rc1 = torch.zeros(e, dtype=torch.int64, device=DEV)
    rc2 = torch.zeros(e, dtype=torch.int64, device=DEV)
    idx, gate, d = ops.route_dispatch(x, w, 8, valid, route_counts=rc1)
    idx2, gate2 = ops.router_topk(x, w, 8)
    d2 = ops.dispatch(idx2, valid, e, torch.zeros(e, 1, dtype=torch.int32, device=DEV),
                      torch.ones(e, dtype=torch.int32, device=DEV), False, None, 0,
                      torch.arange(e, dtype=torch.int32, device=DEV), e, route_counts=rc2)
    M = int(d2.offsets[-1])
    assert torch.equal(idx, idx2) and torch.equal(gate, gate2)
    assert torch.equal(d.counts, d2.counts) and torch.equal(d.offsets, d2.offsets)
    assert torch.equal(d.perm[:M], d2.perm[:M]) and torch.equal(d.row_of_entry[: n * 8], d2.row_of_entry[: n * 8])
    assert torch.equal(rc1, rc2)
    return d


@pytest.mark.parametrize("hidden,n", [(2048, 3000), (4096, 1500), (4096, 64)])
def test_route_dispatch_fused_wide_hidden(hidden, n):
    """The fused route + dispatch at hidden 2048 and 4096 (two and four K
    segments of W_r per workgroup) equals the two calls bit for bit, and the
    stable grouping equals the oracle's."""
    banner(f"route_dispatch fused hidden={hidden} n={n}")
    g = torch.Generator().manual_seed(hidden + n)
    x = torch.randn(n, hidden, generator=g).to(torch.bfloat16).to(DEV)
    w = (0.02 * torch.randn(32, hidden, generator=g)).to(torch.bfloat16).to(DEV)
    valid = (torch.rand(n, generator=g) < 0.9).to(DEV)
    d = _route_vs_two_calls(x, w, valid)
    idx = to_np(ops.router_topk(x, w, 8)[0])
    vm = to_np(valid).astype(bool)
    ref = O.dispatch(idx, vm, 32, np.zeros((32, 1), np.int64), np.ones(32, np.int64), np.zeros((1, 32), np.int64),
                     [0, n], 0, np.arange(32))
    M = int(ref["offsets"][-1])
    assert to_np(d.counts).tolist() == ref["counts"].tolist()
    assert to_np(d.offsets).tolist() == ref["offsets"].tolist()
    assert to_np(d.perm)[:M].tolist() == ref["perm"].tolist()
    assert to_np(d.row_of_entry)[: n * 8].tolist() == ref["row_of_entry"].tolist()


@pytest.mark.parametrize("n", [32, 5000])
def test_route_dispatch_fused_logits(n):
    """The fused route + dispatch's optional fp32 logits output equals the
    router's (one workgroup and many)."""
    banner(f"route_dispatch fused logits n={n}")
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, 1024, generator=g).to(torch.bfloat16).to(DEV)
    w = (0.02 * torch.randn(32, 1024, generator=g)).to(torch.bfloat16).to(DEV)
    idx, gate, d, logits = ops.route_dispatch(x, w, 8, return_logits=True)
    idx2, gate2, logits2 = ops.router_topk(x, w, 8, return_logits=True)
    assert torch.equal(idx, idx2) and torch.equal(gate, gate2) and torch.equal(logits, logits2)


def test_route_dispatch_graph_replay():
    """Captured in a HIP graph (the fused launch, one workgroup and 64), every
    replay equals the eager call, with eager calls on other inputs in
    between (the epoch advances on every replay)."""
    banner("route_dispatch graph replay")
    g = torch.Generator().manual_seed(5)
    for n in (32, 4096):
        xs = [torch.randn(n, 1024, generator=g).to(torch.bfloat16).to(DEV) for _ in range(2)]
        w = (0.02 * torch.randn(32, 1024, generator=g)).to(torch.bfloat16).to(DEV)
        x = xs[0].clone()
        ref = ops.route_dispatch(x, w, 8, check=False)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ops.route_dispatch(x, w, 8, check=False)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                out = ops.route_dispatch(x, w, 8, check=False)
        torch.cuda.current_stream().wait_stream(side)
        for rep in range(3):
            x.copy_(xs[rep % 2])
            want = ops.route_dispatch(x, w, 8, check=False)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out[0], want[0]) and torch.equal(out[1], want[1]), (n, rep)
            assert torch.equal(out[2].offsets, want[2].offsets) and torch.equal(out[2].perm, want[2].perm), (n, rep)
        del ref


def test_route_dispatch_epoch_and_reuse():
    """The fused call's epoch (workspace header word 32) advances once per
    call of more than one workgroup, and one zero-filled workspace serves
    calls of different sizes in any order (fused, two-kernel and one-workgroup
    calls interleaved) with the two calls' bits every time."""
    banner("route_dispatch epoch and workspace reuse")
    from miniep_amd import _lib
    L = _lib.lib()
    e, hid = 32, 1024
    g = torch.Generator().manual_seed(11)
    big = 40000
    ws = torch.zeros(L.mep_route_dispatch_workspace_size(big, e), dtype=torch.uint8, device=DEV)
    words = ws[:256].view(torch.int32)
    w = (0.02 * torch.randn(e, hid, generator=g)).to(torch.bfloat16).to(DEV)
    s = torch.cuda.current_stream().cuda_stream
    epoch = 0
    for n in (4096, 16384, 40000, 32, 4096, 700, 16384):
        x = torch.randn(n, hid, generator=g).to(torch.bfloat16).to(DEV)
        idx = torch.empty(n, 8, dtype=torch.int64, device=DEV)
        gate = torch.empty(n, 8, dtype=torch.bfloat16, device=DEV)
        counts = torch.empty(e, dtype=torch.int32, device=DEV)
        offsets = torch.empty(e + 1, dtype=torch.int32, device=DEV)
        perm = torch.empty(n * 8, dtype=torch.int32, device=DEV)
        row = torch.empty(n * 8, dtype=torch.int32, device=DEV)
        assert L.mep_route_dispatch(x.data_ptr(), w.data_ptr(), None, n, hid, e, 8, 1, idx.data_ptr(),
                                    gate.data_ptr(), None, counts.data_ptr(), offsets.data_ptr(), perm.data_ptr(),
                                    row.data_ptr(), None, ws.data_ptr(), ws.numel(), s) == 0
        assert L.mep_dispatch_check(ws.data_ptr(), s) == 0
        nb = (n + 63) // 64
        if 1 < nb <= 512:
            epoch += 1
        assert int(words[32]) == epoch, (n, int(words[32]), epoch)
        idx2, _ = ops.router_topk(x, w, 8)
        d2 = ops.dispatch(idx2, None, e, torch.zeros(e, 1, dtype=torch.int32, device=DEV),
                          torch.ones(e, dtype=torch.int32, device=DEV), False, None, 0,
                          torch.arange(e, dtype=torch.int32, device=DEV), e)
        assert torch.equal(idx, idx2) and torch.equal(offsets, d2.offsets), n
        assert torch.equal(perm, d2.perm[: n * 8]) and torch.equal(row, d2.row_of_entry[: n * 8]), n
