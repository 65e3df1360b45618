"""Grouped SwiGLU experts on the GPU (mep_grouped_swiglu) vs the oracle.

Bar: max |y - ref| <= 1e-5 * max |ref| (fp32) / 2e-2 * max |ref| (bf16 with
fp32 accumulation), on ragged per-expert row counts including empty experts
and counts around the 256-row tile edge.
"""
import numpy as np
import pytest
import torch

from helpers import TOL_BF16, TOL_F32, banner, rel_err, to_np
from miniep_amd import ops, workloads
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _world1(E):
    return (torch.zeros(E, 1, dtype=torch.int32, device=DEV), torch.ones(E, dtype=torch.int32, device=DEV),
            torch.arange(E, dtype=torch.int32, device=DEV))


def _topk_with_counts(counts, k, n, seed):
    """(n, k) routing whose per-expert entry counts are exactly `counts`."""
    E = len(counts)
    assert sum(counts) == n * k and max(counts) <= n
    rng = np.random.default_rng(seed)
    topk = np.full((n, k), -1, np.int64)
    fill = np.zeros(n, int)
    for e in np.argsort(-np.asarray(counts), kind="stable"):
        order = np.argsort(fill + rng.random(n) * 0.5, kind="stable")[: counts[e]]
        topk[order, fill[order]] = e
        fill[order] += 1
    assert (topk >= 0).all()
    return torch.from_numpy(topk)


def _run(x, topk, w_in, w_out, dtype):
    n, k = topk.shape
    E = w_in.shape[0]
    table, n_rep, g2l = _world1(E)
    xd = x.to(dtype).to(DEV)
    d = ops.dispatch(topk.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E)
    sentinel = torch.full((n * k, x.shape[1]), 7.0, dtype=dtype, device=DEV)
    y = ops.grouped_swiglu(xd, d, w_in.to(dtype).to(DEV), w_out.to(dtype).to(DEV), sentinel)
    return d, y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ragged_counts(dtype):
    banner(f"experts ragged {dtype}")
    E, k, n = 8, 2, 600
    counts = [0, 1, 255, 256, 257, 130, 301, 0]
    assert sum(counts) == n * k
    topk = _topk_with_counts(counts, k, n, 0)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(n, 1024, generator=g)
    w_in, w_out = workloads.expert_weights(g, E)
    d, y = _run(x, topk, w_in, w_out, dtype)
    assert to_np(d.counts).tolist() == counts
    xr = x.to(dtype).float().numpy()
    wi, wo = w_in.to(dtype).float().numpy(), w_out.to(dtype).float().numpy()
    bf = dtype == torch.bfloat16
    ref = O.experts(xr[np.repeat(np.arange(n), k)], topk.numpy().reshape(-1), wi, wo, act_bf16=bf, out_bf16=bf)
    err = rel_err(to_np(y), ref)
    print(f"rel err {err:.3e}")
    assert err <= (TOL_BF16 if bf else TOL_F32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_untouched_rows_and_masks(dtype):
    banner(f"experts masked {dtype}")
    E, k, n = 32, 8, 300
    g = torch.Generator().manual_seed(2)
    topk = torch.rand(n, E, generator=g).topk(k, -1).indices
    valid = torch.rand(n, generator=g) < 0.5
    x = torch.randn(n, 1024, generator=g)
    w_in, w_out = workloads.expert_weights(g, E)
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(topk.to(DEV), valid.to(DEV), E, table, n_rep, False, None, 0, g2l, E)
    y = torch.full((n * k, 1024), 7.0, dtype=dtype, device=DEV)
    ops.grouped_swiglu(x.to(dtype).to(DEV), d, w_in.to(dtype).to(DEV), w_out.to(dtype).to(DEV), y)
    yn = to_np(y)
    masked_rows = np.repeat(~valid.numpy(), k)
    assert (yn[masked_rows] == 7.0).all()
    bf = dtype == torch.bfloat16
    keep = np.repeat(valid.numpy(), k)
    ref = O.experts(x.to(dtype).float().numpy()[np.repeat(np.arange(n), k)][keep],
                    topk.numpy().reshape(-1)[keep], w_in.to(dtype).float().numpy(),
                    w_out.to(dtype).float().numpy(), act_bf16=bf, out_bf16=bf)
    assert rel_err(yn[keep], ref) <= (TOL_BF16 if bf else TOL_F32)


def test_skewed_full_size_sampled_rows():
    """T=16384 Zipf(1.2) bf16: every row computed; 2048 sampled rows vs oracle."""
    banner("experts skewed t=16384")
    L = workloads.make_layer(16384, seed=0, zipf_s=1.2)
    topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices
    d, y = _run(L.x, topk, L.w_in, L.w_out, torch.bfloat16)
    n, k = topk.shape
    rows = np.random.default_rng(0).choice(n * k, 2048, replace=False)
    xr = L.x.to(torch.bfloat16).float().numpy()
    ref = O.experts(xr[rows // k], topk.numpy().reshape(-1)[rows], L.w_in.to(torch.bfloat16).float().numpy(),
                    L.w_out.to(torch.bfloat16).float().numpy(), act_bf16=True, out_bf16=True)
    yn = to_np(y)
    assert rel_err(yn[rows], ref) <= TOL_BF16
    assert not (yn == 7.0).all(axis=1).any()          # every (token, slot) row written


def test_errors():
    banner("experts errors")
    E = 4
    table, n_rep, g2l = _world1(E)
    topk = torch.zeros(10, 2, dtype=torch.long)
    topk[:, 1] = 1
    d = ops.dispatch(topk.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E)
    x = torch.randn(10, 1024, device=DEV)
    with pytest.raises(ValueError):
        ops.grouped_swiglu(x, d, torch.randn(3, 1024, 1024, device=DEV), torch.randn(3, 1024, 512, device=DEV))
    with pytest.raises(RuntimeError, match="inter"):
        ops.grouped_swiglu(x, d, torch.randn(4, 200, 1024, device=DEV), torch.randn(4, 1024, 100, device=DEV))


def test_tile_queue_two_streams_and_repeats():
    """The tiled bf16 GEMMs schedule their tiles through a per-stream buffer
    of counters: launches on two streams at once and many launches in a row
    give the serial result bit for bit, and leave every word at zero."""
    banner("experts tile queue")
    outs = []
    cases = []
    for seed, T in ((3, 4096), (4, 3000)):
        L = workloads.make_layer(T, seed=seed, zipf_s=1.2)
        bf = torch.bfloat16
        x = L.x.to(bf).to(DEV)
        topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices.to(DEV)
        E = L.w_in.shape[0]
        table, n_rep, g2l = _world1(E)
        d = ops.dispatch(topk, None, E, table, n_rep, False, None, 0, g2l, E)
        cases.append((x, d, L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)))
    ref = [ops.grouped_swiglu(*c) for c in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ys = [torch.empty_like(r) for r in ref]
    torch.cuda.synchronize()
    for _ in range(5):
        for s, c, y in zip(streams, cases, ys):
            with torch.cuda.stream(s):
                ops.grouped_swiglu(*c, y)
        torch.cuda.synchronize()
        for y, r in zip(ys, ref):
            assert torch.equal(y, r)
    ops.experts_check()
    for q in ops._QUEUES.values():
        assert int(q.abs().sum()) == 0


def _two_launches(x, d, w_in, w_out, y):
    act = ops.swiglu_gate_up(x, d, w_in)
    return ops.swiglu_down(act, x, d, w_out, y)


def test_one_launch_consecutive_inputs_same_buffers():
    """The tiled one launch hands act from GEMM-1 tiles to GEMM-2 tiles that
    may run on other XCDs (device-scope act stores, GEMM-2 reads of lines its
    XCD has not cached in this launch).  Different inputs and routings, run
    back to back through the same act workspace, y buffer and schedule words
    (A, B, A, B), must each give the two launches' bits: an act line left over
    from the previous call would show here, where a repeated identical input
    would not."""
    banner("experts one launch: consecutive inputs through the same buffers")
    from miniep_amd import _lib
    bf = torch.bfloat16
    Lib = _lib.lib()
    n, k = 8192, 8
    cases = []
    for i in range(2):
        L = workloads.make_layer(n, seed=51 + i, zipf_s=1.2 if i == 0 else 0.6)
        topk = (L.x @ L.w_router.T).topk(k, dim=-1).indices
        E = L.w_in.shape[0]
        table, n_rep, g2l = _world1(E)
        d = ops.dispatch(topk.to(DEV), None, E, table, n_rep, False, None, 0, g2l, E)
        x, wi, wo = L.x.to(bf).to(DEV), L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
        ref = torch.full((n * k, 1024), 7.0, dtype=bf, device=DEV)
        _two_launches(x, d, wi, wo, ref)
        cases.append((x, d, wi, wo, ref))
    assert not torch.equal(cases[0][1].perm, cases[1][1].perm)
    max_rows = n * k
    ws = torch.empty(int(Lib.mep_experts_workspace_size(max_rows, 512, _lib.DTYPE_BF16)), dtype=torch.uint8,
                     device=DEV)
    tq = torch.zeros(int(Lib.mep_experts_queue_ints(max_rows, 32)), dtype=torch.int32, device=DEV)
    y = torch.empty((n * k, 1024), dtype=bf, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    for rep in range(4):
        x, d, wi, wo, ref = cases[rep % 2]
        y.fill_(7.0)
        rc = Lib.mep_grouped_swiglu(x.data_ptr(), n, k, d.perm.data_ptr(), d.offsets.data_ptr(), 32, max_rows,
                                    wi.data_ptr(), wo.data_ptr(), 1024, 512, _lib.DTYPE_BF16, y.data_ptr(),
                                    ws.data_ptr(), ws.numel(), tq.data_ptr(), tq.numel(), st)
        assert rc == 0
        _lib.check(Lib.mep_experts_check(tq.data_ptr(), st), "mep_experts_check")
        assert torch.equal(y, ref), rep
        assert int(tq.abs().sum()) == 0


@pytest.mark.parametrize("case", ["zipf_t16384", "tiny_t300", "ragged_e16", "e64_masked", "zipf_t40000"])
def test_one_launch_equals_two_launches(case):
    """bf16 with more than 2048 entries runs both GEMMs as one launch (each
    XCD's row tiles, GEMM-2 tiles waiting for their GEMM-1 rows).  It must
    give the two separate launches' bits on every dispatched row, leave the
    other rows alone, leave the schedule words at zero and flag nothing:
    many row tiles per XCD (the interleaved order), fewer row tiles than the
    lag (GEMM-1 first, then GEMM-2), ragged counts with empty experts and
    row halves, 64 experts with masked tokens."""
    banner(f"experts one launch vs two: {case}")
    bf = torch.bfloat16
    valid = None
    if case.startswith("zipf"):
        T = int(case.split("_t")[1])
        L = workloads.make_layer(T, seed=11, zipf_s=1.2)
        topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices
        x, w_in, w_out = L.x, L.w_in, L.w_out
    elif case == "tiny_t300":
        g = torch.Generator().manual_seed(12)
        topk = torch.rand(300, 32, generator=g).topk(8, -1).indices
        x = torch.randn(300, 1024, generator=g)
        w_in, w_out = workloads.expert_weights(g, 32)
    elif case == "ragged_e16":
        counts = [0, 1, 129, 256, 257, 6000, 6000, 5000, 3000, 2000, 1000, 357, 0, 0, 0, 0]
        topk = _topk_with_counts(counts, 4, 6000, 13)
        g = torch.Generator().manual_seed(13)
        x = torch.randn(6000, 1024, generator=g)
        w_in, w_out = workloads.expert_weights(g, 16)
    else:
        g = torch.Generator().manual_seed(14)
        topk = torch.rand(3000, 64, generator=g).topk(8, -1).indices
        valid = torch.rand(3000, generator=g) < 0.6
        x = torch.randn(3000, 1024, generator=g)
        w_in, w_out = workloads.expert_weights(g, 64)
    n, k = topk.shape
    E = w_in.shape[0]
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(topk.to(DEV), None if valid is None else valid.to(DEV), E, table, n_rep, False, None, 0, g2l, E)
    xd, wi, wo = x.to(bf).to(DEV), w_in.to(bf).to(DEV), w_out.to(bf).to(DEV)
    y1 = torch.full((n * k, 1024), 7.0, dtype=bf, device=DEV)
    y2 = y1.clone()
    for _ in range(3):                                   # repeated launches reuse the schedule words
        ops.grouped_swiglu(xd, d, wi, wo, y1)
    _two_launches(xd, d, wi, wo, y2)
    ops.experts_check()
    assert torch.equal(y1, y2)
    for q in ops._QUEUES.values():
        assert int(q.abs().sum()) == 0
    if case == "ragged_e16":
        xr = x.to(bf).float().numpy()
        ref = O.experts(xr[np.repeat(np.arange(n), k)], topk.numpy().reshape(-1), w_in.to(bf).float().numpy(),
                        w_out.to(bf).float().numpy(), act_bf16=True, out_bf16=True)
        err = rel_err(to_np(y1), ref)
        print(f"rel err vs oracle {err:.3e}")
        assert err <= TOL_BF16
    if valid is not None:
        assert (to_np(y1)[np.repeat(~valid.numpy(), k)] == 7.0).all()


@pytest.mark.parametrize("case", ["decode_t32", "zipf_t128", "masked_t100", "e64_t16", "h256_t32", "i1024_t24"])
def test_small_batch_one_launch_equals_two_launches(case):
    """Batches of at most 1024 (token, slot) entries run both small-batch
    GEMMs as one launch (GEMM-2's workgroups start loading their weights when
    their chunk's GEMM-1 workgroups near the end of their K loops, then wait
    for act).  Bits equal the two launches on every row, other rows are left
    alone, the schedule words return to zero, no wait gives up, and
    consecutive calls on other inputs (the same act workspace) give each
    input's own result.  h256: GEMM-1's K loop is one block of loads in
    flight (the early count at its start); i1024: GEMM-2 has weight steps
    past those held in LDS."""
    banner(f"experts small-batch one launch vs two: {case}")
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(21)
    E = 64 if case.startswith("e64") else 32
    n = int(case.split("_t")[1])
    H = 256 if case.startswith("h256") else 1024
    I = 256 if case.startswith("h256") else (1024 if case.startswith("i1024") else 512)
    valid = None
    if case.startswith("zipf"):
        L = workloads.make_layer(n, seed=21, zipf_s=1.2)
        topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices
        x, w_in, w_out = L.x, L.w_in, L.w_out
    else:
        topk = torch.rand(n, E, generator=g).topk(8, -1).indices
        x = torch.randn(n, H, generator=g)
        w_in, w_out = workloads.expert_weights(g, E, hidden=H, inter=I)
        if case.startswith("masked"):
            valid = torch.rand(n, generator=g) < 0.7
    k = 8
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(topk.to(DEV), None if valid is None else valid.to(DEV), E, table, n_rep, False, None, 0, g2l, E)
    if case == "zipf_t128":
        assert int(d.counts.max()) > 32                    # an expert of several 32-row chunks
    wi, wo = w_in.to(bf).to(DEV), w_out.to(bf).to(DEV)
    results = []
    for rep in range(2):                                   # a second input through the same buffers
        xd = (x if rep == 0 else torch.randn(x.shape, generator=g)).to(bf).to(DEV)
        y1 = torch.full((n * k, H), 7.0, dtype=bf, device=DEV)
        y2 = y1.clone()
        ops.grouped_swiglu(xd, d, wi, wo, y1)
        _two_launches(xd, d, wi, wo, y2)
        ops.experts_check()
        assert torch.equal(y1, y2), rep
        for q in ops._QUEUES.values():
            assert int(q.abs().sum()) == 0
        if valid is not None:
            assert (to_np(y1)[np.repeat(~valid.numpy(), k)] == 7.0).all()
        results.append(y1)
    assert not torch.equal(results[0], results[1])
    rows = np.repeat(np.arange(n), k)
    keep = np.ones(n * k, bool) if valid is None else np.repeat(valid.numpy(), k)
    ref = O.experts(xd.float().cpu().numpy()[rows[keep]], topk.numpy().reshape(-1)[keep], wi.float().cpu().numpy(),
                    wo.float().cpu().numpy(), act_bf16=True, out_bf16=True)
    assert rel_err(to_np(results[1])[keep], ref) <= TOL_BF16


@pytest.mark.parametrize("stride", [128, 16])
def test_small_batch_kernel_matches_main_kernel_bitwise(stride):
    """Batches of at most 2048 (token, slot) entries run the few-rows-per-expert
    kernel; larger ones the tiled kernel.  The same tokens as a small batch and
    inside a large batch with the other tokens masked give identical bits
    (stride 16: 256 tokens, Zipf-skewed, so the hottest expert needs several
    32-row passes)."""
    banner(f"experts small-batch kernel stride={stride}")
    bf = torch.bfloat16
    L = workloads.make_layer(4096, seed=6, zipf_s=1.2)
    x = L.x.to(bf).to(DEV)
    topk = (L.x @ L.w_router.T).topk(8, dim=-1).indices.to(DEV)
    E = L.w_in.shape[0]
    wi, wo = L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV)
    table, n_rep, g2l = _world1(E)
    sel = torch.arange(0, 4096, stride, device=DEV)
    n = sel.numel()
    d_small = ops.dispatch(topk[sel], None, E, table, n_rep, False, None, 0, g2l, E)
    assert n * 8 <= 2048
    if stride == 16:
        assert int(d_small.counts.max()) > 64          # several passes for the hottest expert
    y_small = ops.grouped_swiglu(x[sel], d_small, wi, wo)
    valid = torch.zeros(4096, dtype=torch.bool, device=DEV)
    valid[sel] = True
    d_big = ops.dispatch(topk, valid, E, table, n_rep, False, None, 0, g2l, E)
    y_big = torch.full((4096 * 8, 1024), 7.0, dtype=bf, device=DEV)
    ops.grouped_swiglu(x, d_big, wi, wo, y_big)
    assert torch.equal(y_small.view(n, 8, -1), y_big.view(4096, 8, -1)[sel])
    # and against the oracle
    rows = np.arange(n * 8)
    xr = x[sel].float().cpu().numpy()
    ref = O.experts(xr[rows // 8], to_np(topk[sel]).reshape(-1), wi.float().cpu().numpy(),
                    wo.float().cpu().numpy(), act_bf16=True, out_bf16=True)
    assert rel_err(to_np(y_small), ref) <= TOL_BF16


@pytest.mark.parametrize("H,I,E,k,n,dtype", [
    (256, 128, 8, 2, 700, torch.bfloat16),      # K = 256 (no steady steps); GEMM-2 on the generic kernel (I % 256)
    (512, 384, 16, 4, 600, torch.bfloat16),     # tiled GEMM-1, generic GEMM-2
    (2048, 256, 8, 8, 100, torch.bfloat16),     # 800 entries: small-batch kernels, K = 2048 / 256
    (768, 640, 12, 6, 1000, torch.bfloat16),    # 3 column tiles of GEMM-1, 5 of 128 gate columns
    (512, 256, 16, 4, 2000, torch.bfloat16),    # tiled kernels for both GEMMs, K = 512 / 256
    (256, 256, 8, 2, 300, torch.float32),       # fp32
])
def test_other_shapes_vs_oracle(H, I, E, k, n, dtype):
    banner(f"experts shape H={H} I={I} E={E} k={k} n={n} {dtype}")
    g = torch.Generator().manual_seed(H + I + E + k)
    x = torch.randn(n, H, generator=g)
    w_in, w_out = workloads.expert_weights(g, E, H, I)
    topk = torch.rand(n, E, generator=g).topk(k, -1).indices
    d, y = _run(x, topk, w_in, w_out, dtype)
    bf = dtype == torch.bfloat16
    xr = x.to(dtype).float().numpy()
    ref = O.experts(xr[np.repeat(np.arange(n), k)], topk.numpy().reshape(-1), w_in.to(dtype).float().numpy(),
                    w_out.to(dtype).float().numpy(), act_bf16=bf, out_bf16=bf)
    err = rel_err(to_np(y), ref)
    print(f"rel err {err:.3e}")
    assert err <= (TOL_BF16 if bf else TOL_F32)


@pytest.mark.parametrize("case", ["decode_t32", "masked_t100", "zipf_t128", "e64_t16", "h256_t32", "h2048_t40",
                                  "bf16_t3000", "f32_t32"])
def test_grouped_swiglu_combine_equals_two_calls(case):
    """mep_grouped_swiglu_combine: for small bf16 top-8 batches the
    small-batch launch ends with the combine (workgroups that wait for every
    GEMM-2 workgroup's y stores, then sum in combine8's order); other sizes
    and fp32 make the two calls.  The layer output equals grouped_swiglu +
    combine bit for bit, masked tokens included, on two inputs in a row
    through the same buffers, and the schedule words return to zero.
    h2048: 2048-wide rows and K = 1024 in GEMM-2 (weight steps past those in
    LDS)."""
    banner(f"experts + combine in one call vs two: {case}")
    dt = torch.float32 if case.startswith("f32") else torch.bfloat16
    g = torch.Generator().manual_seed(33)
    E = 64 if case.startswith("e64") else 32
    n = int(case.split("_t")[1])
    H = 256 if case.startswith("h256") else (2048 if case.startswith("h2048") else 1024)
    I = 256 if case.startswith("h256") else (1024 if case.startswith("h2048") else 512)
    valid = (torch.rand(n, generator=g) < 0.7) if case.startswith("masked") else None
    if case.startswith("zipf"):
        L = workloads.make_layer(n, seed=33, zipf_s=1.2)
        logits = L.x @ L.w_router.T
        x, w_in, w_out = L.x, L.w_in, L.w_out
    else:
        logits = torch.randn(n, E, generator=g)
        x = torch.randn(n, H, generator=g)
        w_in, w_out = workloads.expert_weights(g, E, hidden=H, inter=I)
    top = torch.softmax(logits, -1).topk(8, -1)
    topk, gate = top.indices, top.values
    table, n_rep, g2l = _world1(E)
    d = ops.dispatch(topk.to(DEV), None if valid is None else valid.to(DEV), E, table, n_rep, False, None, 0, g2l, E)
    wi, wo = w_in.to(dt).to(DEV), w_out.to(dt).to(DEV)
    gd = gate.to(dt).to(DEV)
    vd = None if valid is None else valid.to(DEV)
    outs = []
    for rep in range(2):
        xd = (x if rep == 0 else torch.randn(x.shape, generator=g)).to(dt).to(DEV)
        ref = ops.combine(ops.grouped_swiglu(xd, d, wi, wo), gd, d.row_of_entry, vd)
        got = ops.grouped_swiglu_combine(xd, d, wi, wo, gd, vd)
        ops.experts_check()
        assert torch.equal(got, ref), rep
        for q in ops._QUEUES.values():
            assert int(q.abs().sum()) == 0
        if valid is not None:
            assert (to_np(got)[~valid.numpy()] == 0).all()
        outs.append(got)
    assert not torch.equal(outs[0], outs[1])


def test_decode_layer_graph_replay():
    """HipMoEBackend.route_and_call at decode size (router + dispatch, then
    the small-batch experts launch that ends with the combine) captured in a
    HIP graph: every replay equals the eager call on the same input, with
    eager calls on other inputs in between, and the schedule words the
    launch's last workgroups return to zero stay zero."""
    banner("decode layer graph replay")
    from miniep_amd import HipMoEBackend
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(44)
    L = workloads.make_layer(32, seed=44)
    be = HipMoEBackend(L.w_in.to(bf).to(DEV), L.w_out.to(bf).to(DEV), check=False)
    w_r = L.w_router.to(bf).to(DEV)
    xs = [torch.randn(32, 1024, generator=g).to(bf).to(DEV) for _ in range(2)]
    x = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        be.route_and_call(x, w_r, 8)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = be.route_and_call(x, w_r, 8)[0]
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(4):
        x.copy_(xs[rep % 2])
        want = be.route_and_call(x, w_r, 8)[0].clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        be.route_and_call(xs[(rep + 1) % 2], w_r, 8)     # eager work on another input between replays
        torch.cuda.synchronize()
    ops.experts_check()
    for q in ops._QUEUES.values():
        assert int(q.abs().sum()) == 0
