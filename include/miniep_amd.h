/*
 * miniep_amd.h -- C ABI of the MI355X (gfx950) MoE-block hot path.
 *
 * The reference (mini-EP) runs the GraniteMoE MoE block as PyTorch CPU ops
 * behind a per-layer "MoE backend" callable
 *     backend(x_flat (N,H), topk_idx (N,k) int64, topk_gate (N,k), valid_mask (N,) bool|None) -> (N,H)
 * (miniep/modeling.py:131-145, used at :196; the expert-parallel drop-in is
 * miniep/ep.py:186-249) with the router inline in Block.forward
 * (miniep/modeling.py:192-195).  This library replaces the arithmetic of that
 * seam with four hand-written HIP kernel groups:
 *
 *   mep_router_topk     router GEMV + top-k + softmax      modeling.py:192-195
 *   mep_topk_softmax    top-k + softmax from fp32 logits   modeling.py:194-195
 *   mep_dispatch        flatten + histogram + stable rank  modeling.py:94-96,107-117
 *                       + replica round-robin + rank share ep.py:76-96,203-231
 *   mep_grouped_swiglu  run_experts (gather, GEMM-1,       modeling.py:83-104
 *                       SiLU*up, GEMM-2, scatter); also as
 *                       mep_swiglu_gate_up + mep_swiglu_down
 *   mep_combine         gate * y, slot-order sum           modeling.py:120-128,144
 *   mep_grouped_swiglu_combine   the last two in one call (one launch for
 *                       small bf16 top-8 batches)          modeling.py:98-104,120-128,144
 *
 * Conventions
 *  - Every pointer argument is DEVICE memory unless marked "host".
 *  - The library never allocates: buffers, including workspaces, come from
 *    the caller (size queries below).
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *    No call synchronises the stream except mep_dispatch_check().
 *  - Every call returns 0 on success or a negative MEP_ERR_* code; the message
 *    of the last failure on the calling thread is in mep_last_error().
 *  - Layouts are row-major and dense.  Expert weights follow the checkpoint
 *    layout (miniep/weights.py:17-26): w_in (E_local, 2I, H) = [gate rows | up
 *    rows], w_out (E_local, H, I), local experts in sorted global-id order
 *    (miniep/weights.py:54-58).
 *  - Flat entry id of token t, slot s is f = t*k + s (modeling.py:107-117).
 */
#ifndef MINIEP_AMD_H
#define MINIEP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of activations / weights / gates / outputs */
#define MEP_DTYPE_F32 0
#define MEP_DTYPE_BF16 1

/* return codes */
#define MEP_OK 0
#define MEP_ERR_INVALID_ARG (-1)      /* null pointer, negative size, bad dtype   */
#define MEP_ERR_UNSUPPORTED (-2)      /* shape outside what the kernels support  */
#define MEP_ERR_WORKSPACE (-3)        /* workspace smaller than the size query    */
#define MEP_ERR_EXPERT_RANGE (-4)     /* topk_idx outside [0, n_experts)           */
#define MEP_ERR_NOT_RESIDENT (-5)     /* entry routed here for a non-resident expert (ep.py:230) */
#define MEP_ERR_HIP (-6)              /* HIP runtime error (launch, sync)          */

/* Message of the last failing call on this thread ("" if none). */
const char* mep_last_error(void);

/* ABI version of this header (bumped on incompatible changes). */
int mep_abi_version(void);

/* ------------------------------------------------------------------------
 * Router: logits = x @ w_router^T, top-k (descending; equal logits: lower
 * expert id first), gate = softmax over the k selected logits in fp32,
 * stored in `dtype`.  Replaces modeling.py:193-195.  The logits are
 * accumulated in fp32 for both dtypes (the reference accumulates in x.dtype);
 * they are written to `logits` (N, E) fp32 when it is non-NULL.
 *   x         (N, H) dtype          w_router (E, H) dtype
 *   topk_idx  (N, k) int64          topk_gate (N, k) dtype
 * Supported: E in {16, 32, 64}, 1 <= k <= E, H % 256 == 0.
 * ---------------------------------------------------------------------- */
int mep_router_topk(const void* x, const void* w_router, int64_t n_tokens,
                    int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype,
                    int64_t* topk_idx, void* topk_gate, float* logits, void* stream);

/* Top-k + softmax of precomputed fp32 logits (N, E); the selection rule of
 * mep_router_topk.  Replaces modeling.py:194-195.  E <= 256, 1 <= k <= min(E, 32). */
int mep_topk_softmax(const float* logits, int64_t n_tokens, int32_t n_experts,
                     int32_t top_k, int32_t gate_dtype, int64_t* topk_idx,
                     void* topk_gate, void* stream);

/* ------------------------------------------------------------------------
 * Dispatch: this GPU's share of the routed entries, stably grouped by local
 * expert.  Replaces flatten_topk (modeling.py:107-117), the stable argsort /
 * unique_consecutive of run_experts (modeling.py:94-96), Placement.dest_ranks
 * (ep.py:76-96) and the receive side of EPMoEBackend (ep.py:216-231).
 *
 * The N tokens are the concatenation of S source segments (host array
 * seg_tokens[0..S], seg_tokens[0] = 0, seg_tokens[S] = N): segment s is what
 * source rank s sends, with its own round-robin counters rr[s, :] (each
 * source owns a Placement, ep.py:27-33).  S = 1 is one rank's own dispatch;
 * world = 1 with table = 0, g2l = identity is LocalMoEBackend.
 *
 *   topk_idx    (N, k) int64            valid_mask (N,) uint8 or NULL (= all valid)
 *   table       (E, rmax) int32  table[e, j] = rank of e's j-th replica (ep.py:35-45), rmax <= 32
 *   n_rep       (E,) int32       >= 1
 *   has_replicas  0 iff every n_rep[e] == 1; then dest = table[e, 0] and rr
 *                 is neither read nor written (ep.py:84-85)
 *   rr          (S, E) int64 in/out, may be NULL iff has_replicas == 0;
 *               rr[s, e] += #entries of expert e in segment s (ep.py:95)
 *   my_rank     entries with dest == my_rank are kept
 *   g2l         (E,) int32 global -> local expert id, -1 if not resident
 *   n_local     number of local experts (rows of w_in / w_out)
 * Outputs:
 *   counts      (n_local,) int32  rows per local expert
 *   offsets     (n_local + 1,) int32 exclusive prefix of counts
 *   perm        (N*k,) int32  perm[row] = flat entry id, rows [0, offsets[n_local])
 *   row_of_entry(N*k,) int32  row of each entry here, -1 if invalid / elsewhere
 *   dest        (N*k,) int32 or NULL: destination rank, -1 for invalid tokens
 *   route_counts(E,) int64 or NULL: += per-expert valid-entry counts (ep.py:216-217)
 * Invalid expert ids are dropped and recorded; kept entries of non-resident
 * experts are dropped and recorded (ep.py:230 asserts); mep_dispatch_check()
 * reports them.  Supported: 1 <= k <= 32, E <= 256, S <= 16, N*k < 2^31.
 * When its ceil(N*k / 512) blocks fit on the device at once (and there are
 * at most 512), the dispatch is ONE launch whose blocks exchange their
 * per-expert counts through the workspace, tagged with an epoch kept in the
 * workspace header: the workspace must be zero-filled once when it is
 * allocated and then reused as is (calls of any size); calls that overlap in
 * time (different streams) need different workspaces.  Otherwise it runs as
 * a count launch and a scatter launch (and a prefix launch above 512 blocks).
 * ---------------------------------------------------------------------- */
size_t mep_dispatch_workspace_size(int64_t n_tokens, int32_t top_k, int32_t n_experts,
                                   int32_t n_segments, const int64_t* seg_tokens /* host */);

int mep_dispatch(const int64_t* topk_idx, const uint8_t* valid_mask, int64_t n_tokens,
                 int32_t top_k, int32_t n_experts,
                 const int32_t* table, const int32_t* n_rep, int32_t rmax,
                 int32_t has_replicas, int64_t* rr,
                 const int64_t* seg_tokens /* host */, int32_t n_segments,
                 int32_t my_rank, const int32_t* g2l, int32_t n_local,
                 int32_t* counts, int32_t* offsets, int32_t* perm,
                 int32_t* row_of_entry, int32_t* dest, int64_t* route_counts,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Synchronises `stream` and returns MEP_ERR_EXPERT_RANGE / MEP_ERR_NOT_RESIDENT
 * if the last mep_dispatch on `workspace` dropped entries, MEP_ERR_INVALID_ARG
 * if some n_rep[e] lay outside [1, rmax] (the kernels then clamp it), else
 * MEP_OK. */
int mep_dispatch_check(const void* workspace, void* stream);

/* Status bits of mep_dispatch_noalloc (and of the conditions mep_dispatch_check reports). */
#define MEP_DISPATCH_STATUS_RANGE 1u          /* an expert id outside [0, n_experts) was dropped      */
#define MEP_DISPATCH_STATUS_NOT_RESIDENT 2u   /* an entry for a non-resident expert was dropped      */
#define MEP_DISPATCH_STATUS_REPLICAS 4u       /* some n_rep[e] lies outside [1, rmax]                 */
#define MEP_DISPATCH_STATUS_BARRIER 8u        /* mep_route_dispatch: a workgroup gave up waiting     */

/* mep_dispatch without a workspace argument: it allocates nothing and takes
 * no workspace.  No counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * or harnesses that forbid hipMalloc).  Same arguments, kernels and results
 * as mep_dispatch; the workspace is a static device array of this library,
 * 2 MiB per GPU, held until the process ends, and its address is looked up
 * once per device on the first call there.  Calls whose workspace would
 * exceed 2 MiB (mep_dispatch_workspace_size) return MEP_ERR_UNSUPPORTED: e.g.
 * up to 2^21 entries (N*k) with 32 experts.  All calls on one GPU share that
 * array, so calls that overlap on one GPU (different streams) race: serialise
 * them.  `status` (device uint32, may be NULL) receives the OR of the
 * MEP_DISPATCH_STATUS_* conditions of this call, written by the kernels
 * (mep_dispatch_check is not available for this form). */
int mep_dispatch_noalloc(const int64_t* topk_idx, const uint8_t* valid_mask, int64_t n_tokens,
                         int32_t top_k, int32_t n_experts,
                         const int32_t* table, const int32_t* n_rep, int32_t rmax,
                         int32_t has_replicas, int64_t* rr,
                         const int64_t* seg_tokens /* host */, int32_t n_segments,
                         int32_t my_rank, const int32_t* g2l, int32_t n_local,
                         int32_t* counts, int32_t* offsets, int32_t* perm,
                         int32_t* row_of_entry, int32_t* dest, int64_t* route_counts,
                         uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * Router + dispatch of the all-local backend, fused: mep_router_topk
 * followed by mep_dispatch with one segment and every expert on this GPU
 * (LocalMoEBackend: table 0, n_rep 1, g2l identity, n_local = E), the
 * modeling.py:193-196 router feeding modeling.py:94-96,107-117.  The router
 * kernel also counts each 64-token workgroup's entries per expert, which for
 * top_k = 8 is the dispatch's per-block histogram, so the dispatch runs one
 * launch fewer.  Outputs and the workspace check (mep_dispatch_check) are
 * those of the two calls, bit for bit; route_counts (E,) int64 or NULL:
 * += per-expert valid-entry counts.  Supported: top_k = 8, E in {16, 32, 64},
 * H % 256 == 0; other shapes use the two calls.
 * GraniteMoE's shape (bf16, E = 32, H in {1024, 2048, 4096}) runs as ONE
 * launch when its ceil(N / 64) workgroups fit on the device at once (e.g.
 * N <= 32768 on 256 CUs at hidden 1024): each workgroup publishes its
 * per-expert counts, reads everyone's and places its own entries.  The
 * published counts carry a per-call tag kept in the workspace, so the
 * workspace must be zero-filled once when it is allocated and then reused
 * as is; calls that overlap in time (different streams) need different
 * workspaces.  mep_dispatch_check reports MEP_ERR_HIP if a workgroup gave up
 * waiting for the others (they were not all resident).
 * ---------------------------------------------------------------------- */
size_t mep_route_dispatch_workspace_size(int64_t n_tokens, int32_t n_experts);

int mep_route_dispatch(const void* x, const void* w_router, const uint8_t* valid_mask, int64_t n_tokens,
                       int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype,
                       int64_t* topk_idx, void* topk_gate, float* logits,
                       int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* row_of_entry,
                       int64_t* route_counts, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Grouped SwiGLU experts over the dispatched rows (run_experts,
 * modeling.py:83-104), fused with the row gather (modeling.py:143) and the
 * scatter back to entry order:
 *   for row r of local expert e (offsets[e] <= r < offsets[e+1]):
 *     f = perm[r];  a = x[f / k]                         (gather)
 *     h = W_in[e] a;  act = silu(h[:I]) * h[I:]          (GEMM-1 + SwiGLU)
 *     y_entries[f] = W_out[e] act                        (GEMM-2 + scatter)
 * fp32 accumulation; act and y are stored in `dtype`.  Rows of entries that
 * are not dispatched here are left untouched.
 *   x (N, H)   w_in (n_local, 2I, H)   w_out (n_local, H, I)   y_entries (N*k, H)
 * max_rows >= offsets[n_local] (e.g. N*k) bounds the launch.
 * Supported: H % 256 == 0, I % 128 == 0.
 * With bf16, I % 256 == 0 and more than 2048 rows, both GEMMs run as ONE
 * persistent launch: each XCD works through its share of the row tiles, and
 * a row tile's GEMM-2 tiles start once its GEMM-1 tiles are done.  With at
 * most 1024 rows (decode) both small-batch GEMMs also run as one launch:
 * GEMM-2's workgroups load their weights while GEMM-1 runs and start on a
 * 32-row chunk once its GEMM-1 workgroups are done.
 * tile_queue: tile_queue_ints >= mep_experts_queue_ints(max_rows, n_local)
 * int32 of device memory, zero before the first call; the one-launch kernels
 * keep their schedule there (per-XCD tile counters, per-row-tile or
 * per-chunk GEMM-1 completion counts) and every launch leaves it zero again,
 * except word 10: sticky error flags that mep_experts_check reports (a
 * GEMM-2 tile that gave up waiting for its rows after about a second, or the
 * combine of mep_grouped_swiglu_combine for GEMM-2's, a queue that no
 * workgroup drained; either means the results are invalid).  Launches that may run at
 * the same time (on different streams) need different queues; launches on
 * one stream can share one.  No counterpart in the reference (its experts
 * are a Python loop).
 * ---------------------------------------------------------------------- */
size_t mep_experts_queue_ints(int64_t max_rows, int32_t n_local);

/* Synchronises `stream`, then reads tile_queue's error flags:
 * MEP_OK, or MEP_ERR_HIP with the reason in mep_last_error(). */
int mep_experts_check(const int32_t* tile_queue, void* stream);

size_t mep_experts_workspace_size(int64_t max_rows, int32_t inter, int32_t dtype);

int mep_grouped_swiglu(const void* x, int64_t n_tokens, int32_t top_k,
                       const int32_t* perm, const int32_t* offsets, int32_t n_local,
                       int64_t max_rows, const void* w_in, const void* w_out,
                       int32_t hidden, int32_t inter, int32_t dtype, void* y_entries,
                       void* workspace, size_t workspace_bytes, int32_t* tile_queue,
                       size_t tile_queue_ints, void* stream);

/* The two launches of mep_grouped_swiglu as separate calls, for callers that
 * schedule or time them individually (same kernels, same results):
 *   mep_swiglu_gate_up  GEMM-1 + SwiGLU: act[r] = silu(W_g x) * (W_u x), x = x[perm[r]/k]
 *                       act (max_rows, inter) in `dtype`, act_bytes >= max_rows*inter*elem
 *   mep_swiglu_down     GEMM-2 + scatter: y_entries[perm[r]] = W_out act[r]
 * Replace modeling.py:101-102 and :103 respectively. */
int mep_swiglu_gate_up(const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                       const int32_t* offsets, int32_t n_local, int64_t max_rows,
                       const void* w_in, int32_t hidden, int32_t inter, int32_t dtype,
                       void* act, size_t act_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                       void* stream);

int mep_swiglu_down(const void* act, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                    const int32_t* offsets, int32_t n_local, int64_t max_rows,
                    const void* w_out, int32_t hidden, int32_t inter, int32_t dtype,
                    void* y_entries, int32_t* tile_queue, size_t tile_queue_ints, void* stream);

/* Expert weight slots (the live re-slice of server.py:51-62 / weights.py:37-61
 * without re-reading a checkpoint for experts that stay):
 *   mep_grouped_swiglu_slots  mep_grouped_swiglu with local expert j's weights
 *                             in slot w_slot[j] of w_in (n_slots, 2I, H) /
 *                             w_out (n_slots, H, I); w_slot (n_local,) int32
 *                             device.  Same kernels and results.
 *   mep_copy_experts          for i < n: slot dst_slot[i] of (dst_in, dst_out)
 *                             = expert src_index[i] of (src_in, src_out), both
 *                             in the layouts above (src: n_src experts in
 *                             device memory, e.g. this layer's checkpoint
 *                             tensors kept in HBM).  src_index / dst_slot
 *                             are host arrays, checked
 *                             before anything is enqueued; a slot may be named
 *                             once per call. */
int mep_grouped_swiglu_slots(const void* x, int64_t n_tokens, int32_t top_k,
                             const int32_t* perm, const int32_t* offsets, int32_t n_local,
                             int64_t max_rows, const void* w_in, const void* w_out,
                             const int32_t* w_slot, int32_t hidden, int32_t inter, int32_t dtype,
                             void* y_entries, void* workspace, size_t workspace_bytes,
                             int32_t* tile_queue, size_t tile_queue_ints, void* stream);

/*
 * mep_grouped_swiglu_combine: mep_grouped_swiglu followed by mep_combine, the
 * expert half of LocalMoEBackend.__call__ (modeling.py:98-104 run_experts,
 * :120-128 scatter_combine, :144 the gate multiply) in one call.  Arguments
 * are those of the two calls; max_rows must be n_tokens * top_k (every
 * (token, slot) cell of y_entries), out is (n_tokens, H) like mep_combine's.
 * For bf16, top-8 and at most 1024 rows (decode) the small-batch launch of
 * both GEMMs ends with the combine: extra workgroups wait (bounded) until
 * every GEMM-2 workgroup's y stores are complete, then sum in slot order, so
 * the results equal the two calls' bit for bit with one launch fewer.  Other
 * sizes and dtypes make the two calls.  Schedule words 12 and 13 of
 * `tile_queue` serve the combine and are left at zero.
 */
int mep_grouped_swiglu_combine(const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                               const int32_t* offsets, const int32_t* row_of_entry,
                               const void* topk_gate, const uint8_t* valid_mask, int32_t n_local,
                               int64_t max_rows, const void* w_in, const void* w_out, int32_t hidden,
                               int32_t inter, int32_t dtype, void* y_entries, void* workspace,
                               size_t workspace_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                               void* out, void* stream);

int mep_copy_experts(const void* src_in, const void* src_out, int32_t n_src,
                     void* dst_in, void* dst_out, int32_t n_slots,
                     const int32_t* src_index /* host */, const int32_t* dst_slot /* host */,
                     int32_t n, int32_t hidden, int32_t inter, int32_t dtype, void* stream);

/* ------------------------------------------------------------------------
 * Combine: out[t] = sum_{s=0..k-1, row_of_entry[t*k+s] >= 0} gate[t,s] * y_entries[t*k+s]
 * summed in slot order in fp32, stored in `dtype`; invalid tokens give 0.
 * Replaces the gate multiply (modeling.py:144 / ep.py:241) and
 * scatter_combine (modeling.py:120-128).
 *   y_entries (N*k, H)  topk_gate (N, k)  row_of_entry (N*k,) int32  out (N, H)
 * Supported: H % 8 == 0 (bf16) / H % 4 == 0 (fp32).
 * ---------------------------------------------------------------------- */
int mep_combine(const void* y_entries, const void* topk_gate, const int32_t* row_of_entry,
                const uint8_t* valid_mask, int64_t n_tokens, int32_t top_k,
                int32_t hidden, int32_t dtype, void* out, void* stream);

/* ------------------------------------------------------------------------
 * Expert-parallel send side (one GPU's part; the all-to-all itself is the
 * caller's collective).
 *
 * mep_gather_rows: the send buffer, x_flat[token_ids[order]] (ep.py:226):
 *   out[i, :] = x[perm[i] / top_k, :]   for i < n_rows
 * and, when topk_idx / ids_out are given, the experts that travel with them
 * (ep.py:225, flat_expert[order]): ids_out[i] = topk_idx_flat[perm[i]].
 * `perm` is the destination-sorted entry order, i.e. mep_dispatch run over
 * `dest` as the key (world-1 tables, n_experts = world): its `counts` are the
 * send counts (ep.py:222) and its `row_of_entry` the inverse order (ep.py:239).
 *   x (N, H)  perm (n_rows,) int32  topk_idx (N*k,) int64 or NULL
 *   ids_out (n_rows,) int64 or NULL  out (n_rows, H)
 *
 * mep_combine_rows: the return path, gated = back[inv] * gate followed by
 * scatter_combine (ep.py:237-242):
 *   out[t] = sum_{s, row_of_entry[t*k+s] >= 0} gate[t,s] * y_rows[row_of_entry[t*k+s]]
 * in slot order in fp32 (the same reduction as mep_combine, rows read
 * through row_of_entry).
 *   y_rows (rows, H)  topk_gate (N, k)  row_of_entry (N*k,) int32  out (N, H)
 * ---------------------------------------------------------------------- */
int mep_gather_rows(const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                    int64_t n_rows, int32_t hidden, int32_t dtype, const int64_t* topk_idx,
                    int64_t* ids_out, void* out, void* stream);

int mep_combine_rows(const void* y_rows, const void* topk_gate, const int32_t* row_of_entry,
                     const uint8_t* valid_mask, int64_t n_tokens, int32_t top_k,
                     int32_t hidden, int32_t dtype, void* out, void* stream);

/* ------------------------------------------------------------------------
 * The whole MoE block of the all-local backend for one batch: the router
 * hook and the backend call of Block.forward (modeling.py:192-196), i.e.
 * mep_route_dispatch followed by mep_grouped_swiglu_combine, with the outputs
 * of both (topk_idx, topk_gate, logits if non-NULL, counts, offsets, perm,
 * row_of_entry, route_counts += if non-NULL, y_entries, out) bit for bit.
 * Decode batches of GraniteMoE's shape (bf16, 32 experts, top-8, 1..32
 * tokens, hidden 1024 / 2048 / 4096, inter % 256 == 0) run as ONE launch:
 * one workgroup routes while the expert workgroups already stream their
 * weights, and the last GEMM-2 workgroup of each column block combines it
 * (tile_queue_ints >= mep_moe_layer_queue_ints(...) words, zero before the
 * first call; mep_experts_check reports a wait that gave up).  Other shapes
 * make the two calls.  Workspaces: dispatch_ws as mep_route_dispatch's
 * (zero-filled once), experts_ws as mep_grouped_swiglu's.
 * ---------------------------------------------------------------------- */
size_t mep_moe_layer_queue_ints(int64_t n_tokens, int32_t n_experts, int32_t hidden);

int mep_moe_layer(const void* x, const void* w_router, const uint8_t* valid_mask, int64_t n_tokens,
                  int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype, const void* w_in,
                  const void* w_out, int32_t inter, int64_t* topk_idx, void* topk_gate, float* logits,
                  int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* row_of_entry,
                  int64_t* route_counts, void* y_entries, void* dispatch_ws, size_t dispatch_ws_bytes,
                  void* experts_ws, size_t experts_ws_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                  void* out, void* stream);

/* ------------------------------------------------------------------------
 * Test hook, no counterpart in the reference: makes one of the bounded waits
 * of the one-launch kernels give up, so that tests can drive the give-up
 * path from the host (every wait still ends, every kernel exits).  While a
 * site is set, launches of that kind use `polls` as their poll limit and:
 *   MEP_GIVEUP_DISPATCH  the last workgroup of a one-launch dispatch
 *                        (mep_dispatch, mep_route_dispatch) withholds its
 *                        per-expert counts, so every workgroup gives up;
 *   MEP_GIVEUP_ROWS      GEMM-2 tiles of row tile 0 of the tiled one-launch
 *                        experts wait for one GEMM-1 count more than exists;
 *   MEP_GIVEUP_CHUNK     GEMM-2 workgroups of chunk 0 of the small-batch one
 *                        launch wait for one GEMM-1 count more than exists;
 *   MEP_GIVEUP_COMBINE   combine workgroup 0 of the small-batch launch that
 *                        ends with the combine waits for one GEMM-2
 *                        workgroup more than exists;
 *   MEP_GIVEUP_ROUTED    the first GEMM workgroup of mep_moe_layer's one
 *                        launch waits for the routing to be counted twice
 *                        (its give-up makes every output of the call NaN);
 *                        MEP_GIVEUP_CHUNK applies to that launch too (the
 *                        GEMM-2 workgroups of expert 0).
 * A give-up is reported as in normal operation (mep_dispatch_check,
 * mep_experts_check) and poisons what the caller consumes: a dispatch sets
 * offsets[n_local] = -1 and every row_of_entry to -2 (the experts kernels then
 * run no tile, the combine writes NaN for such tokens); a GEMM-2 tile or
 * workgroup writes NaN rows; a combine workgroup writes NaN outputs.
 * MEP_GIVEUP_NONE (0) restores normal operation.  Process-wide setting, read
 * when a launch is enqueued; not for concurrent use.
 * ---------------------------------------------------------------------- */
#define MEP_GIVEUP_NONE 0
#define MEP_GIVEUP_DISPATCH 1
#define MEP_GIVEUP_ROWS 2
#define MEP_GIVEUP_CHUNK 3
#define MEP_GIVEUP_COMBINE 4
#define MEP_GIVEUP_ROUTED 5
int mep_test_force_giveup(int32_t site, int32_t polls);

#ifdef __cplusplus
}
#endif
#endif /* MINIEP_AMD_H */
