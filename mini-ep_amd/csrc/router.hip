// Fused router for the GraniteMoE MoE block (gfx950).
//
// Replaces modeling.py:193-195:
//     router_logits = x_flat @ W_r.T
//     topk_logits, topk_idx = router_logits.topk(k, dim=-1)      (descending)
//     topk_gate = softmax(topk_logits.float(), dim=-1).to(x.dtype)
//
// One wavefront owns 16 tokens, four wavefronts share a workgroup and its LDS
// copy of W_r.  The 16 x E logit tile is computed on the matrix cores (bf16:
// v_mfma_f32_16x16x32_bf16, fp32: v_mfma_f32_16x16x4_f32) with fp32
// accumulation; each wave issues all loads of its x rows for a K segment
// before its first MFMA, so HBM latency is paid once per segment.
// The selection orders (token, expert) pairs by the total order
//     e' before e  <=>  key(e') > key(e)  or  (key(e') == key(e) and e' < e)
// (descending logits, lower expert id first among equal logits, NaN above
// every number, -0.0 == +0.0).  For 32 experts and top-8 the four lanes of a
// token sort their 8 keys each and merge them with sorting networks in
// registers; other shapes rank every pair (rank(e) = #{e' before e}) and put
// rank < k in output slot `rank`.  No atomics decide anything, so the
// selection is deterministic and independent of the launch shape.  With the
// dispatch histogram output (mep_route_dispatch) each workgroup also counts
// the entries per expert of its 64 tokens.
#include "common.h"
#include "router_dev.h"

#include <atomic>

namespace mep {
namespace {

template <int DT, int NF, int KC>
__global__ __launch_bounds__(kWaves * 64) void router_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                             const typename Elem<DT>::T* __restrict__ w,
                                                             int64_t n_tokens, int hidden, int k,
                                                             int64_t* __restrict__ topk_idx,
                                                             typename Elem<DT>::T* __restrict__ gate,
                                                             float* __restrict__ logits, RouterHist hist) {
  typedef typename Elem<DT>::T T;
  constexpr int E = NF * 16;
  constexpr int EB = Elem<DT>::kBytes;
  constexpr int kElemsPerChunk = 16 / EB;                 // 8 bf16 or 4 fp32
  constexpr int kBlockElems = 32 * kElemsPerChunk;        // 4 groups x 8 chunks = 512 B
  constexpr int kSegFit = (kSegBytes / (E * EB)) / kBlockElems * kBlockElems;
  constexpr int kSegElems = kSegFit < 4 * kBlockElems ? kSegFit : 4 * kBlockElems;   // <= 4 K blocks of x in VGPRs
  constexpr int kSegBlocks = kSegElems / kBlockElems;     // K blocks per segment
  constexpr int kRowStride = kSegElems * EB + 16;         // padded LDS row of W (bytes)
  static_assert(kSegBlocks >= 1 && kSegBlocks <= 4, "segment holds 1..4 K blocks");
  __shared__ __attribute__((aligned(16))) unsigned char ws[E * kRowStride];
  __shared__ float lg[kWaves][kRowsPerWave][E + 1];
  __shared__ __attribute__((aligned(16))) uint64_t keys[kWaves][kRowsPerWave * (E + 2)];
  __shared__ __attribute__((aligned(16))) float sel_val[kWaves][kRowsPerWave * 64];
  __shared__ int sel_idx[kWaves][kRowsPerWave * 64];
  __shared__ float rsum[kWaves][kRowsPerWave];
  __shared__ int s_cnt[E];                        // histogram output: entries per expert

  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  if (tid < E) s_cnt[tid] = 0;                    // published by the first barrier below
  const int r = lane & 15, g = lane >> 4;
  const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * kRowsPerWave;
  int64_t tok = t0 + r;
  if (tok >= n_tokens) tok = n_tokens - 1;   // in-bounds read, result discarded
  const T* xrow = x + tok * hidden + g * kElemsPerChunk;

  f32x4 acc[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) acc[nf] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int kCpr = kSegElems / kElemsPerChunk;                     // chunks per W row
  constexpr int kPerThread = E * kCpr / (kWaves * 64);
  static_assert((E * kCpr) % (kWaves * 64) == 0, "W segment splits evenly");
  // MFMAs of K block b: the block's weight fragments are all read from LDS
  // first (independent reads in flight together), then the MFMAs run on them
  auto block_mfmas = [&](const u32x4 (&xb)[8], int b) {
    u32x4 wb[8][NF];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int nf = 0; nf < NF; ++nf)
        wb[j][nf] = *reinterpret_cast<const u32x4*>(
            ws + (nf * 16 + r) * kRowStride + (b * kBlockElems + (4 * j + g) * kElemsPerChunk) * EB);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int nf = 0; nf < NF; ++nf) {
        if constexpr (DT == MEP_DTYPE_BF16) {
          acc[nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, xb[j]), __builtin_bit_cast(bf16x8, wb[j][nf]), acc[nf], 0, 0, 0);
        } else {
          const float* xf = reinterpret_cast<const float*>(&xb[j]);
          const float* wf = reinterpret_cast<const float*>(&wb[j][nf]);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[nf] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[q], wf[q], acc[nf], 0, 0, 0);
        }
      }
  };
  for (int seg = 0; seg < hidden; seg += kSegElems) {
    const int nblk = (hidden - seg) / kBlockElems < kSegBlocks ? (hidden - seg) / kBlockElems : kSegBlocks;
    const bool full = nblk == kSegBlocks;          // every block of the segment is real (H = 1024: always)
    // W_r[:, seg : seg + nblk*kBlockElems] first, then this wave's x rows: the
    // weight loads are waited for (LDS staging) before the x loads that follow
    // them, and the x blocks are then waited for one at a time
    const int live_cpr = nblk * kBlockElems / kElemsPerChunk;
    u32x4 wt[kPerThread];
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int c = tid + i * kWaves * 64, e = c / kCpr, q = c % kCpr;
      if (full || q < live_cpr)
        wt[i] = *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(e) * hidden + seg + q * kElemsPerChunk);
    }
    asm volatile("" ::: "memory");                 // keep the weight loads ahead of the x loads
    u32x4 xa[kSegBlocks][8];
#pragma unroll
    for (int b = 0; b < kSegBlocks; ++b)
      if (full || b < nblk)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          xa[b][j] = *reinterpret_cast<const u32x4*>(xrow + seg + b * kBlockElems + j * 4 * kElemsPerChunk);
    __syncthreads();                               // previous segment's readers are done
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int c = tid + i * kWaves * 64, e = c / kCpr, q = c % kCpr;
      if (full || q < live_cpr) *reinterpret_cast<u32x4*>(ws + e * kRowStride + q * 16) = wt[i];
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < kSegBlocks; ++b) {
      if (!full && b >= nblk) break;
      block_mfmas(xa[b], b);
    }
  }
  router_tail<DT, E, KC>(acc, lg[wave], keys[wave], sel_val[wave], sel_idx[wave], rsum[wave], s_cnt, t0, n_tokens, k,
                         topk_idx, gate, logits, hist);
}

template <int NSEG>
__global__ __launch_bounds__(kWaves * 64) void router32_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w, int64_t n_tokens,
                                                               int64_t* __restrict__ topk_idx,
                                                               uint16_t* __restrict__ gate,
                                                               float* __restrict__ logits, RouterHist hist) {
  constexpr int E = 32, KC = 8;
  __shared__ __attribute__((aligned(16))) unsigned char ws[E * kRowStride32];
  __shared__ float lg[kWaves][kRowsPerWave][E + 1];
  __shared__ int s_cnt[E];
  const int tid = threadIdx.x, wave = tid >> 6;
  if (tid < E) s_cnt[tid] = 0;                    // published by the first barrier of router32_logits
  const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * kRowsPerWave;
  f32x4 acc[2];
  router32_logits<NSEG>(x, w, n_tokens, t0, ws, acc);
  // the E = 32, top-8 selection runs in registers: no key / selection scratch
  router_tail<MEP_DTYPE_BF16, E, KC>(acc, lg[wave], nullptr, nullptr, nullptr, nullptr, s_cnt, t0, n_tokens, KC,
                                      topk_idx, gate, logits, hist);
}

// ---------------------------------------------------------------------------
// Router and dispatch of the all-local backend in one launch (GraniteMoE's
// shape: bf16, 32 experts, top-8).  Each workgroup routes its 64 tokens as
// router32_kernel does; its 512 entries are then one dispatch block.  It ranks
// them by flat entry id per expert inside the block (a token's 8 experts are
// distinct, so an entry's rank is the number of earlier tokens of the block
// that chose the same expert: wave ballots over the 5 id bits, then the waves'
// counts in order) and publishes its histogram row.  The expert totals
// (counts, offsets) and each block's prefix over earlier blocks place every
// entry:
//   row = offsets[e] + #(e in earlier blocks) + #(e earlier in this block),
// the stable grouping by expert of modeling.py:94-96: every workgroup reads
// every row (8 words of four 8-bit counts, 64 bytes) and takes the totals
// and its prefix over earlier blocks.  Results equal router32_kernel followed
// by the dispatch's scatter_kernel bit for bit.
//
// Every workgroup must be resident at once (the host launches at most as
// many as the device holds).  There is no counter and no atomic: each row
// word is a 64-bit (tag << 32 | count) written and read with device-scope
// (sc1) accesses, so a word written on one XCD is read fresh on every other,
// and a workgroup re-reads the words whose tag is not yet this call's.  The
// tag is 2^31 | (the workspace's epoch word + 1): every workgroup reads the
// epoch as it starts, and the last workgroup to finish advances it (by then
// every workgroup has read it).  Words of earlier calls
// carry older tags, and whatever else the library leaves in a workspace
// (counts, flags, table entries: small non-negative values) has a clear top
// bit, so the workspace must only be zero-filled once before its first use
// and can then serve calls of any size.  A wait longer than kRowPolls polls sets
// kFlagBarrier in the block's status word: the workgroup places nothing (its
// entries get kPoisonRow), every workgroup exits, the last one to finish
// poisons the whole call (finish_exchange) and mep_dispatch_check reports it.
constexpr int kRowPolls = 1 << 20;
constexpr int kRowWords = 8;                      // 64-bit words of a histogram row: 4 counts each

struct FusedDispatch {
  int32_t* counts;          // (E,) rows per expert
  int32_t* offsets;         // (E + 1,) exclusive prefix of counts
  int32_t* perm;            // (N k,) perm[row] = flat entry id
  int32_t* row_of_entry;    // (N k,) row of each entry, -1 for masked tokens
  int64_t* route_counts;    // (E,) += entries per expert, or NULL
  uint64_t* rows;           // (n_blocks, kRowWords) tagged histogram rows
  uint32_t* header;         // [0] = n_blocks; [kEpochWord]: the epoch
  uint32_t* flags;          // (2 n_blocks,) status words: count pass (0), scatter pass
  const uint8_t* valid;     // (N,) or NULL
  int polls;                // polls of a row before a workgroup gives up
  int withhold;             // workgroup that withholds its row (test hook; -1: none)
};

__device__ __forceinline__ uint32_t load_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NSEG>
__global__ __launch_bounds__(kWaves * 64) void route_dispatch32_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ w,
                                                                       int64_t n_tokens,
                                                                       int64_t* __restrict__ topk_idx,
                                                                       uint16_t* __restrict__ gate,
                                                                       float* __restrict__ logits, FusedDispatch o) {
  constexpr int E = 32, KC = 8;
  constexpr int kParts = kWaves * 64 / E;         // 8 threads per expert sum the histogram rows
  __shared__ __attribute__((aligned(16))) unsigned char ws[E * kRowStride32];
  __shared__ float lg[kWaves][kRowsPerWave][E + 1];
  __shared__ int s_wcnt[kWaves][E];               // entries of expert e in wave w of this block
  __shared__ int s_part[kParts][2][E];            // per part: entries in earlier blocks / in all blocks
  __shared__ int s_base[E];                       // first row of expert e's entries of this block
  __shared__ uint32_t s_flag;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int b = blockIdx.x, nb = gridDim.x;
  if (tid < kWaves * E) s_wcnt[tid / E][tid % E] = 0;   // published by the first barrier of router32_logits
  if (tid == 0) s_flag = 0u;
  const int64_t t0 = (static_cast<int64_t>(b) * kWaves + wave) * kRowsPerWave;
  // this call's tag; the load goes out before the router's loads and has
  // long landed when the tag is first used
  const uint32_t epoch = (load_dev(o.header + kEpochWord) + 1u) & 0x7fffffffu;
  const uint64_t tag = static_cast<uint64_t>(0x80000000u | epoch) << 32;
  asm volatile("" ::: "memory");
  f32x4 acc[2];
  router32_logits<NSEG>(x, w, n_tokens, t0, ws, acc);
  RouterHist hist{};
  hist.valid = o.valid;
  int sel[2];                                     // experts of this lane's two slots, -1: not dispatched
  router_tail<MEP_DTYPE_BF16, E, KC>(acc, lg[wave], nullptr, nullptr, nullptr, nullptr, nullptr, t0, n_tokens, KC,
                                      topk_idx, gate, logits, hist, sel);

  // 1. rank of each entry among the wave's entries of its expert (lane order =
  // token order; the two slots of a lane hold different experts)
  uint64_t bits0[5], bits1[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    bits0[i] = __ballot((sel[0] >> i) & 1);
    bits1[i] = __ballot((sel[1] >> i) & 1);
  }
  const uint64_t has0 = __ballot(sel[0] >= 0), has1 = __ballot(sel[1] >= 0);
  const uint64_t before = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int rank[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = sel[h];
    const uint64_t m = e >= 0 ? (lanes_with(e, bits0, has0) | lanes_with(e, bits1, has1)) : 0ull;
    rank[h] = __popcll(m & before);
    if (e >= 0 && rank[h] == 0) s_wcnt[wave][e] = __popcll(m);
  }
  __syncthreads();

  // 2. this block's histogram row, then every block's: rows bb = part + 8 u
  // of this thread's expert column, re-read until each carries this call's
  // tag (one workgroup: its own counts, nothing to publish)
  if (nb == 1) {
    const int e = tid % E, part = tid / E;
    int c = 0;
    if (part == 0)
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) c += s_wcnt[ww][e];
    s_part[part][0][e] = 0;
    s_part[part][1][e] = c;
  } else {
    // the row as kRowWords words: tag | four 8-bit counts (a block has at
    // most 64 tokens, so a count fits)
    if (tid < kRowWords && b != o.withhold) {
      uint32_t packed = 0u;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        int c = 0;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) c += s_wcnt[ww][4 * tid + q];
        packed |= static_cast<uint32_t>(c) << (8 * q);
      }
      store_dev(o.rows + static_cast<int64_t>(b) * kRowWords + tid, tag | packed);
    }
    // every block's row: thread (word j, part) reads rows part + 32 u of word
    // j, re-reading each until it carries this call's tag
    constexpr int kPartsW = kWaves * 64 / kRowWords;
    const int j = tid % kRowWords, part = tid / kRowWords;
    int pre[4] = {0, 0, 0, 0}, tot[4] = {0, 0, 0, 0};
    uint32_t bad = 0u;
    constexpr int kBatch = 8;
    for (int bb0 = part; bb0 < nb; bb0 += kPartsW * kBatch) {
      uint64_t v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int bb = bb0 + u * kPartsW;
        v[u] = bb < nb ? load_dev(o.rows + static_cast<int64_t>(bb) * kRowWords + j) : tag;
      }
      for (int it = 0;; ++it) {
        bool stale = false;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) stale |= (v[u] & ~0xffffffffull) != tag;
        if (!stale) break;
        if (it >= o.polls) { bad = kFlagBarrier; break; }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
          if ((v[u] & ~0xffffffffull) != tag)
            v[u] = load_dev(o.rows + static_cast<int64_t>(bb0 + u * kPartsW) * kRowWords + j);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int bb = bb0 + u * kPartsW;
        const uint32_t w = bb < nb ? static_cast<uint32_t>(v[u]) : 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = static_cast<int>((w >> (8 * q)) & 0xffu);
          tot[q] += c;
          pre[q] += bb < b ? c : 0;
        }
      }
    }
    // the wave's parts of word j (lanes j, j + 8, ..., j + 56), then the waves'
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int d = kRowWords; d < 64; d <<= 1) {
        pre[q] += __shfl_xor(pre[q], d, 64);
        tot[q] += __shfl_xor(tot[q], d, 64);
      }
    if (lane < kRowWords)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s_part[wave][0][4 * lane + q] = pre[q];
        s_part[wave][1][4 * lane + q] = tot[q];
      }
    if (bad) s_flag = bad;
    if (tid < E)                                   // no part beyond the waves'
#pragma unroll
      for (int q = kWaves; q < kParts; ++q) s_part[q][0][tid] = s_part[q][1][tid] = 0;
  }
  __syncthreads();
  // a workgroup whose wait gave up has rows of earlier calls: it places
  // nothing and leaves route_counts alone
  const bool gave_up = s_flag != 0u;
  if (tid < E) {
    int pre = 0, tot = 0;
#pragma unroll
    for (int q = 0; q < kParts; ++q) { pre += s_part[q][0][tid]; tot += s_part[q][1][tid]; }
    int incl = tot;                                // inclusive prefix over experts (lanes 0..31 of wave 0)
#pragma unroll
    for (int d = 1; d < E; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    const int off = incl - tot;
    s_base[tid] = off + pre;
    if (b == 0) {
      // device scope, as is the poison that may replace offsets[E]
      o.counts[tid] = tot;
      store_dev(reinterpret_cast<uint32_t*>(o.offsets + tid), static_cast<uint32_t>(off));
      if (tid == E - 1) store_dev(reinterpret_cast<uint32_t*>(o.offsets + E), static_cast<uint32_t>(incl));
      if (o.route_counts != nullptr && !gave_up) o.route_counts[tid] += tot;
    }
  }
  __syncthreads();

  // 3. rows of this lane's entries (row_of_entry with device-scope stores,
  // as is the poison that may replace it)
  const int t = lane >> 2, g = lane & 3;
  if (t0 + t < n_tokens) {
    const int64_t f = (t0 + t) * KC + g * 2;
    int row[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = sel[h];
      row[h] = gave_up ? kPoisonRow : -1;
      if (e >= 0 && !gave_up) {
        int r = s_base[e] + rank[h];
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) r += ww < wave ? s_wcnt[ww][e] : 0;
        row[h] = r;
        o.perm[r] = static_cast<int32_t>(f + h);
      }
    }
    store_dev(reinterpret_cast<uint64_t*>(o.row_of_entry + f),
              (static_cast<uint64_t>(static_cast<uint32_t>(row[1])) << 32) | static_cast<uint32_t>(row[0]));
  }
  if (tid == 0) {
    o.flags[b] = 0u;
    o.flags[nb + b] = s_flag;
    if (b == 0) o.header[0] = static_cast<uint32_t>(nb);
  }
  if (nb > 1) {
    // the last workgroup to finish poisons a call in which one gave up, and
    // advances the epoch (every workgroup has read it)
    __syncthreads();
    if (tid < 64) {
      const int r = finish_exchange(o.header, gave_up, nb);
      if (r & kExchangeGaveUp) poison_dispatch(o.row_of_entry, n_tokens * KC, o.offsets, E);
      if ((r & kExchangeLast) && tid == 0) store_dev(o.header + kEpochWord, epoch);
    }
  }
}

// Top-k + softmax of precomputed logits: one wave per `rows` tokens.
template <int GATE_DT>
__global__ __launch_bounds__(64) void topk_softmax_kernel(const float* __restrict__ logits,
                                                          int64_t n_tokens, int E, int k, int rows,
                                                          int64_t* __restrict__ topk_idx,
                                                          typename Elem<GATE_DT>::T* __restrict__ gate) {
  __shared__ float lg[1024 + 64];
  __shared__ uint64_t keys[1024 + 64];
  __shared__ float sel_val[1024];
  __shared__ int sel_idx[1024];
  __shared__ float rsum[64];
  const int lane = lane_id();
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * rows;
  const int ld = E + 1;
  for (int p = lane; p < rows * E; p += 64) {
    const int t = p / E, e = p - t * E;
    lg[t * ld + e] = (t0 + t < n_tokens) ? logits[(t0 + t) * E + e] : 0.0f;
  }
  __syncthreads();
  select_topk_from_lds<GATE_DT, 0, 0>(lg, ld, rows, E, k, t0, n_tokens, sel_val, sel_idx, rsum,
                                      topk_idx, gate, keys, ld);
}

template <int DT>
hipError_t launch_router(const void* x, const void* w, int64_t n, int hidden, int E, int k,
                         int64_t* idx, void* gate, float* logits, const RouterHist& hist, hipStream_t stream) {
  typedef typename Elem<DT>::T T;
  const int per_block = kWaves * kRowsPerWave;
  const dim3 grid(static_cast<unsigned>((n + per_block - 1) / per_block));
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* gp = static_cast<T*>(gate);
  if constexpr (DT == MEP_DTYPE_BF16) {
    // GraniteMoE's shape: the specialised kernel
    if (E == 32 && k == 8 && (hidden == 1024 || hidden == 2048 || hidden == 4096)) {
      const uint16_t* xb = static_cast<const uint16_t*>(x);
      const uint16_t* wbp = static_cast<const uint16_t*>(w);
      uint16_t* gb = static_cast<uint16_t*>(gate);
      if (hidden == 1024) router32_kernel<1><<<grid, kWaves * 64, 0, stream>>>(xb, wbp, n, idx, gb, logits, hist);
      else if (hidden == 2048) router32_kernel<2><<<grid, kWaves * 64, 0, stream>>>(xb, wbp, n, idx, gb, logits, hist);
      else router32_kernel<4><<<grid, kWaves * 64, 0, stream>>>(xb, wbp, n, idx, gb, logits, hist);
      return hipGetLastError();
    }
  }
  // k = 8 (GraniteMoE's top-8) has a compile-time path; other k use the runtime one
#define MEP_ROUTER_CASE(NF_)                                                                               \
  if (k == 8) router_kernel<DT, NF_, 8><<<grid, kWaves * 64, 0, stream>>>(xp, wp, n, hidden, k, idx, gp, logits, hist); \
  else router_kernel<DT, NF_, 0><<<grid, kWaves * 64, 0, stream>>>(xp, wp, n, hidden, k, idx, gp, logits, hist);
  switch (E) {
    case 16: MEP_ROUTER_CASE(1) break;
    case 32: MEP_ROUTER_CASE(2) break;
    case 64: MEP_ROUTER_CASE(4) break;
    default: return hipErrorInvalidValue;
  }
#undef MEP_ROUTER_CASE
  return hipGetLastError();
}

// Workgroups of route_dispatch32_kernel<NSEG> the current device holds at
// once (its occupancy per CU times the CUs), looked up once per device and NSEG.
constexpr int kMaxDevicesR = 64;
std::atomic<int> g_resident[kMaxDevicesR][3];

template <int NSEG>
int resident_capacity() {
  constexpr int slot = NSEG == 1 ? 0 : (NSEG == 2 ? 1 : 2);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const bool cache = dev >= 0 && dev < kMaxDevicesR;
  if (cache) {
    const int c = g_resident[dev][slot].load(std::memory_order_relaxed);
    if (c != 0) return c > 0 ? c : 0;
  }
  int per_cu = 0, cap = -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, route_dispatch32_kernel<NSEG>, kWaves * 64, 0) ==
          hipSuccess &&
      per_cu > 0)
    cap = per_cu * device_cu_count();
  if (cache) g_resident[dev][slot].store(cap, std::memory_order_relaxed);
  return cap > 0 ? cap : 0;
}

template <int NSEG>
hipError_t launch_fused(const uint16_t* x, const uint16_t* w, int64_t n, int64_t* idx, uint16_t* gate, float* logits,
                        const FusedDispatch& o, int n_blocks, hipStream_t stream) {
  // workgroups wait for each other's rows: all of them must fit at once
  if (n_blocks > 1 && n_blocks > resident_capacity<NSEG>()) return hipErrorNotSupported;
  route_dispatch32_kernel<NSEG><<<n_blocks, kWaves * 64, 0, stream>>>(x, w, n, idx, gate, logits, o);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_route_dispatch_fused(const void* x, const void* w, int64_t n, int hidden, int E, int k, int dtype,
                                       int64_t* idx, void* gate, float* logits, int32_t* counts, int32_t* offsets,
                                       int32_t* perm, int32_t* row_of_entry, int64_t* route_counts, uint64_t* rows,
                                       uint32_t* header, uint32_t* flags, const uint8_t* valid, int n_blocks,
                                       hipStream_t stream) {
  if (dtype != MEP_DTYPE_BF16 || E != 32 || k != 8 || n_blocks < 1 ||
      static_cast<int64_t>(n_blocks) * kWaves * kRowsPerWave < n)
    return hipErrorNotSupported;
  const GiveupTest gt = giveup_test();
  const bool test = gt.site == MEP_GIVEUP_DISPATCH;
  const FusedDispatch o{counts, offsets, perm, row_of_entry, route_counts, rows, header, flags, valid,
                        test ? gt.polls : kRowPolls, test ? n_blocks - 1 : -1};
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* wb = static_cast<const uint16_t*>(w);
  uint16_t* gb = static_cast<uint16_t*>(gate);
  switch (hidden) {
    case 1024: return launch_fused<1>(xb, wb, n, idx, gb, logits, o, n_blocks, stream);
    case 2048: return launch_fused<2>(xb, wb, n, idx, gb, logits, o, n_blocks, stream);
    case 4096: return launch_fused<4>(xb, wb, n, idx, gb, logits, o, n_blocks, stream);
    default: return hipErrorNotSupported;
  }
}

hipError_t launch_router_with_hist(const void* x, const void* w, int64_t n, int hidden, int E, int k, int dtype,
                                   int64_t* idx, void* gate, float* logits, int32_t* bc, uint32_t* header,
                                   uint32_t* flags, int32_t* tables, const uint8_t* valid, int n_blocks,
                                   hipStream_t stream) {
  RouterHist h{bc, header, flags, tables, valid, n_blocks};
  return dtype == MEP_DTYPE_BF16 ? launch_router<MEP_DTYPE_BF16>(x, w, n, hidden, E, k, idx, gate, logits, h, stream)
                                 : launch_router<MEP_DTYPE_F32>(x, w, n, hidden, E, k, idx, gate, logits, h, stream);
}

}  // namespace mep

using namespace mep;

extern "C" int mep_router_topk(const void* x, const void* w_router, int64_t n_tokens,
                               int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype,
                               int64_t* topk_idx, void* topk_gate, float* logits, void* stream) {
  clear_error();
  MEP_REQUIRE(n_tokens >= 0, MEP_ERR_INVALID_ARG, "mep_router_topk: n_tokens < 0");
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "mep_router_topk: unknown dtype %d", dtype);
  MEP_REQUIRE(n_experts == 16 || n_experts == 32 || n_experts == 64, MEP_ERR_UNSUPPORTED,
              "mep_router_topk: n_experts must be 16, 32 or 64 (got %d)", n_experts);
  MEP_REQUIRE(top_k >= 1 && top_k <= n_experts, MEP_ERR_INVALID_ARG,
              "mep_router_topk: top_k %d outside [1, %d]", top_k, n_experts);
  MEP_REQUIRE(hidden > 0 && hidden % 256 == 0, MEP_ERR_UNSUPPORTED,
              "mep_router_topk: hidden %d must be a positive multiple of 256", hidden);
  if (n_tokens == 0) return MEP_OK;
  MEP_REQUIRE(x && w_router && topk_idx && topk_gate, MEP_ERR_INVALID_ARG,
              "mep_router_topk: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  RouterHist none{};
  hipError_t e = dtype == MEP_DTYPE_BF16
                     ? launch_router<MEP_DTYPE_BF16>(x, w_router, n_tokens, hidden, n_experts, top_k,
                                                     topk_idx, topk_gate, logits, none, s)
                     : launch_router<MEP_DTYPE_F32>(x, w_router, n_tokens, hidden, n_experts, top_k,
                                                    topk_idx, topk_gate, logits, none, s);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_router_topk: launch failed: %s", hipGetErrorString(e));
  return MEP_OK;
}

extern "C" int mep_topk_softmax(const float* logits, int64_t n_tokens, int32_t n_experts,
                                int32_t top_k, int32_t gate_dtype, int64_t* topk_idx,
                                void* topk_gate, void* stream) {
  clear_error();
  MEP_REQUIRE(n_tokens >= 0, MEP_ERR_INVALID_ARG, "mep_topk_softmax: n_tokens < 0");
  MEP_REQUIRE(gate_dtype == MEP_DTYPE_F32 || gate_dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "mep_topk_softmax: unknown dtype %d", gate_dtype);
  MEP_REQUIRE(n_experts >= 1 && n_experts <= 256, MEP_ERR_UNSUPPORTED,
              "mep_topk_softmax: n_experts %d outside [1, 256]", n_experts);
  MEP_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= 32, MEP_ERR_INVALID_ARG,
              "mep_topk_softmax: top_k %d outside [1, min(n_experts, 32)]", top_k);
  if (n_tokens == 0) return MEP_OK;
  MEP_REQUIRE(logits && topk_idx && topk_gate, MEP_ERR_INVALID_ARG, "mep_topk_softmax: null pointer");
  // rows per wave: the tile (rows x (E+1)) and the selection (rows x k) fit LDS
  int rows = 1024 / (n_experts + 1);
  if (rows > 64) rows = 64;
  if (rows * top_k > 1024) rows = 1024 / top_k;
  const dim3 grid(static_cast<unsigned>((n_tokens + rows - 1) / rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (gate_dtype == MEP_DTYPE_BF16)
    topk_softmax_kernel<MEP_DTYPE_BF16><<<grid, 64, 0, s>>>(logits, n_tokens, n_experts, top_k, rows,
                                                           topk_idx, static_cast<uint16_t*>(topk_gate));
  else
    topk_softmax_kernel<MEP_DTYPE_F32><<<grid, 64, 0, s>>>(logits, n_tokens, n_experts, top_k, rows,
                                                          topk_idx, static_cast<float*>(topk_gate));
  MEP_CHECK_LAUNCH("mep_topk_softmax");
  return MEP_OK;
}
