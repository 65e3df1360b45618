// Dispatch for the MoE block: one GPU's share of the routed entries, stably
// grouped by local expert, with the balancer's replica round-robin.
//
// Reference semantics (restated):
//   flatten_topk (modeling.py:107-117): entry f = t*k + s, invalid tokens dropped.
//   Placement.dest_ranks (ep.py:76-96): the w-th occurrence (flat order) of
//     expert e inside one source's batch goes to table[e, (rr[e] + w) % n_rep[e]];
//     afterwards rr[e] += count[e].  Layers without replicas use table[e, 0]
//     and leave rr alone.
//   EPMoEBackend (ep.py:216-231): route_counts += bincount; entries for this
//     rank are received source by source in flat order, mapped through g2l
//     (non-resident -> assert), then run_experts sorts them stably by local
//     expert (modeling.py:94-96).
//
// Because everything above is a function of each entry's occurrence index w
// inside (source segment, expert), the whole share is a closed form:
//   kept(f)  <=>  table[e, slot(w)] == my_rank
//   row(f)   =  offsets[g2l[e]] + sum_{s' < s} kept_in_segment(s', e)
//               + #{w' < w : table[e, slot(w')] == my_rank}
// and #{w' < w : (rr + w') % R == j} = (w > c) ? (w - c - 1) / R + 1 : 0 with
// c = (j - rr) mod R.  No atomics decide any position, so the permutation is
// bit-identical to the reference's stable sorts on every run.
//
// Launches over blocks of kChunk consecutive entries of one segment:
//   count_kernel    per-block per-expert histogram (LDS atomics; counts only)
//   prefix_kernel   only above kScanBlocks blocks: one workgroup per expert
//                   turns its histogram column into per-segment exclusive
//                   prefixes and segment totals
//   scatter_kernel  every block takes the prefix of its segment and the
//                   segment totals (from prefix_kernel, or, for few blocks,
//                   re-derived from the histograms: nb x E ints from L2),
//                   then ranks its entries in flat order with wave ballots and
//                   writes perm / row_of_entry / dest.  Block 0 also writes
//                   counts, offsets, route_counts and the updated rr.
#include "common.h"

#include <atomic>

namespace mep {
namespace {

constexpr int kThreads = 512;
constexpr int kChunk = 512;           // entries per block: one round of the block
constexpr int kMaxSeg = 16;
constexpr int kMaxExperts = 256;
constexpr int kMaxReplicas = 32;      // replica slots per expert (a 32-bit mask of this rank's slots)
// above this many blocks the histograms are scanned once by prefix_kernel
// instead of being summed again by every scatter block (nb^2 * E reads)
constexpr int kScanBlocks = 512;

struct DispatchParams {
  const int64_t* topk_idx;
  const uint8_t* valid;
  int64_t n_tokens;
  int k, E;
  const int32_t* table;
  const int32_t* n_rep;
  int rmax, has_rep;
  int64_t* rr;
  int my_rank;
  const int32_t* g2l;
  int n_local;
  int32_t* counts;
  int32_t* offsets;
  int32_t* perm;
  int32_t* row_of_entry;
  int32_t* dest;
  int64_t* route_counts;
  uint32_t* status;     // optional device word: OR of the flags of this call
  // workspace
  uint32_t* header;     // [0] = number of launched blocks
  uint32_t* flags;      // [2 * nbl]: count-kernel flags, scatter-kernel flags
  int64_t* rr_snap;     // [S * E]
  int32_t* bc;          // [nbl * E]
  int32_t* segtot;      // [n_seg * E], written by prefix_kernel
  uint64_t* rows;       // [nbl * E] tagged per-block counts (one-launch dispatch)
  int scanned;          // 1: prefix_kernel turned bc into per-segment exclusive prefixes
  int nb, nbl, n_seg;
  // one launch: polls of a tagged word before a workgroup gives up, and the
  // block that withholds its counts (test hook; -1: none)
  int tag_polls, dbg_withhold;
  int64_t seg_entry[kMaxSeg + 1];
  int seg_block[kMaxSeg + 1];
};

enum : uint32_t { kFlagRange = 1u, kFlagResident = 2u, kFlagReplicas = 4u };

__device__ __forceinline__ int segment_of_block(const DispatchParams& p, int b) {
  int s = 0;
  for (int i = 0; i < p.n_seg; ++i)
    if (b >= p.seg_block[i] && b < p.seg_block[i + 1]) s = i;
  return s;
}

__device__ __forceinline__ void block_range(const DispatchParams& p, int b, int s, int64_t& f0,
                                            int64_t& f1) {
  if (b >= p.nb) { f0 = f1 = 0; return; }
  f0 = p.seg_entry[s] + static_cast<int64_t>(b - p.seg_block[s]) * kChunk;
  f1 = f0 + kChunk;
  if (f1 > p.seg_entry[s + 1]) f1 = p.seg_entry[s + 1];
}


// rr mod R with the sign of R (torch's % on int64 tensors, ep.py:94), in [0, R)
__device__ __forceinline__ int floor_mod(int64_t rr, int R) {
  const int m = static_cast<int>(rr % R);
  return m < 0 ? m + R : m;
}

// #{w' in [0, w) : (rr + w') mod R == j}, summed over the slots j this rank
// holds (bit j of `mine`; R replicas; rrmod = rr mod R).  With w = q R + r,
// each residue class c = (j - rr) mod R holds q + [c < r] of the w' < w, and
// c < r exactly for the r slots j = rrmod, rrmod + 1, ... (mod R): so the sum
// is popc(mine) q + popc(mine & those r slots), one division per call.
// 32-bit: w counts the entries of one expert in one segment (< 2^31), and rr
// enters only through rrmod.
__device__ __forceinline__ uint32_t low_bits(int n) { return n >= 32 ? ~0u : ((1u << n) - 1u); }
__device__ __forceinline__ int kept_before(uint32_t mine, int R, uint32_t w, int rrmod) {
  const uint32_t q = w / static_cast<uint32_t>(R);
  const int r = static_cast<int>(w - q * static_cast<uint32_t>(R));
  const int hi = rrmod + r;                      // slots rrmod .. hi - 1, wrapping past R
  const uint32_t first = low_bits(hi < R ? hi : R) & ~low_bits(rrmod);
  const uint32_t wrap = hi > R ? low_bits(hi - R) : 0u;
  return __popc(mine) * static_cast<int>(q) + __popc(mine & (first | wrap));
}

__global__ __launch_bounds__(kThreads) void count_kernel(DispatchParams p) {
  __shared__ int cnt[kMaxExperts];
  __shared__ uint32_t flag;
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int e = tid; e < p.E; e += kThreads) cnt[e] = 0;
  if (tid == 0) flag = 0;
  __syncthreads();
  const int s = segment_of_block(p, b);
  int64_t f0, f1;
  block_range(p, b, s, f0, f1);
  for (int64_t f = f0 + tid; f < f1; f += kThreads) {
    // both loads issued together (f is in bounds whether or not the token is masked)
    const int64_t e = p.topk_idx[f];
    if (p.valid != nullptr && p.valid[f / p.k] == 0) continue;
    if (e < 0 || e >= p.E) { atomicOr(&flag, kFlagRange); continue; }
    atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < p.E; e += kThreads) p.bc[static_cast<int64_t>(b) * p.E + e] = cnt[e];
  if (tid == 0 && b != 0) p.flags[b] = flag;
  if (b == 0) {
    if (tid == 0) {
      p.header[0] = static_cast<uint32_t>(p.nbl);
      if (p.status != nullptr) *p.status = 0u;      // the scatter kernel ORs into it
    }
    if (p.has_rep)
      for (int i = tid; i < p.n_seg * p.E; i += kThreads) p.rr_snap[i] = p.rr[i];
    // every expert needs 1..rmax replicas (ep.py:21: each expert has an owner)
    for (int e = tid; e < p.E; e += kThreads) {
      const int r = p.n_rep[e];
      if (r < 1 || r > p.rmax) atomicOr(&flag, kFlagReplicas);
    }
  }
  __syncthreads();
  if (b == 0 && tid == 0) p.flags[0] = flag;
}

// One workgroup per expert e: within each source segment, replace the
// column bc[b][e] by its exclusive prefix over the segment's blocks and write
// the segment total to segtot[s][e] -- the same sums the scatter blocks would
// otherwise each rebuild from the whole table.
constexpr int kScanThreads = 256;
__global__ __launch_bounds__(kScanThreads) void prefix_kernel(DispatchParams p) {
  constexpr int V = 8;                                  // blocks per thread per pass
  constexpr int NW = kScanThreads / 64;
  __shared__ int wsum[NW];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int s = 0; s < p.n_seg; ++s) {
    const int b0 = p.seg_block[s], b1 = p.seg_block[s + 1];
    int carry = 0;
    for (int c0 = b0; c0 < b1; c0 += kScanThreads * V) {
      int v[V];
      int sum = 0;
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const int b = c0 + tid * V + u;
        v[u] = b < b1 ? p.bc[static_cast<int64_t>(b) * p.E + e] : 0;
        sum += v[u];
      }
      int x = sum;                                      // inclusive scan over the wave
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      if (lane == 63) wsum[wave] = x;
      __syncthreads();
      int before = 0, total = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        if (w < wave) before += wsum[w];
        total += wsum[w];
      }
      int run = carry + before + x - sum;               // prefix of this thread's first block
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const int b = c0 + tid * V + u;
        if (b < b1) p.bc[static_cast<int64_t>(b) * p.E + e] = run;
        run += v[u];
      }
      carry += total;
      __syncthreads();                                  // wsum is rewritten by the next pass
    }
    if (tid == 0) p.segtot[s * p.E + e] = carry;
  }
}

// LDS copy of the replica table in scatter_kernel when it has at most this many entries
constexpr int kTabLds = 2048;

// One-launch dispatch (scatter_kernel<true>): every block also does
// count_kernel's work for its own entries, publishes its per-expert counts as
// 64-bit words (tag << 32 | count) with device-scope (sc1) stores, and reads
// every block's counts with device-scope loads, re-reading until each word
// carries this call's tag: they give the segment totals and its own prefix
// (the earlier blocks of its segment).  No counter, no atomic across blocks:
// the tag is 2^31 | (the workspace's epoch word + 1), read by every block as
// it starts and advanced by block 0 once it has read every block's counts (by
// then every block has published, so every block has read the epoch).
// Whatever else the dispatch leaves in a workspace (counts, flags, tables,
// round-robin counters below 2^32) has a clear top bit in its high word, so a
// workspace zero-filled once serves calls of any size.  All blocks must be
// resident at once: the host launches it only when they fit.  A wait longer
// than kTagPolls polls sets kFlagBarrier in the block's status word; the
// block then places nothing (its entries get kPoisonRow) and, as the last
// block to finish sees, the whole call is poisoned (see finish_exchange).
constexpr int kTagPolls = 1 << 20;

__device__ __forceinline__ uint32_t load_dev(const uint32_t* q) {
  return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev(const uint64_t* q) {
  return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint64_t* q, uint64_t v) {
  __hip_atomic_store(q, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* q, uint32_t v) {
  __hip_atomic_store(q, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Reads the tagged words w[i * stride] for i in [0, n) (this thread's share:
// i = first, first + step, ...), each re-read until it carries `tag`, and
// calls use(i, count) for each.  Sets *bad after `polls` polls of a batch.
template <typename Use>
__device__ __forceinline__ void read_tagged(const uint64_t* w, int64_t stride, int first, int n, int step,
                                            uint64_t tag, int polls, uint32_t* bad, Use use) {
  constexpr int kBatch = 8;
  for (int i0 = first; i0 < n; i0 += step * kBatch) {
    uint64_t v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + u * step;
      v[u] = i < n ? load_dev(w + i * stride) : tag;
    }
    for (int it = 0;; ++it) {
      bool stale = false;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) stale |= (v[u] & ~0xffffffffull) != tag;
      if (!stale) break;
      if (it >= polls) { *bad = kFlagBarrier; break; }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if ((v[u] & ~0xffffffffull) != tag) v[u] = load_dev(w + (i0 + u * step) * stride);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (i0 + u * step < n) use(i0 + u * step, static_cast<int>(static_cast<uint32_t>(v[u])));
  }
}

template <bool FUSED>
__global__ __launch_bounds__(kThreads) void scatter_kernel(DispatchParams p) {
  __shared__ int segtot[kMaxSeg][kMaxExperts];   // entries of expert e in segment s
  // per-expert tables, copied once per block (every entry looks them up):
  __shared__ int s_tab[kTabLds];                 // table (E x rmax) when it fits
  __shared__ int s_R[kMaxExperts];               // replica count (clamped to [1, rmax])
  __shared__ uint32_t s_mine[kMaxExperts];       // bit j: table[e][j] == my_rank
  __shared__ int s_g2l[kMaxExperts];
  __shared__ int s_rrmod[kMaxSeg * kMaxExperts]; // rr[segment][e] mod R
  __shared__ int pre[kMaxExperts];                // ... in earlier blocks of my segment
  __shared__ int keptbase[kMaxExperts];           // kept entries of e in earlier segments
  __shared__ int loff[kMaxExperts];               // first row of e's local expert
  __shared__ int lcount[kMaxExperts];             // rows per local expert
  __shared__ int lpre[kMaxExperts + 1];           // exclusive prefix of lcount
  __shared__ int lwave[kMaxExperts / 64];
  __shared__ int wcnt[kThreads / 64][kMaxExperts + 1];
  __shared__ uint32_t flag;
  __shared__ int s_cnt[FUSED ? kMaxExperts : 1];  // one launch: this block's entries per expert
  __shared__ uint32_t cflag;                      // one launch: this block's count-pass flags
  __shared__ uint32_t s_bad;                      // one launch: a wait of this block gave up

  const int b = blockIdx.x, tid = threadIdx.x;
  const int E = p.E;
  const int s = segment_of_block(p, b);
  int64_t f0, f1;
  block_range(p, b, s, f0, f1);
  uint64_t tag = 0;
  if constexpr (FUSED) {
    // this call's tag; the load has long landed when the tag is first used
    tag = static_cast<uint64_t>(0x80000000u | ((load_dev(p.header + kEpochWord) + 1u) & 0x7fffffffu)) << 32;
    asm volatile("" ::: "memory");
  }
  // this thread's entry (a block is one round of entries), loaded first so
  // that its latency overlaps the histogram pass below
  static_assert(kChunk == kThreads, "one entry per thread");
  const int64_t f = f0 + tid;
  int key = E;                                    // E: no expert (padding, masked or out of range)
  bool dropped = false, bad_id = false;
  if (f < f1) {
    const bool valid = p.valid == nullptr || p.valid[f / p.k] != 0;
    const int64_t e = p.topk_idx[f];
    if (valid && e >= 0 && e < E) key = static_cast<int>(e);
    else dropped = true;
    bad_id = valid && (e < 0 || e >= E);
  }

  // the per-expert tables: every load goes out with the entry's, before the
  // first barrier (one memory round trip); what derives from them is
  // computed from LDS and registers after it
  static_assert(kThreads >= kMaxExperts, "one expert per thread");
  const bool tab_lds = E * p.rmax <= kTabLds;
  if (tab_lds)
    for (int i = tid; i < E * p.rmax; i += kThreads) s_tab[i] = p.table[i];
  const int my_nrep = tid < E ? p.n_rep[tid] : 1;
  if (tid < E) {
    // replica count clamped to the table width (keeps every table read in
    // bounds); a count outside [1, rmax] is reported by block 0
    s_R[tid] = my_nrep < 1 ? 1 : (my_nrep > p.rmax ? p.rmax : my_nrep);
    s_g2l[tid] = p.g2l[tid];
  }
  // round-robin counters of (segment, expert) i = tid + u kThreads; one launch
  // reads rr itself (block 0 updates it only after every block has read it)
  constexpr int kRrPer = kMaxSeg * kMaxExperts / kThreads;
  int64_t rr_v[kRrPer];
  if (p.has_rep) {
#pragma unroll
    for (int u = 0; u < kRrPer; ++u) {
      const int i = tid + u * kThreads;
      rr_v[u] = i < p.n_seg * E ? (FUSED ? p.rr[i] : p.rr_snap[i]) : 0;
    }
  }
  for (int i = tid; i < p.n_seg * kMaxExperts; i += kThreads) segtot[i / kMaxExperts][i % kMaxExperts] = 0;
  for (int e = tid; e < E; e += kThreads) { pre[e] = 0; lcount[e] = 0; }
  for (int i = tid; i < (kThreads / 64) * (kMaxExperts + 1); i += kThreads)
    wcnt[i / (kMaxExperts + 1)][i % (kMaxExperts + 1)] = 0;
  if (tid == 0) flag = 0;
  if constexpr (FUSED) {
    for (int e = tid; e < E; e += kThreads) s_cnt[e] = 0;
    if (tid == 0) { cflag = 0; s_bad = 0; }
  }
  __syncthreads();
  if (tid < E) {
    const int R = s_R[tid];
    uint32_t mine = 0;
    if (tab_lds)
      for (int j = 0; j < R; ++j) mine |= (s_tab[tid * p.rmax + j] == p.my_rank ? 1u : 0u) << j;
    else
      for (int j = 0; j < R; ++j) mine |= (p.table[tid * p.rmax + j] == p.my_rank ? 1u : 0u) << j;
    s_mine[tid] = mine;
  }
  if (p.has_rep) {
#pragma unroll
    for (int u = 0; u < kRrPer; ++u) {
      const int i = tid + u * kThreads;
      if (i < p.n_seg * E) s_rrmod[i] = floor_mod(rr_v[u], s_R[i % E]);
    }
  }
  uint32_t tag_bad = 0u;
  if constexpr (FUSED) {
    if (b == 0) {
      if (tid == 0) {
        p.header[0] = static_cast<uint32_t>(p.nbl);
        // cleared (and acknowledged) before this block publishes its counts,
        // so before any block ORs into it
        if (p.status != nullptr) store_dev(p.status, 0u);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      // every expert needs 1..rmax replicas (ep.py:21: each expert has an owner)
      if (tid < E && (my_nrep < 1 || my_nrep > p.rmax)) atomicOr(&cflag, kFlagReplicas);
    }
    // count_kernel's pass over this block's entries
    if (key < E) atomicAdd(&s_cnt[key], 1);
    if (bad_id) atomicOr(&cflag, kFlagRange);
    __syncthreads();
    if (b != p.dbg_withhold)
      for (int e = tid; e < E; e += kThreads)
        store_dev(p.rows + static_cast<int64_t>(b) * E + e, tag | static_cast<uint32_t>(s_cnt[e]));
    // every block's counts: the segment totals, and my prefix (the earlier
    // blocks of my segment)
    const int parts = kThreads / E > 0 ? kThreads / E : 1;
    const int e = tid % E, part = tid / E;
    if (part < parts && tid < parts * E) {
      int my_pre = 0;
      int sg = 0, sg_end = p.seg_block[1], run = 0;   // this thread's rows come in increasing order
      read_tagged(p.rows + e, E, part, p.nb, parts, tag, p.tag_polls, &tag_bad, [&](int bb, int c) {
        while (bb >= sg_end) {
          if (run) atomicAdd(&segtot[sg][e], run);
          run = 0;
          ++sg;
          sg_end = p.seg_block[sg + 1];
        }
        run += c;
        if (sg == s && bb < b) my_pre += c;
      });
      if (run) atomicAdd(&segtot[sg][e], run);
      atomicAdd(&pre[e], my_pre);
    }
    if (tag_bad) s_bad = tag_bad;
  }
  __syncthreads();
  // a block whose wait gave up has counts from earlier calls: it places
  // nothing and leaves rr and route_counts alone
  const bool gave_up = FUSED && s_bad != 0u;

  // 1. segment totals and my prefix: from the tagged counts above (one
  // launch), read from prefix_kernel's results, or
  // summed here from the per-block histograms.  The
  // histogram loads of a thread are issued 8 at a time before any of them is
  // used (one L2 round trip per 8 blocks instead of one per block); with one
  // segment the total is summed in a register and added to LDS once.
  if (FUSED) {
  } else if (p.scanned) {
    for (int i = tid; i < p.n_seg * E; i += kThreads) segtot[i / E][i % E] = p.segtot[i];
    for (int e = tid; e < E; e += kThreads) pre[e] = b < p.nb ? p.bc[static_cast<int64_t>(b) * E + e] : 0;
  } else {
    const int parts = kThreads / E > 0 ? kThreads / E : 1;
    const int e = tid % E, part = tid / E;
    if (part < parts && tid < parts * E) {
      int my_pre = 0, my_tot = 0;
      constexpr int kBatch = 8;
      for (int bb0 = part; bb0 < p.nb; bb0 += parts * kBatch) {
        int c[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int bb = bb0 + u * parts;
          c[u] = bb < p.nb ? p.bc[static_cast<int64_t>(bb) * E + e] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int bb = bb0 + u * parts;
          if (bb >= p.nb) continue;
          const int sb = p.n_seg == 1 ? 0 : segment_of_block(p, bb);
          if (p.n_seg == 1) my_tot += c[u];
          else atomicAdd(&segtot[sb][e], c[u]);
          if (sb == s && bb < b) my_pre += c[u];
        }
      }
      if (p.n_seg == 1) atomicAdd(&segtot[0][e], my_tot);
      atomicAdd(&pre[e], my_pre);
    }
  }
  __syncthreads();

  // 2. kept entries per (segment, expert) -> local counts and my segment base
  for (int e = tid; e < E; e += kThreads) {
    int64_t total = 0, base = 0;
    const uint32_t mine = s_mine[e];
    const int R = s_R[e];
    for (int sg = 0; sg < p.n_seg; ++sg) {
      int64_t kept;
      if (p.has_rep) kept = kept_before(mine, R, static_cast<uint32_t>(segtot[sg][e]), s_rrmod[sg * E + e]);
      else kept = (mine & 1u) ? segtot[sg][e] : 0;
      if (sg < s) base += kept;
      total += kept;
    }
    keptbase[e] = static_cast<int>(base);
    const int j = s_g2l[e];
    if (j >= 0 && j < p.n_local) lcount[j] = static_cast<int>(total);
  }
  __syncthreads();
  // exclusive prefix of the local counts: a scan over the first 4 waves
  {
    const int lane = tid & 63, wv = tid >> 6;
    int v = 0, incl = 0;
    if (tid < kMaxExperts) {
      v = tid < p.n_local ? lcount[tid] : 0;
      incl = v;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
      }
      if (lane == 63) lwave[wv] = incl;
    }
    __syncthreads();
    if (tid < kMaxExperts) {
      int add = 0;
#pragma unroll
      for (int w = 0; w < kMaxExperts / 64; ++w) add += w < wv ? lwave[w] : 0;
      lpre[tid] = add + incl - v;
      if (tid == kMaxExperts - 1) lpre[kMaxExperts] = add + incl;
    }
    __syncthreads();
  }
  for (int e = tid; e < E; e += kThreads) {
    const int j = s_g2l[e];
    loff[e] = (j >= 0 && j < p.n_local) ? lpre[j] : 0;
  }
  if (b == 0) {
    for (int j = tid; j <= p.n_local; j += kThreads) {
      // one launch: device scope, as is the poison that may replace offsets[n_local]
      if (FUSED) store_dev(reinterpret_cast<uint32_t*>(p.offsets + j), static_cast<uint32_t>(lpre[j]));
      else p.offsets[j] = lpre[j];
      if (j < p.n_local) p.counts[j] = lcount[j];
    }
    for (int e = gave_up ? E : tid; e < E; e += kThreads) {
      int64_t tot = 0;
      for (int sg = 0; sg < p.n_seg; ++sg) {
        tot += segtot[sg][e];
        if (p.has_rep) p.rr[sg * E + e] = (FUSED ? p.rr[sg * E + e] : p.rr_snap[sg * E + e]) + segtot[sg][e];
      }
      if (p.route_counts != nullptr) p.route_counts[e] += tot;
    }
  }
  __syncthreads();

  // 3. rank this block's entries in flat order and scatter.  One launch:
  // row_of_entry with device-scope stores, as is the poison that may replace it.
  auto put_row = [&](int64_t ff, int32_t v) {
    if (FUSED) store_dev(reinterpret_cast<uint32_t*>(p.row_of_entry + ff), static_cast<uint32_t>(v));
    else p.row_of_entry[ff] = v;
  };
  const int lane = tid & 63, wave = tid >> 6;
  const int nbits = 32 - __clz(E);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  if (gave_up) {
    if (f < f1) {
      put_row(f, kPoisonRow);
      if (p.dest != nullptr) p.dest[f] = -1;
    }
  } else {
  if (dropped) {
    put_row(f, -1);
    if (p.dest != nullptr) p.dest[f] = -1;
  }
  uint64_t peers = ~0ull;
  for (int bit = 0; bit < nbits; ++bit) {
    const bool on = (key >> bit) & 1;
    const uint64_t m = __ballot(on);
    peers &= on ? m : ~m;
  }
  const int rank_w = __popcll(peers & lt_mask);
  if (key < E && rank_w == 0) wcnt[wave][key] = __popcll(peers);
  __syncthreads();
  if (key < E) {
    int w = pre[key] + rank_w;
#pragma unroll
    for (int ww = 0; ww < kThreads / 64; ++ww) w += ww < wave ? wcnt[ww][key] : 0;
    const int e = key;
    const int rrmod = p.has_rep ? s_rrmod[s * E + e] : 0;
    const int R = s_R[e];
    // (rr + w) mod R, floor modulo as torch's % on int64 tensors (ep.py:94)
    const int slot = p.has_rep ? static_cast<int>((static_cast<uint32_t>(rrmod) + static_cast<uint32_t>(w)) % static_cast<uint32_t>(R)) : 0;
    const int d = tab_lds ? s_tab[e * p.rmax + slot] : p.table[e * p.rmax + slot];
    if (p.dest != nullptr) p.dest[f] = d;
    int row = -1;
    if (d == p.my_rank) {
      const int j = s_g2l[e];
      if (j >= 0 && j < p.n_local) {
        const int kb = p.has_rep ? kept_before(s_mine[e], R, static_cast<uint32_t>(w), rrmod) : w;
        row = loff[e] + keptbase[e] + static_cast<int>(kb);
        p.perm[row] = static_cast<int32_t>(f);
      } else {
        atomicOr(&flag, kFlagResident);
      }
    }
    put_row(f, row);
  }
  }
  if (FUSED && tag_bad) atomicOr(&flag, tag_bad);
  __syncthreads();
  if (tid == 0) {
    p.flags[p.nbl + b] = flag;
    if constexpr (FUSED) p.flags[b] = cflag;
    if (p.status != nullptr) {
      const uint32_t f = flag | (FUSED ? cflag : p.flags[b]);   // this block's count and scatter flags
      if (f != 0u) atomicOr(p.status, f);
    }
  }
  if constexpr (FUSED) {
    // the last block to finish poisons a call in which a block gave up, and
    // advances the epoch (every block has read it)
    if (tid < 64) {
      const int r = finish_exchange(p.header, gave_up, static_cast<int>(gridDim.x));
      if (r & kExchangeGaveUp) poison_dispatch(p.row_of_entry, p.seg_entry[p.n_seg], p.offsets, p.n_local);
      if ((r & kExchangeLast) && tid == 0) store_dev(p.header + kEpochWord, static_cast<uint32_t>(tag >> 32) & 0x7fffffffu);
    }
  }
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct WsLayout {
  size_t header, flags, rr_snap, bc, segtot, rows, total;
};

WsLayout ws_layout(int nbl, int n_seg, int E) {
  WsLayout l;
  l.header = 0;
  l.flags = kWsHeaderBytes;
  l.rr_snap = align_up(l.flags + sizeof(uint32_t) * 2 * nbl, 256);
  l.bc = align_up(l.rr_snap + sizeof(int64_t) * n_seg * E, 256);
  l.segtot = align_up(l.bc + sizeof(int32_t) * static_cast<size_t>(nbl) * E, 256);
  l.rows = align_up(l.segtot + sizeof(int32_t) * static_cast<size_t>(n_seg) * E, 256);
  l.total = align_up(l.rows + sizeof(uint64_t) * static_cast<size_t>(nbl) * E, 256);
  return l;
}

int count_blocks(const int64_t* seg_tokens, int n_seg, int k, int* seg_block) {
  int nb = 0;
  for (int s = 0; s < n_seg; ++s) {
    seg_block[s] = nb;
    const int64_t ne = (seg_tokens[s + 1] - seg_tokens[s]) * k;
    nb += static_cast<int>((ne + kChunk - 1) / kChunk);
  }
  seg_block[n_seg] = nb;
  return nb;
}

}  // namespace
}  // namespace mep

using namespace mep;

extern "C" size_t mep_dispatch_workspace_size(int64_t n_tokens, int32_t top_k, int32_t n_experts,
                                              int32_t n_segments, const int64_t* seg_tokens) {
  int64_t one_seg[2] = {0, n_tokens};
  if (n_segments <= 0 || seg_tokens == nullptr) { n_segments = 1; seg_tokens = one_seg; }
  if (n_segments > kMaxSeg || top_k <= 0 || n_experts <= 0) return 0;
  int seg_block[kMaxSeg + 1];
  const int nb = count_blocks(seg_tokens, n_segments, top_k, seg_block);
  return ws_layout(nb > 0 ? nb : 1, n_segments, n_experts).total;
}

namespace mep {

// Static scratch of mep_dispatch_noalloc: the workspace of mep_dispatch
// (header, flags, counter snapshot, per-block histograms, segment totals,
// tagged counts) in a file-scope device array, one copy per GPU, held until
// the process ends.  Device arrays start zero-filled, which is all the
// one-launch dispatch asks of a workspace; every call on a GPU reuses that
// GPU's copy and nothing needs clearing between calls.
constexpr size_t kScratchBytes = size_t(2) << 20;
__device__ __attribute__((aligned(256))) unsigned char dispatch_scratch[kScratchBytes];

namespace {

// Device address of `dispatch_scratch` on the current device, looked up on the first
// call on each device (hipGetSymbolAddress with that device current) and kept
// per device.  The array's name is only a host-side handle; kernels receive
// this address.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_dispatch_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  MEP_REQUIRE(dev >= 0 && dev < kMaxDevices, MEP_ERR_UNSUPPORTED,
              "mep_dispatch_noalloc: device %d beyond the %d supported", dev, kMaxDevices);
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(dispatch_scratch));
    MEP_REQUIRE(e == hipSuccess && ptr != nullptr, MEP_ERR_HIP,
                "mep_dispatch_noalloc: hipGetSymbolAddress(dispatch_scratch): %s", hipGetErrorString(e));
    g_scratch[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return MEP_OK;
}

// Blocks of scatter_kernel<true> the current device holds at once (its
// occupancy per CU times the CUs), looked up once per device.
std::atomic<int> g_fused_cap[kMaxDevices];

int fused_capacity() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const bool cache = dev >= 0 && dev < kMaxDevices;
  if (cache) {
    const int c = g_fused_cap[dev].load(std::memory_order_relaxed);
    if (c != 0) return c > 0 ? c : 0;
  }
  int per_cu = 0, cap = -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, scatter_kernel<true>, kThreads, 0) == hipSuccess &&
      per_cu > 0)
    cap = per_cu * device_cu_count();
  if (cache) g_fused_cap[dev].store(cap, std::memory_order_relaxed);
  return cap > 0 ? cap : 0;
}

// Shared body of mep_dispatch and mep_dispatch_noalloc.  workspace == NULL
// selects the static scratch (whose size bounds the call).
int dispatch_impl(const char* fn, const int64_t* topk_idx, const uint8_t* valid_mask, int64_t n_tokens,
                  int32_t top_k, int32_t n_experts, const int32_t* table, const int32_t* n_rep, int32_t rmax,
                  int32_t has_replicas, int64_t* rr, const int64_t* seg_tokens, int32_t n_segments,
                  int32_t my_rank, const int32_t* g2l, int32_t n_local, int32_t* counts, int32_t* offsets,
                  int32_t* perm, int32_t* row_of_entry, int32_t* dest, int64_t* route_counts,
                  uint32_t* status, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const bool use_scratch = workspace == nullptr;
  MEP_REQUIRE(n_tokens >= 0 && top_k >= 1 && top_k <= 32, MEP_ERR_INVALID_ARG,
              "%s: bad n_tokens %lld / top_k %d", fn, (long long)n_tokens, top_k);
  MEP_REQUIRE(n_experts >= 1 && n_experts <= kMaxExperts, MEP_ERR_UNSUPPORTED,
              "%s: n_experts %d outside [1, %d]", fn, n_experts, kMaxExperts);
  MEP_REQUIRE(n_tokens * top_k < (int64_t(1) << 31), MEP_ERR_UNSUPPORTED,
              "%s: n_tokens * top_k must be < 2^31", fn);
  MEP_REQUIRE(rmax >= 1, MEP_ERR_INVALID_ARG, "%s: rmax %d < 1", fn, rmax);
  MEP_REQUIRE(rmax <= kMaxReplicas, MEP_ERR_UNSUPPORTED, "%s: rmax %d > %d replicas", fn, rmax, kMaxReplicas);
  MEP_REQUIRE(n_local >= 0 && n_local <= n_experts, MEP_ERR_INVALID_ARG,
              "%s: n_local %d outside [0, %d]", fn, n_local, n_experts);
  MEP_REQUIRE(n_segments >= 1 && n_segments <= kMaxSeg && seg_tokens != nullptr,
              MEP_ERR_INVALID_ARG, "%s: need 1..%d segments (got %d)", fn, kMaxSeg, n_segments);
  MEP_REQUIRE(seg_tokens[0] == 0 && seg_tokens[n_segments] == n_tokens, MEP_ERR_INVALID_ARG,
              "%s: seg_tokens must run from 0 to n_tokens", fn);
  for (int s = 0; s < n_segments; ++s)
    MEP_REQUIRE(seg_tokens[s + 1] >= seg_tokens[s], MEP_ERR_INVALID_ARG,
                "%s: seg_tokens must be non-decreasing", fn);
  MEP_REQUIRE(topk_idx || n_tokens == 0, MEP_ERR_INVALID_ARG, "%s: topk_idx is null", fn);
  MEP_REQUIRE(table && n_rep && g2l && offsets, MEP_ERR_INVALID_ARG,
              "%s: null table / n_rep / g2l / offsets", fn);
  // what the kernels write: row_of_entry for every entry, counts for every
  // local expert, perm for every kept row
  MEP_REQUIRE(row_of_entry || n_tokens == 0, MEP_ERR_INVALID_ARG,
              "%s: row_of_entry is null (needed whenever n_tokens > 0)", fn);
  MEP_REQUIRE(counts || n_local == 0, MEP_ERR_INVALID_ARG,
              "%s: counts is null (needed whenever n_local > 0)", fn);
  MEP_REQUIRE(perm || n_tokens == 0 || n_local == 0, MEP_ERR_INVALID_ARG,
              "%s: perm is null (needed whenever n_tokens > 0 and n_local > 0)", fn);
  MEP_REQUIRE(!has_replicas || rr != nullptr, MEP_ERR_INVALID_ARG,
              "%s: rr is required when the layer has replicas", fn);

  DispatchParams p;
  p.nb = count_blocks(seg_tokens, n_segments, top_k, p.seg_block);
  p.nbl = p.nb > 0 ? p.nb : 1;
  const WsLayout l = ws_layout(p.nbl, n_segments, n_experts);
  if (use_scratch) {
    MEP_REQUIRE(l.total <= kScratchBytes, MEP_ERR_UNSUPPORTED,
                "%s: needs %zu B of scratch, more than the %zu B static scratch (fewer tokens or experts per call)",
                fn, l.total, kScratchBytes);
    const int rc = scratch_address(&workspace);
    if (rc != MEP_OK) return rc;
  } else {
    MEP_REQUIRE(workspace_bytes >= l.total, MEP_ERR_WORKSPACE,
                "%s: workspace %zu B < required %zu B", fn, workspace_bytes, l.total);
  }
  char* ws = static_cast<char*>(workspace);
  p.topk_idx = topk_idx; p.valid = valid_mask; p.n_tokens = n_tokens;
  p.k = top_k; p.E = n_experts; p.table = table; p.n_rep = n_rep; p.rmax = rmax;
  p.has_rep = has_replicas ? 1 : 0; p.rr = rr; p.my_rank = my_rank; p.g2l = g2l;
  p.n_local = n_local; p.counts = counts; p.offsets = offsets; p.perm = perm;
  p.row_of_entry = row_of_entry; p.dest = dest; p.route_counts = route_counts;
  p.status = status;
  p.header = reinterpret_cast<uint32_t*>(ws + l.header);
  p.flags = reinterpret_cast<uint32_t*>(ws + l.flags);
  p.rr_snap = reinterpret_cast<int64_t*>(ws + l.rr_snap);
  p.bc = reinterpret_cast<int32_t*>(ws + l.bc);
  p.segtot = reinterpret_cast<int32_t*>(ws + l.segtot);
  p.scanned = p.nb > kScanBlocks ? 1 : 0;
  p.n_seg = n_segments;
  for (int s = 0; s <= n_segments; ++s) p.seg_entry[s] = seg_tokens[s] * top_k;
  for (int s = n_segments + 1; s <= kMaxSeg; ++s) { p.seg_entry[s] = p.seg_entry[n_segments]; p.seg_block[s] = p.nb; }

  p.rows = reinterpret_cast<uint64_t*>(ws + l.rows);
  const GiveupTest gt = giveup_test();
  p.tag_polls = gt.site == MEP_GIVEUP_DISPATCH ? gt.polls : kTagPolls;
  p.dbg_withhold = gt.site == MEP_GIVEUP_DISPATCH ? p.nbl - 1 : -1;

  hipStream_t st = static_cast<hipStream_t>(stream);
  // one launch when every block fits on the device at once
  if (p.nb >= 1 && !p.scanned && p.nb <= fused_capacity()) {
    scatter_kernel<true><<<p.nbl, kThreads, 0, st>>>(p);
    MEP_CHECK_LAUNCH("mep_dispatch(one launch)");
    return MEP_OK;
  }
  count_kernel<<<p.nbl, kThreads, 0, st>>>(p);
  MEP_CHECK_LAUNCH("mep_dispatch(count)");
  if (p.scanned) {
    prefix_kernel<<<n_experts, kScanThreads, 0, st>>>(p);
    MEP_CHECK_LAUNCH("mep_dispatch(prefix)");
  }
  scatter_kernel<false><<<p.nbl, kThreads, 0, st>>>(p);
  MEP_CHECK_LAUNCH("mep_dispatch(scatter)");
  return MEP_OK;
}

}  // namespace
}  // namespace mep

extern "C" int mep_dispatch(const int64_t* topk_idx, const uint8_t* valid_mask, int64_t n_tokens,
                            int32_t top_k, int32_t n_experts, const int32_t* table,
                            const int32_t* n_rep, int32_t rmax, int32_t has_replicas, int64_t* rr,
                            const int64_t* seg_tokens, int32_t n_segments, int32_t my_rank,
                            const int32_t* g2l, int32_t n_local, int32_t* counts, int32_t* offsets,
                            int32_t* perm, int32_t* row_of_entry, int32_t* dest,
                            int64_t* route_counts, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (workspace == nullptr) {
    clear_error();
    set_error("mep_dispatch: null workspace");
    return MEP_ERR_INVALID_ARG;
  }
  return dispatch_impl("mep_dispatch", topk_idx, valid_mask, n_tokens, top_k, n_experts, table, n_rep, rmax,
                       has_replicas, rr, seg_tokens, n_segments, my_rank, g2l, n_local, counts, offsets, perm,
                       row_of_entry, dest, route_counts, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int mep_dispatch_noalloc(const int64_t* topk_idx, const uint8_t* valid_mask, int64_t n_tokens,
                                    int32_t top_k, int32_t n_experts, const int32_t* table,
                                    const int32_t* n_rep, int32_t rmax, int32_t has_replicas, int64_t* rr,
                                    const int64_t* seg_tokens, int32_t n_segments, int32_t my_rank,
                                    const int32_t* g2l, int32_t n_local, int32_t* counts, int32_t* offsets,
                                    int32_t* perm, int32_t* row_of_entry, int32_t* dest,
                                    int64_t* route_counts, uint32_t* status, void* stream) {
  return dispatch_impl("mep_dispatch_noalloc", topk_idx, valid_mask, n_tokens, top_k, n_experts, table, n_rep,
                       rmax, has_replicas, rr, seg_tokens, n_segments, my_rank, g2l, n_local, counts, offsets,
                       perm, row_of_entry, dest, route_counts, status, nullptr, 0, stream);
}

namespace mep {
namespace {

// Dispatch result of an empty batch: no rows, and a workspace that
// mep_dispatch_check reads as one block without flags.
__global__ void empty_route_kernel(int n_local, int32_t* counts, int32_t* offsets, uint32_t* header,
                                   uint32_t* flags) {
  for (int j = threadIdx.x; j <= n_local; j += blockDim.x) {
    offsets[j] = 0;
    if (j < n_local) counts[j] = 0;
  }
  if (threadIdx.x == 0) {
    header[0] = 1u;
    flags[0] = 0u;
    flags[1] = 0u;
  }
}

size_t route_tables_offset(const WsLayout& l) { return l.total; }

WsLayout route_layout(int64_t n_tokens, int32_t n_experts, int* nb_out) {
  const int nb = static_cast<int>((n_tokens * 8 + kChunk - 1) / kChunk);
  *nb_out = nb;
  return ws_layout(nb > 0 ? nb : 1, 1, n_experts);
}

}  // namespace
}  // namespace mep

extern "C" size_t mep_route_dispatch_workspace_size(int64_t n_tokens, int32_t n_experts) {
  if (n_tokens < 0 || n_experts <= 0 || n_experts > kMaxExperts) return 0;
  int nb = 0;
  const WsLayout l = route_layout(n_tokens, n_experts, &nb);
  return route_tables_offset(l) + align_up(sizeof(int32_t) * 3 * n_experts, 256);
}

extern "C" int mep_route_dispatch(const void* x, const void* w_router, const uint8_t* valid_mask, int64_t n_tokens,
                                  int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype,
                                  int64_t* topk_idx, void* topk_gate, float* logits, int32_t* counts,
                                  int32_t* offsets, int32_t* perm, int32_t* row_of_entry, int64_t* route_counts,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const char* fn = "mep_route_dispatch";
  MEP_REQUIRE(n_tokens >= 0, MEP_ERR_INVALID_ARG, "%s: n_tokens < 0", fn);
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG, "%s: unknown dtype %d", fn,
              dtype);
  MEP_REQUIRE(top_k == 8, MEP_ERR_UNSUPPORTED, "%s: top_k must be 8 (got %d); use mep_router_topk + mep_dispatch",
              fn, top_k);
  MEP_REQUIRE(n_experts == 16 || n_experts == 32 || n_experts == 64, MEP_ERR_UNSUPPORTED,
              "%s: n_experts must be 16, 32 or 64 (got %d)", fn, n_experts);
  MEP_REQUIRE(hidden > 0 && hidden % 256 == 0, MEP_ERR_UNSUPPORTED,
              "%s: hidden %d must be a positive multiple of 256", fn, hidden);
  MEP_REQUIRE(n_tokens * top_k < (int64_t(1) << 31), MEP_ERR_UNSUPPORTED, "%s: n_tokens * top_k must be < 2^31",
              fn);
  MEP_REQUIRE(counts && offsets && workspace, MEP_ERR_INVALID_ARG, "%s: null counts / offsets / workspace", fn);
  MEP_REQUIRE(n_tokens == 0 || (x && w_router && topk_idx && topk_gate && perm && row_of_entry),
              MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
  int nb = 0;
  const WsLayout l = route_layout(n_tokens, n_experts, &nb);
  const size_t need = mep_route_dispatch_workspace_size(n_tokens, n_experts);
  MEP_REQUIRE(workspace_bytes >= need, MEP_ERR_WORKSPACE, "%s: workspace %zu B < required %zu B", fn,
              workspace_bytes, need);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n_tokens == 0) {
    empty_route_kernel<<<1, 256, 0, st>>>(n_experts, counts, offsets, reinterpret_cast<uint32_t*>(ws + l.header),
                                          reinterpret_cast<uint32_t*>(ws + l.flags));
    MEP_CHECK_LAUNCH("mep_route_dispatch(empty)");
    return MEP_OK;
  }
  // one launch when the shape has the fused kernel and its workgroups fit on
  // the device at once
  hipError_t e = launch_route_dispatch_fused(x, w_router, n_tokens, hidden, n_experts, top_k, dtype, topk_idx,
                                             topk_gate, logits, counts, offsets, perm, row_of_entry, route_counts,
                                             reinterpret_cast<uint64_t*>(ws + l.rows),
                                             reinterpret_cast<uint32_t*>(ws + l.header),
                                             reinterpret_cast<uint32_t*>(ws + l.flags), valid_mask, nb, st);
  if (e == hipSuccess) return MEP_OK;
  MEP_REQUIRE(e == hipErrorNotSupported, MEP_ERR_HIP, "%s: fused launch failed: %s", fn, hipGetErrorString(e));
  int32_t* tables = reinterpret_cast<int32_t*>(ws + route_tables_offset(l));
  e = launch_router_with_hist(x, w_router, n_tokens, hidden, n_experts, top_k, dtype, topk_idx,
                                         topk_gate, logits, reinterpret_cast<int32_t*>(ws + l.bc),
                                         reinterpret_cast<uint32_t*>(ws + l.header),
                                         reinterpret_cast<uint32_t*>(ws + l.flags), tables, valid_mask, nb, st);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "%s: router launch failed: %s", fn, hipGetErrorString(e));

  DispatchParams p;
  p.nb = nb;
  p.nbl = nb;
  p.seg_block[0] = 0;
  p.seg_block[1] = nb;
  p.topk_idx = topk_idx; p.valid = valid_mask; p.n_tokens = n_tokens;
  p.k = top_k; p.E = n_experts; p.table = tables; p.n_rep = tables + n_experts; p.rmax = 1;
  p.has_rep = 0; p.rr = nullptr; p.my_rank = 0; p.g2l = tables + 2 * n_experts;
  p.n_local = n_experts; p.counts = counts; p.offsets = offsets; p.perm = perm;
  p.row_of_entry = row_of_entry; p.dest = nullptr; p.route_counts = route_counts;
  p.status = nullptr;
  p.header = reinterpret_cast<uint32_t*>(ws + l.header);
  p.flags = reinterpret_cast<uint32_t*>(ws + l.flags);
  p.rr_snap = reinterpret_cast<int64_t*>(ws + l.rr_snap);
  p.bc = reinterpret_cast<int32_t*>(ws + l.bc);
  p.segtot = reinterpret_cast<int32_t*>(ws + l.segtot);
  p.scanned = p.nb > kScanBlocks ? 1 : 0;
  p.tag_polls = kTagPolls;
  p.dbg_withhold = -1;
  p.n_seg = 1;
  p.seg_entry[0] = 0;
  for (int s = 1; s <= kMaxSeg; ++s) p.seg_entry[s] = n_tokens * top_k;
  for (int s = 2; s <= kMaxSeg; ++s) p.seg_block[s] = p.nb;
  if (p.scanned) {
    prefix_kernel<<<n_experts, kScanThreads, 0, st>>>(p);
    MEP_CHECK_LAUNCH("mep_route_dispatch(prefix)");
  }
  scatter_kernel<false><<<p.nbl, kThreads, 0, st>>>(p);
  MEP_CHECK_LAUNCH("mep_route_dispatch(scatter)");
  return MEP_OK;
}

extern "C" int mep_dispatch_check(const void* workspace, void* stream) {
  clear_error();
  MEP_REQUIRE(workspace != nullptr, MEP_ERR_INVALID_ARG, "mep_dispatch_check: null workspace");
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_dispatch_check: %s", hipGetErrorString(e));
  uint32_t nbl = 0;
  e = hipMemcpy(&nbl, workspace, sizeof(nbl), hipMemcpyDeviceToHost);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_dispatch_check: %s", hipGetErrorString(e));
  MEP_REQUIRE(nbl >= 1 && nbl < (1u << 24), MEP_ERR_INVALID_ARG,
              "mep_dispatch_check: workspace holds no dispatch result");
  uint32_t acc = 0;
  uint32_t buf[1024];
  const char* flags = static_cast<const char*>(workspace) + kWsHeaderBytes;
  for (uint32_t i = 0; i < 2 * nbl; i += 1024) {
    const uint32_t n = (2 * nbl - i) < 1024 ? (2 * nbl - i) : 1024;
    e = hipMemcpy(buf, flags + sizeof(uint32_t) * i, sizeof(uint32_t) * n, hipMemcpyDeviceToHost);
    MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_dispatch_check: %s", hipGetErrorString(e));
    for (uint32_t j = 0; j < n; ++j) acc |= buf[j];
  }
  static_assert(kFlagRange == MEP_DISPATCH_STATUS_RANGE && kFlagResident == MEP_DISPATCH_STATUS_NOT_RESIDENT &&
                    kFlagReplicas == MEP_DISPATCH_STATUS_REPLICAS && kFlagBarrier == MEP_DISPATCH_STATUS_BARRIER,
                "status bits of the header");
  MEP_REQUIRE(!(acc & kFlagBarrier), MEP_ERR_HIP,
              "mep_route_dispatch: a workgroup gave up waiting for the others' histogram rows (workgroups not "
              "resident together); results invalid");
  MEP_REQUIRE(!(acc & kFlagReplicas), MEP_ERR_INVALID_ARG,
              "mep_dispatch: n_rep[e] outside [1, rmax] for some expert (every expert needs an owner)");
  MEP_REQUIRE(!(acc & kFlagRange), MEP_ERR_EXPERT_RANGE,
              "mep_dispatch: expert id outside [0, n_experts) dropped");
  MEP_REQUIRE(!(acc & kFlagResident), MEP_ERR_NOT_RESIDENT,
              "mep_dispatch: entry routed to this rank for a non-resident expert dropped");
  return MEP_OK;
}
