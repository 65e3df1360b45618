// Device code of the fused router (router.hip), shared with the decode
// layer's one launch (grouped_swiglu.hip) so both route with the same
// instructions: the total-order keys, the top-k selections, the logit tile
// of the GraniteMoE shape and the tail that writes indices and gates.
#pragma once

#include "common.h"

namespace mep {
namespace {

constexpr int kRowsPerWave = 16;

// Total-order key of a float: larger float -> larger key; NaN above +inf;
// -0.0 maps to the key of +0.0 so that equal floats have equal keys.
__device__ __forceinline__ uint32_t order_key(float v) {
  if (v != v) return 0xffffffffu;
  if (v == 0.0f) v = 0.0f;
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Select the top-k of the `rows` x E fp32 tile in LDS (row stride `ld`) and
// write topk_idx / gate for tokens t0 .. t0+rows-1.  Executed by one wave on its
// own LDS slices; every wave of the workgroup calls it (it contains barriers).
// Each logit gets the 64-bit key (order_key << 32) | ~e: unique per expert and
// ordered exactly as "larger logit first, lower id among equals", so
// rank(e) = #{j : key_j > key_e} -- one 64-bit compare and one add per j.
// `keys` is LDS scratch of rows x kld 64-bit words (kld even), `sel_val` /
// `sel_idx` rows * k entries, `rsum` rows.  EC is the expert count as a
// compile-time constant (0 = runtime E, one key read at a time).
template <int GATE_DT, int EC, int KC>
__device__ void select_topk_from_lds(const float* lg, int ld, int rows, int E_rt, int k_rt,
                                     int64_t t0, int64_t n_tokens, float* sel_val,
                                     int* sel_idx, float* rsum, int64_t* topk_idx,
                                     typename Elem<GATE_DT>::T* gate, uint64_t* keys, int kld) {
  const int lane = lane_id();
  const int E = EC > 0 ? EC : E_rt;
  const int k = KC > 0 ? KC : k_rt;
  const int pairs = rows * E;
  for (int p = lane; p < pairs; p += 64) {
    const int t = p / E, e = p - t * E;
    keys[t * kld + e] = (static_cast<uint64_t>(order_key(lg[t * ld + e])) << 32) | static_cast<uint32_t>(~e);
  }
  __syncthreads();
  for (int p = lane; p < pairs; p += 64) {
    const int t = p / E, e = p - t * E;
    const uint64_t* row = keys + t * kld;
    const uint64_t ke = row[e];
    int rank = 0;
    if constexpr (EC > 0) {
      uint64_t kv[EC];
#pragma unroll
      for (int j2 = 0; j2 < EC / 2; ++j2) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(row + 2 * j2);
        kv[2 * j2] = (static_cast<uint64_t>(v.y) << 32) | v.x;
        kv[2 * j2 + 1] = (static_cast<uint64_t>(v.w) << 32) | v.z;
      }
#pragma unroll
      for (int j = 0; j < EC; ++j) rank += kv[j] > ke;
    } else {
      for (int j = 0; j < E; ++j) rank += row[j] > ke;
    }
    if (rank < k) {
      sel_val[t * k + rank] = lg[t * ld + e];
      sel_idx[t * k + rank] = e;
    }
  }
  __syncthreads();
  // softmax over each token's k selected logits, summed in slot order
  if constexpr (KC > 0) {
    // one lane per token: the k values in registers (16-byte LDS reads)
    for (int t = lane; t < rows; t += 64) {
      float v[KC];
      if constexpr (KC % 4 == 0) {
#pragma unroll
        for (int q = 0; q < KC / 4; ++q) {
          const f32x4 w4 = *reinterpret_cast<const f32x4*>(sel_val + t * KC + 4 * q);
          v[4 * q] = w4.x; v[4 * q + 1] = w4.y; v[4 * q + 2] = w4.z; v[4 * q + 3] = w4.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < KC; ++q) v[q] = sel_val[t * KC + q];
      }
      float ex[KC], sum = 0.0f;
#pragma unroll
      for (int q = 0; q < KC; ++q) { ex[q] = expf(v[q] - v[0]); sum += ex[q]; }
      if (t0 + t < n_tokens) {
#pragma unroll
        for (int q = 0; q < KC; ++q) {
          topk_idx[(t0 + t) * KC + q] = sel_idx[t * KC + q];
          gate[(t0 + t) * KC + q] = Elem<GATE_DT>::from_f32(ex[q] / sum);
        }
      }
    }
  } else {
    for (int t = lane; t < rows; t += 64) {
      const float m = sel_val[t * k];
      float s = 0.0f;
      for (int j = 0; j < k; ++j) s += expf(sel_val[t * k + j] - m);
      rsum[t] = s;
    }
    __syncthreads();
    for (int p = lane; p < rows * k; p += 64) {
      const int t = p / k;
      if (t0 + t >= n_tokens) continue;
      const float g = expf(sel_val[p] - sel_val[t * k]) / rsum[t];
      topk_idx[(t0 + t) * k + (p - t * k)] = sel_idx[p];
      gate[(t0 + t) * k + (p - t * k)] = Elem<GATE_DT>::from_f32(g);
    }
  }
}

// Float of a total-order key (inverse of order_key; -0.0 comes back as +0.0,
// NaN as NaN).
__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t u = static_cast<uint32_t>(key >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// Descending compare-exchange of two keys.
__device__ __forceinline__ void cx_desc(uint64_t& a, uint64_t& b) {
  const bool keep = a > b;
  const uint64_t hi = keep ? a : b, lo = keep ? b : a;
  a = hi;
  b = lo;
}

// The key of the lane XOR 1 or XOR 2 within this lane's group of four
// (DPP quad_perm [1,0,3,2] / [2,3,0,1]).
template <int CTRL>
__device__ __forceinline__ uint64_t quad_swap(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, 0xF, 0xF,
                                             false);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// k[0..7] sorted descending, the four lanes of a token each holding 8 of its
// 32 keys: every lane sorts its 8 (Batcher's 19-comparator network), then
// takes the top 8 of its list and the partner lane's twice (partner = lane
// XOR 1, then XOR 2): c[i] = max(a[i], b[7-i]) is the top 8 of the 16 as a
// bitonic sequence, and a 12-comparator bitonic merge sorts it.  All four
// lanes end with the token's top 8 in order (keys are distinct).
__device__ __forceinline__ void top8_of_32(uint64_t (&k)[8]) {
  cx_desc(k[0], k[2]); cx_desc(k[1], k[3]); cx_desc(k[4], k[6]); cx_desc(k[5], k[7]);
  cx_desc(k[0], k[4]); cx_desc(k[1], k[5]); cx_desc(k[2], k[6]); cx_desc(k[3], k[7]);
  cx_desc(k[0], k[1]); cx_desc(k[2], k[3]); cx_desc(k[4], k[5]); cx_desc(k[6], k[7]);
  cx_desc(k[2], k[4]); cx_desc(k[3], k[5]);
  cx_desc(k[1], k[4]); cx_desc(k[3], k[6]);
  cx_desc(k[1], k[2]); cx_desc(k[3], k[4]); cx_desc(k[5], k[6]);
#pragma unroll
  for (int level = 0; level < 2; ++level) {
    uint64_t o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = level == 0 ? quad_swap<0xB1>(k[i]) : quad_swap<0x4E>(k[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = k[i] > o[7 - i] ? k[i] : o[7 - i];
    cx_desc(k[0], k[4]); cx_desc(k[1], k[5]); cx_desc(k[2], k[6]); cx_desc(k[3], k[7]);
    cx_desc(k[0], k[2]); cx_desc(k[1], k[3]); cx_desc(k[4], k[6]); cx_desc(k[5], k[7]);
    cx_desc(k[0], k[1]); cx_desc(k[2], k[3]); cx_desc(k[4], k[5]); cx_desc(k[6], k[7]);
  }
}

// Optional histogram output of the router (the fused route + dispatch path):
// per workgroup of 64 tokens, entries of each expert among its valid tokens,
// which is the dispatch's per-block histogram when top_k = 8 (64 tokens x 8
// slots = one 512-entry dispatch block).
struct RouterHist {
  int32_t* bc;              // (n_blocks, E) histograms, or NULL: no histogram
  uint32_t* header;         // dispatch workspace header: [0] = n_blocks
  uint32_t* flags;          // the dispatch's per-block count flags (written 0)
  int32_t* tables;          // table (E) = 0, n_rep (E) = 1, g2l (E) = identity
  const uint8_t* valid;     // (N,) or NULL
  int n_blocks;
};

// Top-KC of a 16 x EC tile (compile-time EC and KC, both multiples of 4) by
// one wave, with no workgroup barrier: lane 4 t + g owns token t and experts
// g*EC/4 .. (g+1)*EC/4 - 1.  Every key is the 64-bit (order_key << 32 | ~e)
// of select_topk_from_lds: unique per expert and ordered exactly as "larger
// logit first, lower id among equals".  EC = 32, KC = 8: sorting networks in
// registers (top8_of_32).  Otherwise each lane writes its experts' keys to the
// wave's LDS rows, reads its token's whole row once and ranks its own experts
// against it; rank < KC goes to slot `rank`.  Then lane (t, g) writes slots
// g*KC/4 .. of token t; the softmax is computed by every lane of the token in
// the same order (max = slot 0, exp of differences summed in slot order), so
// the gates equal the general path's bit for bit.  All data is wave-private,
// so s_waitcnt on LDS orders it.  With a histogram output, each lane adds
// its slots' experts of valid tokens to the workgroup's `s_cnt`.
template <int GATE_DT, int EC, int KC>
__device__ void select_topk_wave(const float* lg, int ld, int64_t t0, int64_t n_tokens, float* sel_val,
                                 int* sel_idx, int64_t* topk_idx, typename Elem<GATE_DT>::T* gate,
                                 uint64_t* keys, int kld, const RouterHist& hist, int* s_cnt,
                                 int* sel_out) {
  static_assert(EC % 4 == 0 && KC % 4 == 0 && KC <= EC && kRowsPerWave * 4 == 64, "lane layout");
  constexpr int EG = EC / 4, SG = KC / 4;
  const int lane = lane_id();
  const int t = lane >> 2, g = lane & 3;
  int my_idx[SG];
  float my_gate[SG];
  if constexpr (EC == 32 && KC == 8) {
    uint64_t k[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = g * 8 + i;
      k[i] = (static_cast<uint64_t>(order_key(lg[t * ld + e])) << 32) | static_cast<uint32_t>(~e);
    }
    top8_of_32(k);
    float sv[8], ex[8], sum = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) sv[q] = key_value(k[q]);
#pragma unroll
    for (int q = 0; q < 8; ++q) { ex[q] = expf(sv[q] - sv[0]); sum += ex[q]; }
#pragma unroll
    for (int h = 0; h < SG; ++h) {
      uint64_t kq = k[h];
      float eq = ex[h];
#pragma unroll
      for (int gg = 1; gg < 4; ++gg)
        if (g == gg) { kq = k[gg * SG + h]; eq = ex[gg * SG + h]; }
      my_idx[h] = static_cast<int>(~static_cast<uint32_t>(kq));
      my_gate[h] = eq / sum;
    }
  } else {
    float v[EG];
    uint64_t ke[EG];
#pragma unroll
    for (int i = 0; i < EG; ++i) {
      const int e = g * EG + i;
      v[i] = lg[t * ld + e];
      ke[i] = (static_cast<uint64_t>(order_key(v[i])) << 32) | static_cast<uint32_t>(~e);
      keys[t * kld + e] = ke[i];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0): the row is in LDS
    __builtin_amdgcn_wave_barrier();
    int rank[EG];
#pragma unroll
    for (int i = 0; i < EG; ++i) rank[i] = 0;
    const uint64_t* row = keys + t * kld;
#pragma unroll
    for (int j2 = 0; j2 < EC / 2; ++j2) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(row + 2 * j2);
      const uint64_t a = (static_cast<uint64_t>(q.y) << 32) | q.x;
      const uint64_t b = (static_cast<uint64_t>(q.w) << 32) | q.z;
#pragma unroll
      for (int i = 0; i < EG; ++i) rank[i] += (a > ke[i]) + (b > ke[i]);
    }
#pragma unroll
    for (int i = 0; i < EG; ++i) {
      if (rank[i] < KC) {
        sel_val[t * KC + rank[i]] = v[i];
        sel_idx[t * KC + rank[i]] = g * EG + i;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    float sv[KC];
#pragma unroll
    for (int q = 0; q < KC / 4; ++q) {
      const f32x4 w4 = *reinterpret_cast<const f32x4*>(sel_val + t * KC + 4 * q);
      sv[4 * q] = w4.x; sv[4 * q + 1] = w4.y; sv[4 * q + 2] = w4.z; sv[4 * q + 3] = w4.w;
    }
    float ex[KC], sum = 0.0f;
#pragma unroll
    for (int q = 0; q < KC; ++q) { ex[q] = expf(sv[q] - sv[0]); sum += ex[q]; }
#pragma unroll
    for (int h = 0; h < SG; ++h) {
      my_idx[h] = sel_idx[t * KC + g * SG + h];
      my_gate[h] = ex[g * SG + h] / sum;
    }
  }
  if (sel_out != nullptr) {
    // the experts of this lane's slots for the fused dispatch: -1 for tokens
    // past the end or masked out
    const bool counted = t0 + t < n_tokens && (hist.valid == nullptr || hist.valid[t0 + t] != 0);
#pragma unroll
    for (int h = 0; h < SG; ++h) sel_out[h] = counted ? my_idx[h] : -1;
  }
  if (t0 + t < n_tokens) {
#pragma unroll
    for (int h = 0; h < SG; ++h) {
      topk_idx[(t0 + t) * KC + g * SG + h] = my_idx[h];
      gate[(t0 + t) * KC + g * SG + h] = Elem<GATE_DT>::from_f32(my_gate[h]);
    }
    if (hist.bc != nullptr && (hist.valid == nullptr || hist.valid[t0 + t] != 0)) {
#pragma unroll
      for (int h = 0; h < SG; ++h) atomicAdd(&s_cnt[my_idx[h]], 1);
    }
  }
}

// The end of every router kernel: the wave's 16 x E logit tile (MFMA C
// layout: lane holds rows 4*(lane/16) + i, column lane%16 of each 16-column
// fragment) goes to the wave's LDS rows, optionally to `logits`, then the
// selection, the gates and (fused path) the workgroup's dispatch histogram.
// Called by every thread of the workgroup (it contains barriers).
template <int DT, int E, int KC>
__device__ __forceinline__ void router_tail(const f32x4* acc, float (*lgw)[E + 1], uint64_t* keysw, float* sel_valw,
                                            int* sel_idxw, float* rsumw, int* s_cnt, int64_t t0, int64_t n_tokens,
                                            int k, int64_t* __restrict__ topk_idx,
                                            typename Elem<DT>::T* __restrict__ gate, float* __restrict__ logits,
                                            const RouterHist& hist, int* sel_out = nullptr) {
  constexpr int NF = E / 16;
  const int tid = threadIdx.x, lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int nf = 0; nf < NF; ++nf)
#pragma unroll
    for (int i = 0; i < 4; ++i) lgw[4 * g + i][nf * 16 + r] = acc[nf][i];
  constexpr bool kWaveSelect = KC > 0 && KC % 4 == 0 && E % 4 == 0;
  if constexpr (kWaveSelect) {
    // the tile is this wave's own: order the LDS writes before the reads
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
  } else {
    __syncthreads();
  }
  if (logits != nullptr) {
    for (int p = lane; p < kRowsPerWave * E; p += 64) {
      const int t = p / E;
      if (t0 + t < n_tokens) logits[(t0 + t) * E + (p - t * E)] = lgw[t][p - t * E];
    }
  }
  if constexpr (kWaveSelect) {
    select_topk_wave<DT, E, KC>(&lgw[0][0], E + 1, t0, n_tokens, sel_valw, sel_idxw, topk_idx, gate, keysw, E + 2,
                                hist, s_cnt, sel_out);
    if (hist.bc != nullptr) {
      // the workgroup's histogram is the dispatch's histogram of block b
      __syncthreads();
      const int b = blockIdx.x;
      if (tid < E) hist.bc[static_cast<int64_t>(b) * E + tid] = s_cnt[tid];
      if (tid == 0) hist.flags[b] = 0u;
      if (b == 0) {
        if (tid == 0) hist.header[0] = static_cast<uint32_t>(hist.n_blocks);
        if (tid < E) {
          hist.tables[tid] = 0;                    // table[e, 0]: every expert on rank 0
          hist.tables[E + tid] = 1;                // n_rep[e]
          hist.tables[2 * E + tid] = tid;          // g2l: identity
        }
      }
    }
  } else {
    select_topk_from_lds<DT, E, KC>(&lgw[0][0], E + 1, kRowsPerWave, E, k, t0, n_tokens, sel_valw, sel_idxw, rsumw,
                                    topk_idx, gate, keysw, E + 2);
  }
}

// Logit tiles on the matrix cores.  A workgroup of kWaves waves owns
// kWaves x 16 tokens; W_r is staged through LDS in K segments of at most
// kSegBytes (all waves share it), x is streamed straight from HBM into the
// MFMA A operand with every load of a segment issued before its first MFMA.
// K is walked in blocks of 512 bytes per row (32 chunks of 16 B); MFMA step j
// of a block takes chunk 4j + g in lane group g = lane/16 (the MFMA's own K
// order), so one load instruction reads 64 contiguous bytes of each of the 16
// rows.  LDS rows of W are padded by 16 B, which spreads the 16 rows of a
// fragment read over distinct banks.
constexpr int kWaves = 4;
constexpr int kSegBytes = 64 * 1024;

// The router of the GraniteMoE shape: bf16, 32 experts, top-8, hidden a
// multiple of 1024 (NSEG segments of 1024), everything else as router_kernel.
// With the hidden size a compile-time constant every address is a base plus
// an immediate, so per K segment the workgroup issues its W_r loads first
// (16 x 16 B per thread), then each wave its 16 x rows (32 x 16 B per lane,
// all in flight), stages W_r in LDS as soon as its loads have landed, and
// runs the MFMAs of each 256-wide K block as that block of x arrives, with
// the block's 16 weight fragments read from LDS before its 16 MFMAs (read
// and multiply interleaved one by one, the LDS latency is paid 64 times).
// One wave's 16 x 32 logit tile of the GraniteMoE router shape (bf16, 32
// experts, hidden 1024 * NSEG); `ws` is the workgroup's LDS copy of one W_r
// segment.  Called by every thread of the workgroup (it contains barriers).
template <int NSEG>
__device__ __forceinline__ void router32_logits(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                int64_t n_tokens, int64_t t0, unsigned char* ws, f32x4 (&acc)[2]) {
  constexpr int NF = 2, H = 1024 * NSEG;
  constexpr int kRowStride = 1024 * 2 + 16;        // bytes of one W_r row segment in LDS (16 B pad: conflict-free)
  const int tid = threadIdx.x, lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  int64_t tok = t0 + r;
  if (tok >= n_tokens) tok = n_tokens - 1;        // in-bounds read, result discarded
  const uint16_t* xrow = x + tok * H + g * 8;
  // W_r chunk i of this thread: row (tid >> 7) + 2 i, 16 bytes at column (tid & 127) * 8
  const uint16_t* wrow = w + static_cast<int64_t>(tid >> 7) * H + (tid & 127) * 8;
  const int wlds = (tid >> 7) * kRowStride + (tid & 127) * 16;
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) acc[nf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int seg = 0; seg < NSEG; ++seg) {
    u32x4 wt[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) wt[i] = *reinterpret_cast<const u32x4*>(wrow + 2 * i * H + seg * 1024);
    asm volatile("" ::: "memory");               // the weight loads go out first
    u32x4 xa[4][8];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < 8; ++j) xa[b][j] = *reinterpret_cast<const u32x4*>(xrow + seg * 1024 + b * 256 + j * 32);
    if (seg > 0) __syncthreads();                 // the previous segment's fragment reads are done
#pragma unroll
    for (int i = 0; i < 16; ++i) *reinterpret_cast<u32x4*>(ws + wlds + 2 * i * kRowStride) = wt[i];
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      u32x4 wb[8][NF];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int nf = 0; nf < NF; ++nf)
          wb[j][nf] = *reinterpret_cast<const u32x4*>(ws + (nf * 16 + r) * kRowStride + (b * 256 + (4 * j + g) * 8) * 2);
      __builtin_amdgcn_sched_barrier(0);          // all 16 fragment reads issued before the MFMAs
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int nf = 0; nf < NF; ++nf)
          acc[nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[b][j]),
                                                            __builtin_bit_cast(bf16x8, wb[j][nf]), acc[nf], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

constexpr int kRowStride32 = 1024 * 2 + 16;

// Lanes whose expert in key array `bits` (the 5 id-bit ballots, `present` =
// lanes with an expert) equals v.
__device__ __forceinline__ uint64_t lanes_with(int v, const uint64_t (&bits)[5], uint64_t present) {
  uint64_t m = present;
#pragma unroll
  for (int i = 0; i < 5; ++i) m &= ((v >> i) & 1) ? bits[i] : ~bits[i];
  return m;
}

}  // namespace
}  // namespace mep
