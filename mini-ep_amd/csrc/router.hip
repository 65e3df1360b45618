// Fused router for the GraniteMoE MoE block (gfx950).
//
// Replaces modeling.py:193-195:
//     router_logits = x_flat @ W_r.T
//     topk_logits, topk_idx = router_logits.topk(k, dim=-1)      (descending)
//     topk_gate = softmax(topk_logits.float(), dim=-1).to(x.dtype)
//
// One wavefront owns 16 tokens.  The 16 x E logit tile is computed on the
// matrix cores (bf16: v_mfma_f32_16x16x32_bf16, fp32: v_mfma_f32_16x16x4_f32)
// with fp32 accumulation, x rows streamed straight from HBM into the MFMA A
// operand and W_r read through the L1/L2 (64 KiB, shared by every wave).
// The tile then goes to LDS and every (token, expert) pair gets its rank
//     rank(e) = #{e' : key(e') > key(e)  or  (key(e') == key(e) and e' < e)}
// which is a total order: descending logits, lower expert id first among
// equal logits (NaN ranks above every number, -0.0 == +0.0).  Pairs with
// rank < k land directly in output slot `rank`; no sort, no atomics, so the
// selection is deterministic and independent of the launch shape.
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
// write topk_idx / gate for tokens t0 .. t0+rows-1.  Executed by one wave.
// `sel_val` / `sel_idx` are LDS scratch of rows * k entries, `rsum` of rows.
template <int GATE_DT>
__device__ void select_topk_from_lds(const float* lg, int ld, int rows, int E, int k,
                                     int64_t t0, int64_t n_tokens, float* sel_val,
                                     int* sel_idx, float* rsum, int64_t* topk_idx,
                                     typename Elem<GATE_DT>::T* gate) {
  const int lane = lane_id();
  const int pairs = rows * E;
  for (int p = lane; p < pairs; p += 64) {
    const int t = p / E, e = p - t * E;
    const float* row = lg + t * ld;
    const uint32_t ke = order_key(row[e]);
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const uint32_t kj = order_key(row[j]);
      rank += (kj > ke) | ((kj == ke) & (j < e));
    }
    if (rank < k) {
      sel_val[t * k + rank] = row[e];
      sel_idx[t * k + rank] = e;
    }
  }
  __syncthreads();
  // softmax denominator per token, summed in slot order
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

// Logit tile of 16 tokens x (16*NF) experts on the matrix cores.
// K is walked in blocks of 512 bytes per row; lane group g = lane/16 owns the
// bytes [128g, 128g+128) of each block (8 chunks of 16 B).  Chunk j of every
// group feeds MFMA step j; A and B use the same permutation of K, so the
// accumulated dot products are unchanged.
template <int DT, int NF>
__global__ __launch_bounds__(64) void router_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                    const typename Elem<DT>::T* __restrict__ w,
                                                    int64_t n_tokens, int hidden, int k,
                                                    int64_t* __restrict__ topk_idx,
                                                    typename Elem<DT>::T* __restrict__ gate,
                                                    float* __restrict__ logits) {
  typedef typename Elem<DT>::T T;
  constexpr int E = NF * 16;
  constexpr int kElemsPerChunk = 16 / Elem<DT>::kBytes;   // 8 bf16 or 4 fp32
  constexpr int kBlockElems = 32 * kElemsPerChunk;        // 4 groups x 8 chunks
  __shared__ float lg[kRowsPerWave][E + 1];
  __shared__ float sel_val[kRowsPerWave * 64];
  __shared__ int sel_idx[kRowsPerWave * 64];
  __shared__ float rsum[kRowsPerWave];

  const int lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRowsPerWave;
  int64_t tok = t0 + r;
  if (tok >= n_tokens) tok = n_tokens - 1;   // in-bounds read, result discarded
  const T* xrow = x + tok * hidden + g * (8 * kElemsPerChunk);
  const T* wrow[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) wrow[nf] = w + (nf * 16 + r) * hidden + g * (8 * kElemsPerChunk);

  f32x4 acc[NF];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf) acc[nf] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < hidden; kb += kBlockElems) {
    u32x4 xa[8];
    u32x4 wb[NF][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xa[j] = *reinterpret_cast<const u32x4*>(xrow + kb + j * kElemsPerChunk);
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        wb[nf][j] = *reinterpret_cast<const u32x4*>(wrow[nf] + kb + j * kElemsPerChunk);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int nf = 0; nf < NF; ++nf) {
        if constexpr (DT == MEP_DTYPE_BF16) {
          acc[nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, xa[j]), __builtin_bit_cast(bf16x8, wb[nf][j]), acc[nf], 0, 0, 0);
        } else {
          const float* xf = reinterpret_cast<const float*>(&xa[j]);
          const float* wf = reinterpret_cast<const float*>(&wb[nf][j]);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[nf] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[q], wf[q], acc[nf], 0, 0, 0);
        }
      }
    }
  }
  // C layout of the 16x16 MFMA: lane holds rows 4*(lane/16) + i, column lane%16.
#pragma unroll
  for (int nf = 0; nf < NF; ++nf)
#pragma unroll
    for (int i = 0; i < 4; ++i) lg[4 * g + i][nf * 16 + r] = acc[nf][i];
  __syncthreads();

  if (logits != nullptr) {
    for (int p = lane; p < kRowsPerWave * E; p += 64) {
      const int t = p / E;
      if (t0 + t < n_tokens) logits[(t0 + t) * E + (p - t * E)] = lg[t][p - t * E];
    }
  }
  select_topk_from_lds<DT>(&lg[0][0], E + 1, kRowsPerWave, E, k, t0, n_tokens, sel_val, sel_idx,
                           rsum, topk_idx, gate);
}

// Top-k + softmax of precomputed logits: one wave per `rows` tokens.
template <int GATE_DT>
__global__ __launch_bounds__(64) void topk_softmax_kernel(const float* __restrict__ logits,
                                                          int64_t n_tokens, int E, int k, int rows,
                                                          int64_t* __restrict__ topk_idx,
                                                          typename Elem<GATE_DT>::T* __restrict__ gate) {
  __shared__ float lg[1024 + 64];
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
  select_topk_from_lds<GATE_DT>(lg, ld, rows, E, k, t0, n_tokens, sel_val, sel_idx, rsum,
                                topk_idx, gate);
}

template <int DT>
hipError_t launch_router(const void* x, const void* w, int64_t n, int hidden, int E, int k,
                         int64_t* idx, void* gate, float* logits, hipStream_t stream) {
  typedef typename Elem<DT>::T T;
  const dim3 grid(static_cast<unsigned>((n + kRowsPerWave - 1) / kRowsPerWave));
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* gp = static_cast<T*>(gate);
  switch (E) {
    case 16: router_kernel<DT, 1><<<grid, 64, 0, stream>>>(xp, wp, n, hidden, k, idx, gp, logits); break;
    case 32: router_kernel<DT, 2><<<grid, 64, 0, stream>>>(xp, wp, n, hidden, k, idx, gp, logits); break;
    case 64: router_kernel<DT, 4><<<grid, 64, 0, stream>>>(xp, wp, n, hidden, k, idx, gp, logits); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace
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
  hipError_t e = dtype == MEP_DTYPE_BF16
                     ? launch_router<MEP_DTYPE_BF16>(x, w_router, n_tokens, hidden, n_experts, top_k,
                                                     topk_idx, topk_gate, logits, s)
                     : launch_router<MEP_DTYPE_F32>(x, w_router, n_tokens, hidden, n_experts, top_k,
                                                    topk_idx, topk_gate, logits, s);
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
