// Combine / unpermute for the MoE block.
//
// Replaces the gate multiply and scatter_combine of the reference
// (modeling.py:144, :120-128; ep.py:239-242):
//     gated = outs * topk_gate[keep].unsqueeze(1)
//     buf = zeros(n, k, H); buf[token_ids, slot_ids] = gated; out = buf.sum(dim=1)
// GEMM-2 already wrote every expert output row to its (token, slot) cell of
// y_entries (the reference's `buf` layout), so the combine is a streaming
// reduction: each thread owns 16 bytes of one token's output row, loads the
// k cells of that token (k x 16 B, all in flight), and sums gate * y in slot
// order in fp32 -- the same fixed order on every run, no atomics.
//
// The expert-parallel return path (ep.py:237-242: inv[order] = arange,
// gated = back[inv] * gate, scatter_combine) is the same reduction with the
// (token, slot) row read through `row_of_entry` (the inverse of the
// destination sort): mep_combine_rows.  Its send-buffer counterpart,
// mep_gather_rows (ep.py:226, x_flat[token_ids[order]]), copies the rows of x
// in send order.
#include "combine_dev.h"
#include "common.h"

namespace mep {
namespace {

constexpr int kThreads = 256;
// combine8_kernel: one wave per block (half a 1024-wide bf16 row); against
// 256-thread blocks it streams y about 2 % faster (52.8 -> 51.8 us at T=16384)
constexpr int kCombine8Threads = 64;
constexpr int kMaxK = 32;

// Thread q of the launch owns 16-byte chunk c = q % cpr of token t = q / cpr
// (cpr = 16-byte chunks per row, any row length that is a multiple of 16 B;
// n_tokens * cpr < 2^31, checked by the entry point).
template <int NT = kThreads>
__device__ __forceinline__ bool chunk_of_thread(int64_t n_tokens, int cpr, int64_t& t, int& c) {
  const uint32_t q = blockIdx.x * static_cast<uint32_t>(NT) + threadIdx.x;
  t = q / static_cast<uint32_t>(cpr);
  c = static_cast<int>(q - static_cast<uint32_t>(t) * cpr);
  return t < n_tokens;
}

template <int DT>
__device__ __forceinline__ void accumulate_cell(float* acc, float g, const u32x4& v) {
  if constexpr (DT == MEP_DTYPE_BF16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += g * bf16_to_f32(static_cast<uint16_t>(w[q] & 0xffffu));
      acc[2 * q + 1] += g * bf16_to_f32(static_cast<uint16_t>(w[q] >> 16));
    }
  } else {
    acc[0] += g * __uint_as_float(v.x);
    acc[1] += g * __uint_as_float(v.y);
    acc[2] += g * __uint_as_float(v.z);
    acc[3] += g * __uint_as_float(v.w);
  }
}

// Any k: the token's row_of_entry entries and gates are read by each of its
// threads (the same addresses across the row's threads, served once by the
// cache); cells are summed in slot order.  INDEXED: cell (t, s) is row
// row_of_entry[t*k+s] of y (the expert-parallel return path); otherwise it is
// row t*k+s (the (token, slot) layout GEMM-2 writes).
template <int DT, bool INDEXED>
__global__ __launch_bounds__(kThreads) void combine_kernel(const typename Elem<DT>::T* __restrict__ y,
                                                           const typename Elem<DT>::T* __restrict__ gate,
                                                           const int32_t* __restrict__ row_of_entry,
                                                           const uint8_t* __restrict__ valid,
                                                           int64_t n_tokens, int k, int hidden,
                                                           typename Elem<DT>::T* __restrict__ out) {
  constexpr int EPC = 16 / Elem<DT>::kBytes;
  int64_t t;
  int c;
  if (!chunk_of_thread(n_tokens, hidden / EPC, t, c)) return;
  const bool tok_ok = valid == nullptr || valid[t] != 0;
  bool poison = false;                                  // an entry of a dispatch that gave up: NaN
  float acc[EPC];
#pragma unroll
  for (int q = 0; q < EPC; ++q) acc[q] = 0.0f;
  if (tok_ok) {
#pragma unroll 8
    for (int s = 0; s < k; ++s) {
      const int32_t row = row_of_entry[t * k + s];
      poison |= row == kPoisonRow;
      if (row < 0) continue;                            // cell computed elsewhere
      const float g = Elem<DT>::to_f32(gate[t * k + s]);
      const int64_t cell = INDEXED ? static_cast<int64_t>(row) : t * k + s;
      const u32x4 v = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(y + cell * hidden + c * EPC));   // read once
      accumulate_cell<DT>(acc, g, v);
    }
  }
#pragma unroll
  for (int q = 0; q < EPC; ++q) acc[q] = poison ? __builtin_nanf("") : acc[q];
  *reinterpret_cast<u32x4*>(out + t * hidden + c * EPC) = pack_row_chunk<DT>(acc);
}

// k = 8, (token, slot) layout: combine8_chunk (combine_dev.h), the same
// slot-order sum as combine_kernel, with y read by non-temporal loads.
template <int DT>
__global__ __launch_bounds__(kCombine8Threads) void combine8_kernel(const typename Elem<DT>::T* __restrict__ y,
                                                            const typename Elem<DT>::T* __restrict__ gate,
                                                            const int32_t* __restrict__ row_of_entry,
                                                            const uint8_t* __restrict__ valid,
                                                            int64_t n_tokens, int hidden,
                                                            typename Elem<DT>::T* __restrict__ out) {
  typedef typename Elem<DT>::T T;
  constexpr int EPC = 16 / Elem<DT>::kBytes;
  int64_t t;
  int c;
  if (!chunk_of_thread<kCombine8Threads>(n_tokens, hidden / EPC, t, c)) return;
  // y is read exactly once: non-temporal loads keep these 268 MB (T=16384)
  // from evicting x and the weights from the 256 MB MALL before the next layer
  combine8_chunk<DT>(y, gate, row_of_entry, valid, t, c, hidden, out, [](const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  });
}

// out[i, :] = x[perm[i] / top_k, :] (and ids_out[i] = topk_flat[perm[i]]):
// one thread per 16 bytes of an output row.
template <int DT>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                               const int32_t* __restrict__ perm,
                                                               int64_t n_rows, int top_k, int hidden,
                                                               const int64_t* __restrict__ topk_flat,
                                                               int64_t* __restrict__ ids_out,
                                                               typename Elem<DT>::T* __restrict__ out) {
  constexpr int EPC = 16 / Elem<DT>::kBytes;
  const int cpr = hidden / EPC;                         // 16-byte chunks per row
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t i = q / cpr;
  if (i >= n_rows) return;
  const int c = static_cast<int>(q - i * cpr);
  const int32_t f = perm[i];
  const int64_t src = f / top_k;
  *reinterpret_cast<u32x4*>(out + i * hidden + c * EPC) =
      *reinterpret_cast<const u32x4*>(x + src * hidden + c * EPC);
  if (ids_out != nullptr && c == 0) ids_out[i] = topk_flat[f];
}

template <bool INDEXED>
int combine_entry(const char* fn, const void* y, const void* topk_gate, const int32_t* row_of_entry,
                  const uint8_t* valid_mask, int64_t n_tokens, int32_t top_k, int32_t hidden, int32_t dtype,
                  void* out, void* stream) {
  clear_error();
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "%s: unknown dtype %d", fn, dtype);
  MEP_REQUIRE(n_tokens >= 0 && top_k >= 1 && top_k <= kMaxK, MEP_ERR_INVALID_ARG,
              "%s: bad n_tokens / top_k %d", fn, top_k);
  const int epc = 16 / dtype_bytes(dtype);
  MEP_REQUIRE(hidden > 0 && hidden % epc == 0, MEP_ERR_UNSUPPORTED,
              "%s: hidden %d is not a multiple of %d for this dtype", fn, hidden, epc);
  const int64_t cpr = hidden / epc;                    // threads per token row
  MEP_REQUIRE(n_tokens * cpr < (int64_t(1) << 31), MEP_ERR_UNSUPPORTED,
              "%s: n_tokens * hidden too large", fn);
  if (n_tokens == 0) return MEP_OK;
  MEP_REQUIRE(y && topk_gate && row_of_entry && out, MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
  MEP_REQUIRE((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
              MEP_ERR_INVALID_ARG, "%s: y / out must be 16-byte aligned", fn);
  const dim3 grid(static_cast<unsigned>((n_tokens * cpr + kThreads - 1) / kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!INDEXED && top_k == 8) {
    const dim3 grid8(static_cast<unsigned>((n_tokens * cpr + kCombine8Threads - 1) / kCombine8Threads));
    if (dtype == MEP_DTYPE_BF16)
      combine8_kernel<MEP_DTYPE_BF16><<<grid8, kCombine8Threads, 0, s>>>(
          static_cast<const uint16_t*>(y), static_cast<const uint16_t*>(topk_gate), row_of_entry, valid_mask,
          n_tokens, hidden, static_cast<uint16_t*>(out));
    else
      combine8_kernel<MEP_DTYPE_F32><<<grid8, kCombine8Threads, 0, s>>>(
          static_cast<const float*>(y), static_cast<const float*>(topk_gate), row_of_entry, valid_mask,
          n_tokens, hidden, static_cast<float*>(out));
  } else if (dtype == MEP_DTYPE_BF16)
    combine_kernel<MEP_DTYPE_BF16, INDEXED><<<grid, kThreads, 0, s>>>(
        static_cast<const uint16_t*>(y), static_cast<const uint16_t*>(topk_gate), row_of_entry,
        valid_mask, n_tokens, top_k, hidden, static_cast<uint16_t*>(out));
  else
    combine_kernel<MEP_DTYPE_F32, INDEXED><<<grid, kThreads, 0, s>>>(
        static_cast<const float*>(y), static_cast<const float*>(topk_gate), row_of_entry,
        valid_mask, n_tokens, top_k, hidden, static_cast<float*>(out));
  hipError_t e = hipGetLastError();
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MEP_OK;
}

}  // namespace
}  // namespace mep

using namespace mep;

extern "C" int mep_combine(const void* y_entries, const void* topk_gate, const int32_t* row_of_entry,
                           const uint8_t* valid_mask, int64_t n_tokens, int32_t top_k, int32_t hidden,
                           int32_t dtype, void* out, void* stream) {
  return combine_entry<false>("mep_combine", y_entries, topk_gate, row_of_entry, valid_mask, n_tokens, top_k,
                              hidden, dtype, out, stream);
}

extern "C" int mep_combine_rows(const void* y_rows, const void* topk_gate, const int32_t* row_of_entry,
                                const uint8_t* valid_mask, int64_t n_tokens, int32_t top_k, int32_t hidden,
                                int32_t dtype, void* out, void* stream) {
  return combine_entry<true>("mep_combine_rows", y_rows, topk_gate, row_of_entry, valid_mask, n_tokens, top_k,
                             hidden, dtype, out, stream);
}

extern "C" int mep_gather_rows(const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                               int64_t n_rows, int32_t hidden, int32_t dtype, const int64_t* topk_idx,
                               int64_t* ids_out, void* out, void* stream) {
  clear_error();
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "mep_gather_rows: unknown dtype %d", dtype);
  MEP_REQUIRE(n_tokens >= 0 && n_rows >= 0 && top_k >= 1 && n_rows <= n_tokens * top_k, MEP_ERR_INVALID_ARG,
              "mep_gather_rows: bad sizes");
  const int epc = 16 / dtype_bytes(dtype);
  MEP_REQUIRE(hidden > 0 && hidden % epc == 0, MEP_ERR_UNSUPPORTED,
              "mep_gather_rows: hidden %d is not a multiple of %d", hidden, epc);
  MEP_REQUIRE((ids_out == nullptr) == (topk_idx == nullptr), MEP_ERR_INVALID_ARG,
              "mep_gather_rows: topk_idx and ids_out go together");
  if (n_rows == 0) return MEP_OK;
  MEP_REQUIRE(x && perm && out, MEP_ERR_INVALID_ARG, "mep_gather_rows: null pointer");
  MEP_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
              MEP_ERR_INVALID_ARG, "mep_gather_rows: x / out must be 16-byte aligned");
  const int64_t chunks = n_rows * (hidden / epc);
  const dim3 grid(static_cast<unsigned>((chunks + kThreads - 1) / kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MEP_DTYPE_BF16)
    gather_rows_kernel<MEP_DTYPE_BF16><<<grid, kThreads, 0, s>>>(static_cast<const uint16_t*>(x), perm, n_rows,
                                                                top_k, hidden, topk_idx, ids_out,
                                                                static_cast<uint16_t*>(out));
  else
    gather_rows_kernel<MEP_DTYPE_F32><<<grid, kThreads, 0, s>>>(static_cast<const float*>(x), perm, n_rows,
                                                               top_k, hidden, topk_idx, ids_out,
                                                               static_cast<float*>(out));
  MEP_CHECK_LAUNCH("mep_gather_rows");
  return MEP_OK;
}
