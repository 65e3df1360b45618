// Device code of the slot-order combine for top-8, shared by combine8_kernel
// (combine.hip) and the small-batch experts launch that ends with the combine
// (grouped_swiglu.hip), so both sum in exactly the same order.
//
// One thread owns 16-byte chunk c of token t's output row: out[t, chunk] =
// sum over slots s = 0..7 of gate[t, s] * y[t*8 + s, chunk] in fp32, in slot
// order, over the present cells (row_of_entry[t*8 + s] >= 0) of valid tokens
// (modeling.py:120-128, :144).  `load_y` reads one 16-byte chunk of y (the
// caller picks the cache policy); the 8 cells, their row_of_entry entries,
// the gates and the valid flag are independent loads issued together, and an
// absent cell is skipped with a select, so whatever it holds never reaches
// the sum.  A token with a poisoned entry (kPoisonRow: its dispatch gave up)
// gets NaN.
#pragma once

#include "common.h"

namespace mep {

template <int DT>
__device__ __forceinline__ u32x4 pack_row_chunk(const float* acc) {
  u32x4 o;
  if constexpr (DT == MEP_DTYPE_BF16) {
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
  } else {
    o.x = __float_as_uint(acc[0]);
    o.y = __float_as_uint(acc[1]);
    o.z = __float_as_uint(acc[2]);
    o.w = __float_as_uint(acc[3]);
  }
  return o;
}

// DEV: the token's row_of_entry entries and gates are read with device-scope
// loads (written earlier in the same launch, possibly on another XCD), and so
// is `poison` if given: nonzero there makes the chunk NaN, as a poisoned
// entry does (one more load issued with the others, not a round trip before).
template <int DT, class LoadY, bool DEV = false>
__device__ __forceinline__ void combine8_chunk(const typename Elem<DT>::T* __restrict__ y,
                                               const typename Elem<DT>::T* __restrict__ gate,
                                               const int32_t* __restrict__ row_of_entry,
                                               const uint8_t* __restrict__ valid, int64_t t, int c, int hidden,
                                               typename Elem<DT>::T* __restrict__ out, LoadY load_y,
                                               const int32_t* poison_word = nullptr) {
  typedef typename Elem<DT>::T T;
  constexpr int K = 8;
  constexpr int EPC = 16 / Elem<DT>::kBytes;
  const T* ybase = y + (t * K) * hidden + c * EPC;
  u32x4 v[K];
#pragma unroll
  for (int s = 0; s < K; ++s) v[s] = load_y(ybase + static_cast<int64_t>(s) * hidden);
  int32_t row[K];
  float g[K];
  int32_t pw = 0;
  if constexpr (DEV) {
    if (poison_word != nullptr) pw = __hip_atomic_load(poison_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    static_assert(DT == MEP_DTYPE_BF16, "device-scope reads of bf16 gates");
    const uint64_t* rp = reinterpret_cast<const uint64_t*>(row_of_entry + t * K);
    const uint64_t* gp = reinterpret_cast<const uint64_t*>(gate + t * K);
#pragma unroll
    for (int h = 0; h < K / 2; ++h) {
      const uint64_t v = __hip_atomic_load(rp + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      row[2 * h] = static_cast<int32_t>(static_cast<uint32_t>(v));
      row[2 * h + 1] = static_cast<int32_t>(static_cast<uint32_t>(v >> 32));
    }
#pragma unroll
    for (int h = 0; h < K / 4; ++h) {
      const uint64_t v = __hip_atomic_load(gp + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int q = 0; q < 4; ++q) g[4 * h + q] = bf16_to_f32(static_cast<uint16_t>(v >> (16 * q)));
    }
  } else {
#pragma unroll
    for (int s = 0; s < K; ++s) {
      row[s] = row_of_entry[t * K + s];
      g[s] = Elem<DT>::to_f32(gate[t * K + s]);
    }
  }
  const bool tok_ok = valid == nullptr || valid[t] != 0;
  bool poison = pw != 0;
  float acc[EPC];
#pragma unroll
  for (int q = 0; q < EPC; ++q) acc[q] = 0.0f;
#pragma unroll
  for (int s = 0; s < K; ++s) {
    const bool here = tok_ok && row[s] >= 0;
    poison |= row[s] == kPoisonRow;
    float yv[EPC];
    if constexpr (DT == MEP_DTYPE_BF16) {
      const uint32_t w[4] = {v[s].x, v[s].y, v[s].z, v[s].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        yv[2 * q] = bf16_to_f32(static_cast<uint16_t>(w[q] & 0xffffu));
        yv[2 * q + 1] = bf16_to_f32(static_cast<uint16_t>(w[q] >> 16));
      }
    } else {
      yv[0] = __uint_as_float(v[s].x);
      yv[1] = __uint_as_float(v[s].y);
      yv[2] = __uint_as_float(v[s].z);
      yv[3] = __uint_as_float(v[s].w);
    }
#pragma unroll
    for (int q = 0; q < EPC; ++q) {
      const float sum = acc[q] + g[s] * yv[q];
      acc[q] = here ? sum : acc[q];
    }
  }
#pragma unroll
  for (int q = 0; q < EPC; ++q) acc[q] = poison ? __builtin_nanf("") : acc[q];
  *reinterpret_cast<u32x4*>(out + t * hidden + c * EPC) = pack_row_chunk<DT>(acc);
}

}  // namespace mep
