// Expert weight slots: copy whole experts between weight arrays.
//
// The reference re-slices a rank's experts on every rebalance: the new
// placement's owned + replica experts are read from the checkpoint in sorted
// id order and swapped in for every layer (server.py:51-62, weights.py:37-61).
// Here a rank keeps its experts in per-layer slots (w_in (n_slots, 2I, H),
// w_out (n_slots, H, I)), the grouped GEMM reads local expert j from slot
// w_slot[j] (mep_grouped_swiglu_slots), and a rebalance copies only the
// experts that become resident into free slots: one launch moves any number
// of (source expert -> slot) pairs.  Pure streaming copy, 16-byte vectors,
// bound by HBM bandwidth (or by the link, for a source in pinned host memory).
#include "common.h"

namespace mep {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPairs = 128;          // pairs per launch (kernel argument space)

struct CopyBatch {
  const unsigned char* src_in;
  const unsigned char* src_out;
  unsigned char* dst_in;
  unsigned char* dst_out;
  int64_t in_bytes, out_bytes;          // bytes of one expert in w_in / w_out (multiples of 16)
  int n;
  int32_t src[kMaxPairs];
  int32_t dst[kMaxPairs];
};

// Block (b, i) copies chunk range b of pair i: w_in bytes first, then w_out.
__global__ __launch_bounds__(kThreads) void copy_experts_kernel(CopyBatch c) {
  const int i = blockIdx.y;
  const int64_t total = (c.in_bytes + c.out_bytes) / 16;
  const int64_t in_chunks = c.in_bytes / 16;
  const u32x4* sin = reinterpret_cast<const u32x4*>(c.src_in + c.src[i] * c.in_bytes);
  const u32x4* sout = reinterpret_cast<const u32x4*>(c.src_out + c.src[i] * c.out_bytes);
  u32x4* din = reinterpret_cast<u32x4*>(c.dst_in + c.dst[i] * c.in_bytes);
  u32x4* dout = reinterpret_cast<u32x4*>(c.dst_out + c.dst[i] * c.out_bytes);
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * kThreads) {
    if (q < in_chunks) din[q] = sin[q];
    else dout[q - in_chunks] = sout[q - in_chunks];
  }
}

}  // namespace
}  // namespace mep

using namespace mep;

extern "C" int mep_copy_experts(const void* src_in, const void* src_out, int32_t n_src, void* dst_in,
                                void* dst_out, int32_t n_slots, const int32_t* src_index,
                                const int32_t* dst_slot, int32_t n, int32_t hidden, int32_t inter,
                                int32_t dtype, void* stream) {
  clear_error();
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "mep_copy_experts: unknown dtype %d", dtype);
  MEP_REQUIRE(n >= 0 && n_src >= 0 && n_slots >= 0 && hidden > 0 && inter > 0, MEP_ERR_INVALID_ARG,
              "mep_copy_experts: bad sizes");
  if (n == 0) return MEP_OK;
  MEP_REQUIRE(src_in && src_out && dst_in && dst_out && src_index && dst_slot, MEP_ERR_INVALID_ARG,
              "mep_copy_experts: null pointer");
  const int64_t eb = dtype_bytes(dtype);
  const int64_t in_bytes = int64_t(2) * inter * hidden * eb, out_bytes = int64_t(hidden) * inter * eb;
  MEP_REQUIRE(in_bytes % 16 == 0 && out_bytes % 16 == 0, MEP_ERR_UNSUPPORTED,
              "mep_copy_experts: expert matrices must be multiples of 16 bytes");
  MEP_REQUIRE(((reinterpret_cast<uintptr_t>(src_in) | reinterpret_cast<uintptr_t>(src_out) |
                reinterpret_cast<uintptr_t>(dst_in) | reinterpret_cast<uintptr_t>(dst_out)) % 16) == 0,
              MEP_ERR_INVALID_ARG, "mep_copy_experts: buffers must be 16-byte aligned");
  // every index is checked here, on the host, before anything is enqueued;
  // a slot written twice in one call would make the result depend on timing
  for (int i = 0; i < n; ++i) {
    MEP_REQUIRE(src_index[i] >= 0 && src_index[i] < n_src, MEP_ERR_INVALID_ARG,
                "mep_copy_experts: source expert %d outside [0, %d)", src_index[i], n_src);
    MEP_REQUIRE(dst_slot[i] >= 0 && dst_slot[i] < n_slots, MEP_ERR_INVALID_ARG,
                "mep_copy_experts: slot %d outside [0, %d)", dst_slot[i], n_slots);
    for (int j = 0; j < i; ++j)
      MEP_REQUIRE(dst_slot[j] != dst_slot[i], MEP_ERR_INVALID_ARG, "mep_copy_experts: slot %d written twice",
                  dst_slot[i]);
  }
  CopyBatch c;
  c.src_in = static_cast<const unsigned char*>(src_in);
  c.src_out = static_cast<const unsigned char*>(src_out);
  c.dst_in = static_cast<unsigned char*>(dst_in);
  c.dst_out = static_cast<unsigned char*>(dst_out);
  c.in_bytes = in_bytes;
  c.out_bytes = out_bytes;
  // 64 KiB per block (16 chunks per thread): 48 blocks per GraniteMoE expert,
  // so even a one-expert copy spreads over many CUs
  const int64_t chunks = (in_bytes + out_bytes) / 16;
  const unsigned bx = static_cast<unsigned>((chunks + kThreads * 16 - 1) / (kThreads * 16));
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i0 = 0; i0 < n; i0 += kMaxPairs) {
    c.n = n - i0 < kMaxPairs ? n - i0 : kMaxPairs;
    for (int i = 0; i < c.n; ++i) {
      c.src[i] = src_index[i0 + i];
      c.dst[i] = dst_slot[i0 + i];
    }
    copy_experts_kernel<<<dim3(bx, static_cast<unsigned>(c.n)), kThreads, 0, s>>>(c);
    MEP_CHECK_LAUNCH("mep_copy_experts");
  }
  return MEP_OK;
}
