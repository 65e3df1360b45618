// Shared helpers for the gfx950 MoE kernels: bf16 conversion, MFMA operand
// types, error reporting for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/miniep_amd.h"

namespace mep {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// 16-byte vector used for every 128-bit load / store (a native clang vector, so
// arrays of it stay in registers; HIP's struct-based uint4 does not always)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- bf16 ----
// bf16 is carried as its raw 16-bit pattern.  Conversion to float is exact;
// conversion from float rounds to nearest even (NaN -> quiet NaN), which is
// what torch's .to(torch.bfloat16) does.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  // v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)f, (__bf16)0.0f};
  return static_cast<uint16_t>(__builtin_bit_cast(uint32_t, v) & 0xffffu);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Element traits: storage type and conversions for the two supported dtypes.
template <int DT> struct Elem;
template <> struct Elem<MEP_DTYPE_F32> {
  typedef float T;
  static constexpr int kBytes = 4;
  __device__ static float load(const float* p) { return *p; }
  __device__ static float to_f32(float v) { return v; }
  __device__ static float from_f32(float v) { return v; }
};
template <> struct Elem<MEP_DTYPE_BF16> {
  typedef uint16_t T;
  static constexpr int kBytes = 2;
  __device__ static float to_f32(uint16_t v) { return bf16_to_f32(v); }
  __device__ static uint16_t from_f32(float v) { return f32_to_bf16(v); }
};

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ------------------------------------------------------------ host side ----
void set_error(const char* fmt, ...);
void clear_error();
// compute units of the current device (cached per device)
int device_cu_count();
// The router kernel with its histogram output (router.hip): per 64-token
// workgroup b, bc[b * E + e] = entries of expert e among its valid tokens;
// it also writes the dispatch workspace's header[0] = n_blocks, flags[b] = 0
// and the world-1 tables (table 0, n_rep 1, g2l identity) into tables[3E].
// top_k must be 8.
hipError_t launch_router_with_hist(const void* x, const void* w, int64_t n, int hidden, int E, int k, int dtype,
                                   int64_t* idx, void* gate, float* logits, int32_t* bc, uint32_t* header,
                                   uint32_t* flags, int32_t* tables, const uint8_t* valid, int n_blocks,
                                   hipStream_t stream);

// The fused router + dispatch (one launch) of the all-local backend for
// bf16, E = 32, top-8, hidden 1024 / 2048 / 4096: outputs as
// mep_route_dispatch.  `rows` holds n_blocks x E tagged histogram words and
// the workspace header's word 32 the epoch; both must be zero before the
// first call on a workspace.  Returns hipErrorNotSupported, with nothing
// enqueued, when the shape differs or when the n_blocks workgroups do not
// all fit on the device at once.
hipError_t launch_route_dispatch_fused(const void* x, const void* w, int64_t n, int hidden, int E, int k, int dtype,
                                       int64_t* idx, void* gate, float* logits, int32_t* counts, int32_t* offsets,
                                       int32_t* perm, int32_t* row_of_entry, int64_t* route_counts, uint64_t* rows,
                                       uint32_t* header, uint32_t* flags, const uint8_t* valid, int n_blocks,
                                       hipStream_t stream);
// dispatch status bit of the fused route + dispatch: a workgroup gave up
// waiting for another's histogram row
constexpr uint32_t kFlagBarrier = 8u;

// Header of a dispatch workspace: 128-byte lines, then the status flags.
// Word 0: the number of launched blocks; kEpochWord: the epoch of the
// one-launch exchange (its tags); kDoneWord: groups of workgroups of the
// current one-launch call that have finished; kGiveupWord: nonzero once one
// of them gave up waiting; line 4 + g: workgroups of group g that have
// finished.  All but the first two are zero between calls.  (Each counter
// has a line of its own: device-scope atomics on one line are performed one
// after another, and a few hundred workgroups counting on one word would
// queue for microseconds.)
constexpr int kEpochWord = 32, kDoneWord = 64, kGiveupWord = 96, kGroupDoneWord = 128;
constexpr int kMaxDoneGroups = 64;
constexpr int kWsHeaderBytes = 4 * kGroupDoneWord + kMaxDoneGroups * 128;

// row_of_entry value of an entry of a one-launch dispatch that gave up (a
// workgroup waited too long for another's counts): the call's placement is
// invalid, offsets[n_local] is -1 (the experts kernels then run no tile) and
// the combine writes NaN for the token.
constexpr int32_t kPoisonRow = -2;

// Test hook (mep_test_force_giveup): the bounded wait that launches force to
// give up, and its poll limit; site 0 is normal operation.
struct GiveupTest {
  int site;
  int polls;
};
GiveupTest giveup_test();

// End of a workgroup of a one-launch dispatch exchange, called by every lane
// of wave 0 after a barrier that follows all of the workgroup's stores.  Lane
// 0 records a give-up in the header, then counts the workgroup finished in
// its group's word (groups of at least 16 consecutive blocks, at most
// kMaxDoneGroups of them); the group's last workgroup returns that word to
// zero and counts the group finished.  The last workgroup of the call to
// finish (by then every other one has read the epoch and completed its
// stores) returns the count and the give-up word to zero and gets
// kExchangeLast, plus kExchangeGaveUp if any workgroup gave up; the others
// get 0.  Only the last workgroup may advance the epoch: a workgroup that was
// not resident with the others can start after the early ones have exited,
// and must still read this call's epoch.
constexpr int kExchangeLast = 1, kExchangeGaveUp = 2;
__device__ __forceinline__ int finish_exchange(uint32_t* header, bool gave_up, int n_blocks) {
  int r = 0;
  if ((threadIdx.x & 63) == 0) {
    if (gave_up) __hip_atomic_fetch_or(header + kGiveupWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the give-up is recorded before the count
    const int per = max(16, (n_blocks + kMaxDoneGroups - 1) / kMaxDoneGroups);
    const int g = static_cast<int>(blockIdx.x) / per, n_groups = (n_blocks + per - 1) / per;
    uint32_t* const gw = header + kGroupDoneWord + 32 * g;
    const uint32_t in_g = __hip_atomic_fetch_add(gw, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (in_g == static_cast<uint32_t>(min(per, n_blocks - g * per) - 1)) {
      __hip_atomic_store(gw, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t done =
          __hip_atomic_fetch_add(header + kDoneWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (done == static_cast<uint32_t>(n_groups - 1)) {
        const uint32_t gu = __hip_atomic_exchange(header + kGiveupWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(header + kDoneWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        r = kExchangeLast | (gu != 0u ? kExchangeGaveUp : 0);
      }
    }
  }
  return __shfl(r, 0, 64);
}

// The poison of a one-launch dispatch that gave up (the last workgroup's
// wave 0): every row_of_entry entry kPoisonRow, offsets[n_local] = -1, with
// device-scope stores (the values they replace were stored that way too).
__device__ __forceinline__ void poison_dispatch(int32_t* row_of_entry, int64_t n_entries, int32_t* offsets,
                                                int n_local) {
  const int lane = threadIdx.x & 63;
  for (int64_t f = lane; f < n_entries; f += 64)
    __hip_atomic_store(row_of_entry + f, kPoisonRow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane == 0) __hip_atomic_store(offsets + n_local, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

inline int dtype_bytes(int dtype) {
  return dtype == MEP_DTYPE_F32 ? 4 : (dtype == MEP_DTYPE_BF16 ? 2 : 0);
}

}  // namespace mep

// Report a failed precondition from a C-ABI entry point.
#define MEP_REQUIRE(cond, code, ...)          \
  do {                                        \
    if (!(cond)) {                            \
      ::mep::set_error(__VA_ARGS__);          \
      return (code);                          \
    }                                         \
  } while (0)

// Check the launch that was just enqueued.
#define MEP_CHECK_LAUNCH(what)                                                   \
  do {                                                                           \
    hipError_t _e = hipGetLastError();                                           \
    if (_e != hipSuccess) {                                                      \
      ::mep::set_error("%s: launch failed: %s", (what), hipGetErrorString(_e));  \
      return MEP_ERR_HIP;                                                        \
    }                                                                            \
  } while (0)
