// Grouped SwiGLU experts on the gfx950 matrix cores.
//
// Replaces run_experts (modeling.py:83-104) and the row gather in front of it
// (modeling.py:143):
//     for each local expert e:  h = X_e @ W_in[e].T ; gate, up = h.chunk(2)
//                               y = (silu(gate) * up) @ W_out[e].T ; out[idx] = y
// as two launches over the dispatched rows (grouped by expert, ragged):
//   GEMM-1  act[r, :] = silu(x[perm[r]/k] W_g^T) * (x[perm[r]/k] W_u^T)
//           A rows are gathered from x inside the tile load (no permuted copy
//           of x is ever written); every output tile holds matching gate and
//           up columns, so SwiGLU runs in registers in the epilogue.
//   GEMM-2  y_entries[perm[r], :] = act[r, :] W_out^T
//           rows are scattered straight to their (token, slot) cell.
//
// Tiling: BM x BN output tile per workgroup, K staged 128 bytes per row at a
// time (64 bf16 / 32 fp32) through double-buffered LDS with one barrier per
// K step; the next K step's global loads are in flight while the current one
// feeds the MFMAs.  LDS rows are 8 chunks of 16 B with the chunk index XOR-ed
// by (row & 7), which makes both the 16-byte stores and the MFMA fragment
// reads (16 rows x one chunk) bank-conflict free.
// MFMA: v_mfma_f32_16x16x32_bf16 (bf16) or 4 x v_mfma_f32_16x16x4_f32 per
// 16-byte chunk (fp32); accumulation is fp32 in both cases.
//
// Scheduling: the ragged tile list (expert, m-tile, n-tile) is derived on the
// device from `offsets`, so no host round trip is needed for the counts.  The
// grid is an upper bound; workgroup b runs logical tile
//   (b mod 8) * ceil(T/8) + b / 8
// so the 32 CUs of one XCD (workgroups are dealt to the 8 XCDs round-robin)
// sweep one contiguous run of tiles and share its weights and rows in their L2.
#include "common.h"

namespace mep {
namespace {

constexpr int kRowBytes = 128;   // K bytes per row per LDS stage
constexpr int kChunks = 8;       // 16-byte chunks per LDS row

template <int BM_, int BN_, int WM_, int WN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int BMW = BM / WM, BNW = BN / WN;
  static constexpr int MF = BMW / 16, NF = BNW / 16;
  static constexpr int APT = BM * kChunks / NT;   // A chunks loaded per thread per stage
  static constexpr int BPT = BN * kChunks / NT;   // B chunks loaded per thread per stage
  static constexpr int STAGE_BYTES = (BM + BN) * kRowBytes;
  static_assert(BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "tile / wave shape");
  static_assert(NF % 2 == 0, "gate and up halves need an even number of 16-col fragments");
  static_assert((BM * kChunks) % NT == 0 && (BN * kChunks) % NT == 0, "load split");
};

struct GemmParams {
  const void* A;             // GEMM-1: x (n_tokens, K);  GEMM-2: act (max_rows, K)
  const int32_t* perm;       // row -> flat entry id
  const int32_t* offsets;    // (n_local + 1) row offsets per local expert
  const void* W;             // GEMM-1: w_in (n_local, 2N, K); GEMM-2: w_out (n_local, N, K)
  void* C;                   // GEMM-1: act (max_rows, N); GEMM-2: y_entries (N*k, N)
  int64_t w_expert_stride;   // elements per expert in W
  int n_local, top_k;
  int K;                     // reduction length
  int N;                     // output columns (GEMM-1: I; GEMM-2: H)
  int n_tiles_n;             // column tiles per row tile
};

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

template <int DT, class Cfg, bool GEMM1>
__global__ __launch_bounds__(Cfg::NT) void grouped_gemm_kernel(GemmParams p) {
  typedef typename Elem<DT>::T T;
  constexpr int EB = Elem<DT>::kBytes;
  constexpr int EPC = 16 / EB;                     // elements per 16-byte chunk
  constexpr int BKE = kRowBytes / EB;              // K elements per stage
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
  constexpr int MF = Cfg::MF, NF = Cfg::NF;
  constexpr int CN = GEMM1 ? BN / 2 : BN;          // output columns per tile
  constexpr int C_LD = CN * EB + 16;               // staging row stride (bytes)
  constexpr int SMEM = (2 * Cfg::STAGE_BYTES > BM * C_LD) ? 2 * Cfg::STAGE_BYTES : BM * C_LD;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  __shared__ int s_prefix[257];
  __shared__ int s_tile[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;

  // ---- tile schedule from the device-side offsets --------------------------
  const int nl = p.n_local;
  for (int j = tid; j < nl; j += NT) {
    const int rows = p.offsets[j + 1] - p.offsets[j];
    s_prefix[j + 1] = ((rows + BM - 1) / BM) * p.n_tiles_n;
  }
  if (tid == 0) s_prefix[0] = 0;
  __syncthreads();
  if (tid == 0) {
    for (int j = 0; j < nl; ++j) s_prefix[j + 1] += s_prefix[j];
  }
  __syncthreads();
  const int total = s_prefix[nl];
  const int per_xcd = (total + 7) / 8;
  const int slot = blockIdx.x / 8;
  if (slot >= per_xcd) return;
  const int lt = (blockIdx.x % 8) * per_xcd + slot;
  if (lt >= total) return;
  if (tid == 0) s_tile[0] = -1;
  __syncthreads();
  for (int j = tid; j < nl; j += NT) {
    if (lt >= s_prefix[j] && lt < s_prefix[j + 1]) {
      const int u = lt - s_prefix[j];
      s_tile[0] = j;
      s_tile[1] = p.offsets[j] + (u / p.n_tiles_n) * BM;
      s_tile[2] = p.offsets[j + 1];
      s_tile[3] = u % p.n_tiles_n;
    }
  }
  __syncthreads();
  const int e = s_tile[0];
  if (e < 0) return;
  const int row0 = s_tile[1], row_end = s_tile[2], nt = s_tile[3];
  const int K = p.K;

  // ---- global source pointers of the chunks this thread stages -------------
  const T* a_src[Cfg::APT];
  const T* b_src[Cfg::BPT];
  const int ch = tid % kChunks;
#pragma unroll
  for (int i = 0; i < Cfg::APT; ++i) {
    const int r = tid / kChunks + i * (NT / kChunks);
    const int row = (row0 + r < row_end) ? row0 + r : row0;   // tail rows: any valid row
    int64_t src;
    if constexpr (GEMM1) src = p.perm[row] / p.top_k;
    else src = row;
    a_src[i] = static_cast<const T*>(p.A) + src * K + ch * EPC;
  }
  const T* wexp = static_cast<const T*>(p.W) + static_cast<int64_t>(e) * p.w_expert_stride;
#pragma unroll
  for (int i = 0; i < Cfg::BPT; ++i) {
    const int r = tid / kChunks + i * (NT / kChunks);
    int wrow;
    if constexpr (GEMM1) wrow = (r < BN / 2) ? nt * (BN / 2) + r : p.N + nt * (BN / 2) + (r - BN / 2);
    else wrow = nt * BN + r;
    b_src[i] = wexp + static_cast<int64_t>(wrow) * K + ch * EPC;
  }

  u32x4 ra[Cfg::APT], rb[Cfg::BPT];
  auto load_global = [&](int kt) {
    const int koff = kt * BKE;
#pragma unroll
    for (int i = 0; i < Cfg::APT; ++i) ra[i] = *reinterpret_cast<const u32x4*>(a_src[i] + koff);
#pragma unroll
    for (int i = 0; i < Cfg::BPT; ++i) rb[i] = *reinterpret_cast<const u32x4*>(b_src[i] + koff);
  };
  auto store_lds = [&](int st) {
    unsigned char* As = smem + st * Cfg::STAGE_BYTES;
    unsigned char* Bs = As + BM * kRowBytes;
#pragma unroll
    for (int i = 0; i < Cfg::APT; ++i) {
      const int r = tid / kChunks + i * (NT / kChunks);
      *reinterpret_cast<u32x4*>(As + r * kRowBytes + ((ch ^ (r & 7)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < Cfg::BPT; ++i) {
      const int r = tid / kChunks + i * (NT / kChunks);
      *reinterpret_cast<u32x4*>(Bs + r * kRowBytes + ((ch ^ (r & 7)) << 4)) = rb[i];
    }
  };

  f32x4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fragment rows (within the LDS tile) this lane reads
  const int lr = lane & 15, lg = lane >> 4;
  int a_row[MF], b_row[NF];
#pragma unroll
  for (int i = 0; i < MF; ++i) a_row[i] = wm * Cfg::BMW + i * 16 + lr;
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    if constexpr (GEMM1)
      b_row[j] = (j < NF / 2) ? wn * (Cfg::BNW / 2) + j * 16 + lr
                              : BN / 2 + wn * (Cfg::BNW / 2) + (j - NF / 2) * 16 + lr;
    else
      b_row[j] = wn * Cfg::BNW + j * 16 + lr;
  }

  auto compute = [&](int st) {
    const unsigned char* As = smem + st * Cfg::STAGE_BYTES;
    const unsigned char* Bs = As + BM * kRowBytes;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = kk * 4 + lg;
      u32x4 af[MF], bfr[NF];
#pragma unroll
      for (int i = 0; i < MF; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(As + a_row[i] * kRowBytes + ((c ^ (a_row[i] & 7)) << 4));
#pragma unroll
      for (int j = 0; j < NF; ++j)
        bfr[j] = *reinterpret_cast<const u32x4*>(Bs + b_row[j] * kRowBytes + ((c ^ (b_row[j] & 7)) << 4));
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          if constexpr (DT == MEP_DTYPE_BF16) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, af[i]), __builtin_bit_cast(bf16x8, bfr[j]), acc[i][j], 0, 0, 0);
          } else {
            const float* a4 = reinterpret_cast<const float*>(&af[i]);
            const float* b4 = reinterpret_cast<const float*>(&bfr[j]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[q], b4[q], acc[i][j], 0, 0, 0);
          }
        }
    }
  };

  // ---- main loop -------------------------------------------------------------
  const int KT = K / BKE;
  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < KT - 1; ++kt) {
    load_global(kt + 1);
    compute(kt & 1);
    store_lds((kt + 1) & 1);
    __syncthreads();
  }
  compute((KT - 1) & 1);
  __syncthreads();

  // ---- epilogue: registers -> LDS tile -> 16-byte row stores -----------------
  // 16x16 MFMA C layout: lane holds rows 4*(lane/16) + i, column lane % 16.
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < (GEMM1 ? NF / 2 : NF); ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = wm * Cfg::BMW + i * 16 + lg * 4 + q;
        int c;
        float v;
        if constexpr (GEMM1) {
          c = wn * (Cfg::BNW / 2) + j * 16 + lr;
          v = silu_f(acc[i][j][q]) * acc[i][j + NF / 2][q];
        } else {
          c = wn * Cfg::BNW + j * 16 + lr;
          v = acc[i][j][q];
        }
        *reinterpret_cast<T*>(smem + r * C_LD + c * EB) = Elem<DT>::from_f32(v);
      }
  __syncthreads();
  constexpr int CPR = CN * EB / 16;   // 16-byte chunks per output row
  T* C = static_cast<T*>(p.C);
  for (int q = tid; q < BM * CPR; q += NT) {
    const int r = q / CPR, c = q - r * CPR;
    if (row0 + r >= row_end) continue;
    int64_t dst;
    if constexpr (GEMM1) dst = static_cast<int64_t>(row0 + r) * p.N + nt * CN + c * EPC;
    else dst = static_cast<int64_t>(p.perm[row0 + r]) * p.N + nt * CN + c * EPC;
    *reinterpret_cast<u32x4*>(C + dst) = *reinterpret_cast<const u32x4*>(smem + r * C_LD + c * 16);
  }
}

template <int DT, class Cfg, bool GEMM1>
hipError_t launch(const GemmParams& p, int64_t max_rows, hipStream_t stream) {
  int64_t tiles = ((max_rows + Cfg::BM - 1) / Cfg::BM + p.n_local) * p.n_tiles_n;
  tiles = (tiles + 7) / 8 * 8;
  if (tiles == 0) return hipSuccess;
  grouped_gemm_kernel<DT, Cfg, GEMM1><<<dim3(static_cast<unsigned>(tiles)), Cfg::NT, 0, stream>>>(p);
  return hipGetLastError();
}

// Tile shapes: bf16 256x256 (GEMM-1: 128 gate + 128 up columns) on 8 waves
// (4 x 2, 64 x 128 per wave, 2 waves per SIMD, no spills);
// fp32 64x128 on 4 waves.
typedef TileCfg<256, 256, 4, 2> CfgBf16;
typedef TileCfg<64, 128, 2, 2> CfgF32;

template <int DT, class Cfg>
int run_gate_up(const void* x, int top_k, const int32_t* perm, const int32_t* offsets, int n_local,
                int64_t max_rows, const void* w_in, int hidden, int inter, void* act,
                hipStream_t stream) {
  GemmParams g1;
  g1.A = x; g1.perm = perm; g1.offsets = offsets; g1.W = w_in; g1.C = act;
  g1.w_expert_stride = static_cast<int64_t>(2) * inter * hidden;
  g1.n_local = n_local; g1.top_k = top_k; g1.K = hidden; g1.N = inter;
  g1.n_tiles_n = inter / (Cfg::BN / 2);
  hipError_t e = launch<DT, Cfg, true>(g1, max_rows, stream);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_swiglu_gate_up: %s", hipGetErrorString(e));
  return MEP_OK;
}

template <int DT, class Cfg>
int run_down(const void* act, int top_k, const int32_t* perm, const int32_t* offsets, int n_local,
             int64_t max_rows, const void* w_out, int hidden, int inter, void* y, hipStream_t stream) {
  GemmParams g2;
  g2.A = act; g2.perm = perm; g2.offsets = offsets; g2.W = w_out; g2.C = y;
  g2.w_expert_stride = static_cast<int64_t>(hidden) * inter;
  g2.n_local = n_local; g2.top_k = top_k; g2.K = inter; g2.N = hidden;
  g2.n_tiles_n = hidden / Cfg::BN;
  hipError_t e = launch<DT, Cfg, false>(g2, max_rows, stream);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_swiglu_down: %s", hipGetErrorString(e));
  return MEP_OK;
}

// Shared argument checks of the three expert entry points.
int check_expert_args(const char* fn, int64_t n_tokens, int top_k, int n_local, int64_t max_rows,
                      int hidden, int inter, int dtype) {
  MEP_REQUIRE(dtype == MEP_DTYPE_F32 || dtype == MEP_DTYPE_BF16, MEP_ERR_INVALID_ARG,
              "%s: unknown dtype %d", fn, dtype);
  MEP_REQUIRE(n_tokens >= 0 && top_k >= 1 && max_rows >= 0 && n_local >= 0, MEP_ERR_INVALID_ARG,
              "%s: negative size", fn);
  MEP_REQUIRE(n_local <= 256, MEP_ERR_UNSUPPORTED, "%s: n_local %d > 256", fn, n_local);
  MEP_REQUIRE(hidden > 0 && hidden % 256 == 0, MEP_ERR_UNSUPPORTED,
              "%s: hidden %d must be a positive multiple of 256", fn, hidden);
  MEP_REQUIRE(inter > 0 && inter % 128 == 0, MEP_ERR_UNSUPPORTED,
              "%s: inter %d must be a positive multiple of 128", fn, inter);
  MEP_REQUIRE(max_rows <= n_tokens * top_k, MEP_ERR_INVALID_ARG,
              "%s: max_rows %lld exceeds n_tokens * top_k", fn, (long long)max_rows);
  return MEP_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace mep

using namespace mep;


extern "C" int mep_swiglu_gate_up(const void* x, int64_t n_tokens, int32_t top_k,
                                  const int32_t* perm, const int32_t* offsets, int32_t n_local,
                                  int64_t max_rows, const void* w_in, int32_t hidden, int32_t inter,
                                  int32_t dtype, void* act, size_t act_bytes, void* stream) {
  clear_error();
  int rc = check_expert_args("mep_swiglu_gate_up", n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(x && perm && offsets && w_in && act, MEP_ERR_INVALID_ARG, "mep_swiglu_gate_up: null pointer");
  const size_t need = static_cast<size_t>(max_rows) * inter * dtype_bytes(dtype);
  MEP_REQUIRE(act_bytes >= need, MEP_ERR_WORKSPACE, "mep_swiglu_gate_up: act %zu B < required %zu B",
              act_bytes, need);
  MEP_REQUIRE(aligned16(x) && aligned16(w_in) && aligned16(act), MEP_ERR_INVALID_ARG,
              "mep_swiglu_gate_up: buffers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MEP_DTYPE_BF16)
    return run_gate_up<MEP_DTYPE_BF16, CfgBf16>(x, top_k, perm, offsets, n_local, max_rows, w_in, hidden,
                                                inter, act, s);
  return run_gate_up<MEP_DTYPE_F32, CfgF32>(x, top_k, perm, offsets, n_local, max_rows, w_in, hidden,
                                            inter, act, s);
}

extern "C" int mep_swiglu_down(const void* act, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                               const int32_t* offsets, int32_t n_local, int64_t max_rows,
                               const void* w_out, int32_t hidden, int32_t inter, int32_t dtype,
                               void* y_entries, void* stream) {
  clear_error();
  int rc = check_expert_args("mep_swiglu_down", n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(act && perm && offsets && w_out && y_entries, MEP_ERR_INVALID_ARG,
              "mep_swiglu_down: null pointer");
  MEP_REQUIRE(aligned16(act) && aligned16(w_out) && aligned16(y_entries), MEP_ERR_INVALID_ARG,
              "mep_swiglu_down: buffers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MEP_DTYPE_BF16)
    return run_down<MEP_DTYPE_BF16, CfgBf16>(act, top_k, perm, offsets, n_local, max_rows, w_out, hidden,
                                             inter, y_entries, s);
  return run_down<MEP_DTYPE_F32, CfgF32>(act, top_k, perm, offsets, n_local, max_rows, w_out, hidden, inter,
                                         y_entries, s);
}

extern "C" size_t mep_experts_workspace_size(int64_t max_rows, int32_t inter, int32_t dtype) {
  const int eb = dtype_bytes(dtype);
  if (max_rows < 0 || inter <= 0 || eb == 0) return 0;
  return static_cast<size_t>(max_rows) * inter * eb + 256;
}

extern "C" int mep_grouped_swiglu(const void* x, int64_t n_tokens, int32_t top_k,
                                  const int32_t* perm, const int32_t* offsets, int32_t n_local,
                                  int64_t max_rows, const void* w_in, const void* w_out,
                                  int32_t hidden, int32_t inter, int32_t dtype, void* y_entries,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_expert_args("mep_grouped_swiglu", n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(workspace != nullptr, MEP_ERR_INVALID_ARG, "mep_grouped_swiglu: null workspace");
  const size_t need = mep_experts_workspace_size(max_rows, inter, dtype);
  MEP_REQUIRE(workspace_bytes >= need, MEP_ERR_WORKSPACE,
              "mep_grouped_swiglu: workspace %zu B < required %zu B", workspace_bytes, need);
  rc = mep_swiglu_gate_up(x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, hidden, inter, dtype,
                          workspace, workspace_bytes, stream);
  if (rc != MEP_OK) return rc;
  return mep_swiglu_down(workspace, n_tokens, top_k, perm, offsets, n_local, max_rows, w_out, hidden, inter,
                         dtype, y_entries, stream);
}
