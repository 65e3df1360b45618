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
// Tiling: BM x BN output tile, 8 waves (4 x 2) of 64 x 128.  K is staged 128
// bytes per row at a time (64 bf16 / 32 fp32) through two LDS stages filled by
// global_load_lds_dwordx4 (global memory straight into LDS, no VGPR staging):
// one instruction moves 8 rows x 128 B; lane L lands at byte 16 L, so it
// fetches logical chunk (L%8) ^ (L/8) of its row, which stores each row's
// chunks XOR-swizzled by (row & 7) and makes the fragment reads (16 rows x one
// chunk) bank-conflict free.  The MFMA takes the weight fragment as its first
// operand, so it produces C^T: each lane holds 4 consecutive output columns of
// one row, and the epilogue packs them into 8-byte LDS writes.
// MFMA: v_mfma_f32_16x16x32_bf16 (bf16) or 4 x v_mfma_f32_16x16x4_f32 per
// 16-byte chunk (fp32); accumulation is fp32 in both cases.
//
// Scheduling: persistent.  One workgroup per CU walks a list of tiles
// (expert, m-tile, n-tile) derived on the device from `offsets` (no host round
// trip for the counts).  Workgroups are dealt to the 8 XCDs round-robin, so
// workgroup b takes tiles (b mod 8) * ceil(T/8) + b/8 + i * (grid/8): the CUs
// of one XCD sweep one contiguous run of tiles and share weights and rows in
// their L2.  While a tile's epilogue drains through one LDS stage, the next
// tile's first K step is already streaming into the other.
#include "common.h"

namespace mep {
namespace {

constexpr int kRowBytes = 128;   // K bytes per row per LDS stage
// s_waitcnt immediate for "vmcnt(0)" alone (gfx9 encoding: expcnt and lgkmcnt at max)
constexpr int kVmcnt0 = 0x0F70;

template <int BM_, int BN_, int WM_, int WN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int NWAVES = WM * WN;
  static constexpr int BMW = BM / WM, BNW = BN / WN;
  static constexpr int MF = BMW / 16, NF = BNW / 16;
  static constexpr int STAGE_BYTES = (BM + BN) * kRowBytes;
  static constexpr int NBLK = (BM + BN) / 8;      // 1 KiB DMA blocks per stage
  static constexpr int BPW = NBLK / NWAVES;       // blocks per wave per stage
  static_assert(BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "tile / wave shape");
  static_assert(NF % 2 == 0, "gate and up halves need an even number of 16-col fragments");
  static_assert(NBLK % NWAVES == 0 && (BM / 8) % BPW == 0, "a wave's blocks are all A or all B rows");
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

// silu(v) = v / (1 + e^-v) with the hardware exp2 and reciprocal (about 1 ulp
// each); saturates correctly: v -> -inf gives -0, v -> +inf gives v.
__device__ __forceinline__ float silu_f(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * 1.4426950408889634f));
}

constexpr int pow2_floor(int v) { int r = 1; while (r * 2 <= v) r *= 2; return r; }

// Workgroup barrier that orders LDS only: this wave's LDS reads and writes
// complete (lgkmcnt(0)) before it arrives.  __syncthreads() also waits for
// every outstanding global access (vmcnt(0)); in the epilogue that would wait
// for the previous pass's stores and the next tile's first DMA stage.  The
// empty asm statements keep the compiler from moving memory accesses across.
constexpr int kLgkmcnt0 = 0xC07F;   // s_waitcnt lgkmcnt(0) alone (vmcnt 63, expcnt 7)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int DT, class Cfg, bool GEMM1>
__global__ __launch_bounds__(Cfg::NT) void grouped_gemm_kernel(GemmParams p) {
  typedef typename Elem<DT>::T T;
  constexpr int EB = Elem<DT>::kBytes;
  constexpr int EPC = 16 / EB;                     // elements per 16-byte chunk
  constexpr int BKE = kRowBytes / EB;              // K elements per stage
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
  constexpr int MF = Cfg::MF, NF = Cfg::NF, BPW = Cfg::BPW;
  constexpr int STAGE = Cfg::STAGE_BYTES;
  constexpr int CN = GEMM1 ? BN / 2 : BN;          // output columns per tile
  // epilogue staging through one stage: PASS_COLS columns of all BM rows at a time
  constexpr int PASS_COLS = pow2_floor(STAGE / (BM * EB)) < CN ? pow2_floor(STAGE / (BM * EB)) : CN;
  constexpr int NPASS = CN / PASS_COLS;
  constexpr int SROW = PASS_COLS * EB;             // staging row bytes
  constexpr int SCPR = SROW / 16;                  // 16-byte chunks per staging row
  static_assert(CN % PASS_COLS == 0 && SCPR >= 1 && (SCPR & (SCPR - 1)) == 0, "staging geometry");
  static_assert(PASS_COLS % 16 == 0, "a 16-column fragment never straddles two passes");

  // One LDS object only: with a second __shared__ variable the compiler tags
  // LDS accesses with alias scopes and then makes every fragment read wait for
  // the in-flight DMA into the other stage (vmcnt(0)), which serialises the
  // pipeline.  The schedule tables therefore live at the end of `smem`.
  constexpr int NLMAX = 256;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * STAGE + (2 * NLMAX + 2 + 2 * BM) * 4];
  int* const s_prefix = reinterpret_cast<int*>(smem + 2 * STAGE);   // [NLMAX + 1] tiles before expert j
  int* const s_off = s_prefix + NLMAX + 1;                          // [NLMAX + 1] row offsets
  int* const s_rows = s_off + NLMAX + 1;                            // [2][BM] perm of a tile's rows

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int K = p.K;
  const int nl = p.n_local;

  // ---- tile table: tiles per expert, prefix over experts ---------------------
  for (int j = tid; j <= nl; j += NT) s_off[j] = p.offsets[j];
  __syncthreads();
  for (int j = tid; j < nl; j += NT)
    s_prefix[j + 1] = ((s_off[j + 1] - s_off[j] + BM - 1) / BM) * p.n_tiles_n;
  if (tid == 0) s_prefix[0] = 0;
  __syncthreads();
  if (tid == 0)
    for (int j = 0; j < nl; ++j) s_prefix[j + 1] += s_prefix[j];
  __syncthreads();
  const int total = __builtin_amdgcn_readfirstlane(s_prefix[nl]);
  const int per_xcd = (total + 7) / 8;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8, nslots = gridDim.x / 8;
  const int n_my = slot < per_xcd ? (per_xcd - slot + nslots - 1) / nslots : 0;
  // tiles of this workgroup: xcd * per_xcd + slot + i * nslots, i < n_my, below total
  auto tile_id = [&](int i) { return xcd * per_xcd + slot + i * nslots; };
  auto tile_valid = [&](int i) { return i < n_my && tile_id(i) < total; };
  if (!tile_valid(0)) return;

  struct Tile { int e, row0, row_end, nt; };
  auto decode = [&](int lt) {
    int lo = 0, hi = nl - 1;                       // largest j with s_prefix[j] <= lt
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_prefix[mid] <= lt) lo = mid; else hi = mid - 1;
    }
    const int u = lt - s_prefix[lo];
    Tile t;                                        // uniform: keep it in SGPRs
    t.e = __builtin_amdgcn_readfirstlane(lo);
    t.row0 = __builtin_amdgcn_readfirstlane(s_off[lo] + (u / p.n_tiles_n) * BM);
    t.row_end = __builtin_amdgcn_readfirstlane(s_off[lo + 1]);
    t.nt = __builtin_amdgcn_readfirstlane(u % p.n_tiles_n);
    return t;
  };

  // ---- row maps: perm[row0 .. row0 + BM) of a tile DMA'd into LDS a tile
  // ahead (clamped to the tile's last row, so every lane reads inside perm);
  // GEMM-1 gathers its A rows through it, GEMM-2 scatters its output rows.
  static_assert(BM % 64 == 0 && BM / 64 <= Cfg::NWAVES, "row-map DMA: one 64-row instruction per wave");
  auto rowmap_dma = [&](const Tile& t, int parity) {
    if (wave < BM / 64) {
      const int r = min(t.row0 + wave * 64 + lane, t.row_end - 1);
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(p.perm + r),
                                       (__attribute__((address_space(3))) void*)(s_rows + parity * BM + wave * 64),
                                       4, 0, 0);
    }
  };

  // ---- direct global -> LDS staging -------------------------------------------
  // Wave w moves stage blocks w*BPW .. w*BPW+BPW-1 (block q = stage rows 8q..8q+7;
  // A rows [0, BM), B rows [BM, BM + BN)).  Each lane keeps one 32-bit byte
  // offset per block from a wave-uniform base (x / act, or the expert's W).
  const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
  const bool wave_loads_a = (wave * BPW) * 8 < BM;
  uint32_t src_off[BPW];
  const unsigned char* g_base;
  auto setup = [&](const Tile& t, int parity) {
    // recompute the per-lane row terms here instead of keeping them live across
    // the whole tile loop (hoisted, they outgrow the register budget and spill)
    int lrow_v = lrow, lchunk_v = lchunk;
    asm volatile("" : "+v"(lrow_v), "+v"(lchunk_v));
    if (wave_loads_a) {
      g_base = static_cast<const unsigned char*>(p.A);
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int r = (wave * BPW + i) * 8 + lrow_v;
        int64_t src_row;
        if constexpr (GEMM1) src_row = s_rows[parity * BM + r] / p.top_k;       // gather (row map clamped)
        else src_row = min(t.row0 + r, t.row_end - 1);                         // tail rows: any valid row
        src_off[i] = static_cast<uint32_t>((src_row * K + lchunk_v * EPC) * EB);
      }
    } else {
      g_base = static_cast<const unsigned char*>(p.W) + static_cast<int64_t>(t.e) * p.w_expert_stride * EB;
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int rb = (wave * BPW + i) * 8 + lrow_v - BM;
        int wrow;
        if constexpr (GEMM1) wrow = (rb < BN / 2) ? t.nt * (BN / 2) + rb : p.N + t.nt * (BN / 2) + (rb - BN / 2);
        else wrow = t.nt * BN + rb;
        src_off[i] = static_cast<uint32_t>((static_cast<int64_t>(wrow) * K + lchunk_v * EPC) * EB);
      }
    }
  };
  auto load_stage = [&](int kt, unsigned char* stage) {
    const uint32_t koff = static_cast<uint32_t>(kt * kRowBytes);
#pragma unroll
    for (int i = 0; i < BPW; ++i)
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(g_base + src_off[i] + koff),
                                       (__attribute__((address_space(3))) void*)(stage + (wave * BPW + i) * 1024),
                                       16, 0, 0);
  };

  // ---- fragments and MFMAs ------------------------------------------------------
  // Lane (lr, lg) reads 16 B of row base + 16 i + lr at physical chunk
  // (4 kk + lg) ^ (lr & 7): one per-lane base per fragment set plus immediates.
  const int lr = lane & 15, lg = lane >> 4;
  uint32_t cp[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) cp[kk] = static_cast<uint32_t>(((kk * 4 + lg) ^ (lr & 7)) << 4);
  const uint32_t a_lane = static_cast<uint32_t>((wm * Cfg::BMW + lr) * kRowBytes);
  uint32_t b_lane_lo, b_lane_hi;   // GEMM-1: gate / up halves; GEMM-2: one contiguous range
  if constexpr (GEMM1) {
    b_lane_lo = static_cast<uint32_t>((BM + wn * (Cfg::BNW / 2) + lr) * kRowBytes);
    b_lane_hi = static_cast<uint32_t>((BM + BN / 2 + wn * (Cfg::BNW / 2) + lr) * kRowBytes);
  } else {
    b_lane_lo = static_cast<uint32_t>((BM + wn * Cfg::BNW + lr) * kRowBytes);
    b_lane_hi = b_lane_lo + (NF / 2) * 16 * kRowBytes;
  }
  f32x4 acc[MF][NF];
  auto compute = [&](const unsigned char* S) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 af[MF], bfr[NF];
#pragma unroll
      for (int i = 0; i < MF; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(S + a_lane + cp[kk] + i * 16 * kRowBytes);
#pragma unroll
      for (int j = 0; j < NF; ++j) {
        const uint32_t b = (j < NF / 2 ? b_lane_lo + j * 16 * kRowBytes : b_lane_hi + (j - NF / 2) * 16 * kRowBytes);
        bfr[j] = *reinterpret_cast<const u32x4*>(S + b + cp[kk]);
      }
      // weight fragment first: the MFMA yields C^T (lane: one row, 4 columns)
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          if constexpr (DT == MEP_DTYPE_BF16) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, bfr[j]), __builtin_bit_cast(bf16x8, af[i]), acc[i][j], 0, 0, 0);
          } else {
            const float* a4 = reinterpret_cast<const float*>(&af[i]);
            const float* b4 = reinterpret_cast<const float*>(&bfr[j]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b4[q], a4[q], acc[i][j], 0, 0, 0);
          }
        }
    }
  };

  // ---- epilogue helpers -----------------------------------------------------------
  // Lane holds, for fragment (i, j), row wm*BMW + 16 i + lr and the 4 columns
  // 16 j + 4 lg + q of its wave's column range.  Staging row r of a pass is
  // SROW bytes with 16-byte chunks XOR-swizzled by (r & (SCPR-1)).
  T* const C = static_cast<T*>(p.C);
  auto stage_addr = [&](int r, int cbyte) {
    return r * SROW + ((((cbyte >> 4) ^ (r & (SCPR - 1)))) << 4) + (cbyte & 15);
  };
  auto epilogue = [&](const Tile& t, int parity, unsigned char* S) {
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
      const int c0 = pass * PASS_COLS;
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const int r = wm * Cfg::BMW + i * 16 + lr;
#pragma unroll
        for (int j = 0; j < (GEMM1 ? NF / 2 : NF); ++j) {
          const int c = (GEMM1 ? wn * (Cfg::BNW / 2) : wn * Cfg::BNW) + j * 16 + lg * 4;
          if (c < c0 || c >= c0 + PASS_COLS) continue;             // wave-uniform
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[q] = GEMM1 ? silu_f(acc[i][j][q]) * acc[i][j + NF / 2][q] : acc[i][j][q];
          unsigned char* dst = S + stage_addr(r, (c - c0) * EB);
          if constexpr (DT == MEP_DTYPE_BF16) {
            uint2 w;
            w.x = pack_bf16x2(v[0], v[1]);
            w.y = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<uint2*>(dst) = w;
          } else {
            *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
          }
        }
      }
      lds_barrier();
      for (int q = tid; q < BM * SCPR; q += NT) {
        const int r = q / SCPR, ch = q % SCPR;
        if (t.row0 + r >= t.row_end) continue;
        int64_t dst;
        if constexpr (GEMM1) dst = static_cast<int64_t>(t.row0 + r) * p.N;
        else dst = static_cast<int64_t>(s_rows[parity * BM + r]) * p.N;
        dst += t.nt * CN + c0 + ch * EPC;
        *reinterpret_cast<u32x4*>(C + dst) = *reinterpret_cast<const u32x4*>(S + stage_addr(r, ch * 16));
      }
      if (pass + 1 < NPASS) lds_barrier();
    }
  };

  // ---- persistent tile loop -------------------------------------------------------
  // Per tile: step kt computes from stage kt&1 while step kt+1 streams into the
  // other stage; each wave's vmcnt(0) plus the barrier publish it.  KT is even,
  // so the last step reads stage 1 and stage 0 is free for the next tile's
  // first step, which streams in during that last step and while this tile's
  // epilogue drains via stage 1.  The next tile's row map streams in during
  // this tile's K loop.
  unsigned char* const stage0 = smem;
  unsigned char* const stage1 = smem + STAGE;
  const int KT = K / BKE;
  Tile cur = decode(tile_id(0));
  rowmap_dma(cur, 0);
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  lds_barrier();
  setup(cur, 0);
  load_stage(0, stage0);
  for (int it = 0; tile_valid(it); ++it) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    lds_barrier();
    const bool has_next = tile_valid(it + 1);
    Tile nxt = cur;
    if (has_next) {
      nxt = decode(tile_id(it + 1));
      rowmap_dma(nxt, (it + 1) & 1);              // its buffer's last reader was the previous epilogue
    }
    for (int kt = 0; kt < KT - 1; ++kt) {
      load_stage(kt + 1, (kt & 1) ? stage0 : stage1);
      compute((kt & 1) ? stage1 : stage0);
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      lds_barrier();
    }
    // last step: stage 0 is free (barrier above).  The next tile's first step
    // streams into it from here (GEMM-2) or from the end of this step (GEMM-1,
    // whose gather setup would otherwise be live across the step's MFMAs and
    // spill); either way the epilogue's staging writes wait for it, as the
    // compiler makes LDS writes after an LDS DMA do.
    const Tile done = cur;
    if (!GEMM1 && has_next) {
      cur = nxt;
      setup(cur, (it + 1) & 1);
      load_stage(0, stage0);
    }
    compute(stage1);
    lds_barrier();                                 // every wave is done with stage 1
    if (GEMM1 && has_next) {
      cur = nxt;
      setup(cur, (it + 1) & 1);                    // row map landed during the K loop
      load_stage(0, stage0);
    }
    epilogue(done, it & 1, stage1);
  }
}

template <int DT, class Cfg, bool GEMM1>
hipError_t launch(const GemmParams& p, int64_t max_rows, hipStream_t stream) {
  static int n_cu = 0;
  if (n_cu == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
      n_cu = 256;
  }
  int64_t tiles = ((max_rows + Cfg::BM - 1) / Cfg::BM + p.n_local) * p.n_tiles_n;
  if (tiles == 0) return hipSuccess;
  int64_t grid = tiles < n_cu ? tiles : n_cu;      // one persistent workgroup per CU
  grid = (grid + 7) / 8 * 8;
  grouped_gemm_kernel<DT, Cfg, GEMM1><<<dim3(static_cast<unsigned>(grid)), Cfg::NT, 0, stream>>>(p);
  return hipGetLastError();
}

// Tile shapes: bf16 256x256 (GEMM-1: 128 gate + 128 up columns) on 8 waves
// (4 x 2, 64 x 128 per wave, 2 waves per SIMD, no spills); fp32 128x128 on
// 4 waves.
typedef TileCfg<256, 256, 4, 2> CfgBf16;
typedef TileCfg<128, 128, 2, 2> CfgF32;

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
  // the kernels address x, act and one expert's weights with 32-bit byte offsets
  const int64_t eb = dtype_bytes(dtype);
  MEP_REQUIRE(n_tokens * hidden * eb < (int64_t(1) << 32) && max_rows * inter * eb < (int64_t(1) << 32),
              MEP_ERR_UNSUPPORTED, "%s: x or act larger than 4 GiB", fn);
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
