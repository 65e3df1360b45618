// Grouped SwiGLU experts on the gfx950 matrix cores.
//
// Replaces run_experts (modeling.py:83-104) and the row gather in front of it
// (modeling.py:143):
//     for each local expert e:  h = X_e @ W_in[e].T ; gate, up = h.chunk(2)
//                               y = (silu(gate) * up) @ W_out[e].T ; out[idx] = y
// over the dispatched rows (grouped by expert, ragged), as two GEMMs:
//   GEMM-1  act[r, :] = silu(x[perm[r]/k] W_g^T) * (x[perm[r]/k] W_u^T)
//           A rows are gathered from x inside the tile load (no permuted copy
//           of x is ever written); every output tile holds matching gate and
//           up columns, so SwiGLU runs in registers in the epilogue.
//   GEMM-2  y_entries[perm[r], :] = act[r, :] W_out^T
//           rows are scattered straight to their (token, slot) cell.
//
// Tiling (bf16, moe_gemm_bf16_kernel): 256 x 256 output tile, 8 waves (4 x 2)
// of 64 x 128.  K is staged 128 bytes per row at a time (64 bf16) through two
// LDS stages filled by buffer_load ... lds (global memory straight into LDS,
// no VGPR staging): one instruction moves 8 rows x 128 B; lane L lands at
// byte 16 L, so it fetches logical chunk (L%8) ^ (L/8) of its row, which
// stores each row's chunks XOR-swizzled by (row & 7) and makes the fragment
// reads (16 rows x one chunk) bank-conflict free.  The MFMA
// (v_mfma_f32_16x16x32_bf16, fp32 accumulation in VGPRs) takes the weight
// fragment as its first operand, so it produces C^T; with the weight rows
// permuted per 32-column group a lane ends up holding 8 consecutive output
// columns of one row.  GEMM-1 applies SiLU * up in registers and stores 16 B
// per lane; GEMM-2 regroups rows through a per-wave LDS slice into whole
// 128-byte lines and stores them non-temporally (y_entries is read once, by
// the combine).  fp32 keeps the simpler two-stage grouped_gemm_kernel.
//
// Scheduling (bf16, more than 1024 rows): persistent, one workgroup per CU,
// both GEMMs in one launch (kModeBoth; kModeGateUp / kModeDown run one of
// them).  The row tiles, derived on the device from `offsets` (no host round
// trip for the counts), are split into one contiguous range per XCD; each
// XCD's workgroups take its GEMM-1 column tiles, then its GEMM-2 column tiles,
// the first item of each workgroup fixed and the rest claimed one at a time
// from the queue's counter in the caller's `tile_queue`, and take other
// queues' items once their own is drained.  A GEMM-2 tile starts when every
// GEMM-1 tile of its row tile has counted its act rows complete.  The next
// tile's first two stages stream in during the last four steps and the
// epilogue of the current one.  Within a step, a wave two MFMA groups in runs
// at raised priority, which keeps the two waves of a SIMD from moving in
// lockstep.  At most 1024 rows (decode, small batches) run the small-batch
// kernels below instead: a workgroup per 32-row chunk and column block,
// weights streamed straight into registers, both GEMMs in one launch.  Every
// path walks K in the same order, so they give the same bits.
#include "combine_dev.h"
#include "common.h"
#include "router_dev.h"

#include <type_traits>

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
  const int32_t* w_slot;     // (n_local,) slot of local expert j in W, or NULL: slot j
  int n_local, top_k;
  int K;                     // reduction length
  int N;                     // output columns (GEMM-1: I; GEMM-2: H)
  int n_tiles_n;             // column tiles per row tile
  uint32_t a_bytes;          // size of A in bytes (< 4 GiB)
  uint32_t k_magic;          // entry / top_k == umulhi(entry, k_magic) >> k_shift for entry < 2^31
  int k_shift;
  int* flags;                // error flags word of the schedule buffer (sched::kFlags), or NULL
  int wait_limit;            // small-batch one launch: polls before a wait gives up
  int dbg_chunk;             // ... whose GEMM-2 waits for one count more (test hook; -1: none)
};

// Round-up reciprocal for exact division by d of every n < 2^31: with
// s = ceil(log2 d) and m = ceil(2^(31+s) / d) (< 2^32 for d >= 2),
// n / d == (n * m) >> (31 + s) == umulhi(n, m) >> (s - 1).  d == 1 is
// flagged by m = 0 (the quotient is n).
void div_magic(uint32_t d, uint32_t* magic, int* shift) {
  if (d <= 1) { *magic = 0; *shift = 0; return; }
  int s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  *magic = static_cast<uint32_t>(((uint64_t(1) << (31 + s)) + d - 1) / d);
  *shift = s - 1;
}

// silu(v) = v / (1 + e^-v) with the hardware exp2 and reciprocal (about 1 ulp
// each); saturates correctly: v -> -inf gives -0, v -> +inf gives v.
__device__ __forceinline__ float silu_f(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * 1.4426950408889634f));
}

// pre[j] = sum over experts i < j of ceil(rows_i / ROWS) * mult, pre[nl] = the
// total, with rows_i = off[i+1] - off[i] (off and pre in LDS).  One wave
// (the caller's wave 0) scans 64 experts per pass with lane shuffles; the
// caller synchronises the workgroup before and after.
template <int ROWS>
__device__ void scan_units(const int* off, int* pre, int nl, int mult) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int j0 = 0; j0 < nl; j0 += 64) {
    const int j = j0 + lane;
    int c = j < nl ? ((off[j + 1] - off[j] + ROWS - 1) / ROWS) * mult : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(c, d, 64);
      if (lane >= d) c += v;
    }
    if (j < nl) pre[j + 1] = carry + c;
    carry += __shfl(c, 63, 64);
  }
  if (lane == 0) pre[0] = 0;
}

// error flag of the schedule buffer: the offsets came from a dispatch that
// gave up (sched::kFlagInput)
constexpr int kFlagInputBit = 4;

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
  // (offsets[nl] < 0: the dispatch gave up; no expert has rows, the call is flagged)
  {
    const int last = p.offsets[nl];
    for (int j = tid; j <= nl; j += NT) s_off[j] = last < 0 ? 0 : p.offsets[j];
    if (last < 0 && blockIdx.x == 0 && tid == 0 && p.flags != nullptr) atomicOr(p.flags, kFlagInputBit);
  }
  __syncthreads();
  if (tid < 64) scan_units<BM>(s_off, s_prefix, nl, p.n_tiles_n);
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
      const int slot = p.w_slot != nullptr ? p.w_slot[t.e] : t.e;
      g_base = static_cast<const unsigned char*>(p.W) + static_cast<int64_t>(slot) * p.w_expert_stride * EB;
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
  const int n_cu = device_cu_count();
  int64_t tiles = ((max_rows + Cfg::BM - 1) / Cfg::BM + p.n_local) * p.n_tiles_n;
  if (tiles == 0) return hipSuccess;
  int64_t grid = tiles < n_cu ? tiles : n_cu;      // one persistent workgroup per CU
  grid = (grid + 7) / 8 * 8;
  grouped_gemm_kernel<DT, Cfg, GEMM1><<<dim3(static_cast<unsigned>(grid)), Cfg::NT, 0, stream>>>(p);
  return hipGetLastError();
}

// ============================================================================
// bf16 path: 8 waves, two 64 KiB LDS stages of two K-steps each, inline-asm
// MFMAs with VGPR accumulators.
//
// Tile 256 x 256 (GEMM-1: 128 gate + 128 up columns), 8 waves (4 x 2) of
// 64 x 128.  One MFMA step covers 32 of K; a stage holds two steps (128 bytes
// of every A row and weight row) and is filled by buffer_load_dwordx4 ... lds:
// one instruction moves 8 whole 128-byte lines (full lines move about 25 %
// faster than the 64-byte half lines of one-step stages; measured).  Stage d
// of a tile sits in buffer d & 1, and the stages of consecutive tiles run on
// through the same two buffers, so the next tile's first stages stream in
// while this tile's last steps and its epilogue run.  Within stage d:
//   even step 2d   - MFMAs on the fragments of step 2d (read during step 2d-1),
//                    read the fragments of step 2d+1 (same stage), then wait
//                    for stage d+1's DMA and join a barrier;
//   odd step 2d+1  - issue stage d+2's DMA into buffer d & 1 (free: its last
//                    fragments were read during step 2d, before that barrier),
//                    MFMAs on step 2d+1, read the fragments of step 2d+2 from
//                    stage d+1 (published by that barrier).  No barrier.
// So a stage's DMA has two steps to land, and there is one barrier per stage.
// MFMAs run column-major (the 4 MFMAs of weight fragment j, then j+1): row
// fragments are double-buffered, weight fragment j is refilled right after its
// group.  The MFMAs are inline asm with "+v" accumulators: the 128
// accumulators stay in arch VGPRs next to everything else (the kernel uses
// all 256 a wave has at two waves per SIMD), so the epilogue reads them without 128
// v_accvgpr_read moves (with the builtin the compiler moves them between
// register files and spills).
//
// Epilogue straight from the accumulators (16-byte stores, see pair_cols;
// GEMM-2 regroups them into whole lines in LDS), no workgroup barrier.
// GEMM-2 rotates the K order of a tile by its column-tile index (n_tile * KD /
// 4 stages), which spreads the tiles running at the same time over more
// memory channels.  GEMM-1 does not: its 4 column tiles of a row tile run
// side by side on one XCD and then read the same gathered x rows at about the
// same time, so 3 of the 4 reads hit that XCD's L2 (measured on one box: 234
// -> 223 us without the rotation).  Either way the order depends only on the
// output columns, so every output element is summed in the same order
// wherever its row sits in the dispatch.
namespace bfk {
constexpr int BM = 256, BN = 256, NT = 512, NW = 8;
constexpr int KS = 32;                        // K per MFMA step (16x16x32)
constexpr int RB = 128;                       // bytes per row of a stage: two steps of K
constexpr int HALF = BM * RB;                 // A rows of one stage (32 KiB); the weight rows take as much
constexpr int BREGION = 2 * HALF;             // weight rows of both stages start at 64 KiB
constexpr int MF = 4, NF = 8;                 // 16 x 16 fragments per wave (64 x 128)
constexpr int BPW = 8;                        // 1 KiB DMA blocks (8 rows x 128 B) per wave per stage
constexpr int NLMAX = 256;
// GEMM-2 output staging: 8 rows x 256 B (a wave's 128 columns) per wave,
// after the stage buffers; the tables follow it
constexpr int STG_ROWS = 8, STG_WAVE = STG_ROWS * 256, STG = 4 * HALF;
constexpr int TABLES = STG + NW * STG_WAVE;
// row tile -> expert, one byte each, for launches of at most RT_TAB row
// tiles (T <= 256k tokens at top-8); larger ones search the prefix table
constexpr int RT_TAB = 8192;
constexpr int LDS_BYTES = TABLES + (2 * (NLMAX + 1) + 2 * BM + 8 + NLMAX) * 4 + RT_TAB;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of one workgroup");
// buffer resource word 3 for raw 32-bit buffer access on gfx9-family parts
constexpr int kBufWord3 = 0x00020000;
static_assert(BN * RB == HALF, "A and weight rows of a stage are the same size");
static_assert((BM + BN) / 8 == NW * BPW, "DMA blocks cover the stage");
static_assert(BPW == NF, "one DMA block per MFMA group of an odd step");
}  // namespace bfk

// Words of the bf16 tiled kernels' schedule buffer (`tile_queue` of the C ABI,
// int32, sched::words(max_rows, n_local) of them).  Each word that many
// workgroups update has a 128-byte line of its own (index x kLine): device-
// scope atomics on one line are performed one after another where the line
// lives, so counters sharing a line queue behind each other's traffic.
//   line q < 8       items taken from XCD q's queue
//   line 8           workgroups finished
//   line 9           items computed
//   line 10          error flags, sticky (never cleared by a launch;
//                    mep_experts_check reads and clears them):
//                    kFlagWait  a GEMM-2 tile gave up waiting for its rows
//                               (or the combine for GEMM-2's); its
//                               outputs are NaN
//                    kFlagDrain items computed != items listed (never expected)
//                    kFlagInput offsets[n_local] < 0: the dispatch gave up,
//                               no tile ran
//   line 11          bit per drained queue
//   lines 12, 13     small-batch launch ending with the combine: GEMM-2
//                    workgroups done, combine workgroups past their wait
//   line 16 + r      row tile r's GEMM-1 column tiles finished (kModeBoth);
//                    the small-batch launch of both GEMMs: chunk r's GEMM-1
//                    counts and GEMM-2 workgroups past their wait (words 0, 1)
// Every launch leaves every word but the flags zero.
namespace sched {
constexpr int kLine = 32;                      // ints per 128-byte line
constexpr int kQueue = 0, kDone = 8 * kLine, kItems = 9 * kLine, kFlags = 10 * kLine, kDrained = 11 * kLine,
              kG2Done = 12 * kLine, kCombDone = 13 * kLine, kRowDone = 16 * kLine;
__host__ __device__ constexpr int queue_word(int q) { return kQueue + q * kLine; }
__host__ __device__ constexpr int row_word(int r) { return kRowDone + r * kLine; }
constexpr int kFlagWait = 1, kFlagDrain = 2, kFlagInput = kFlagInputBit;
constexpr int kWaitLimit = 1 << 20;            // polls of one row counter (about a second)
// the small-batch launch of both GEMMs runs up to this many rows
constexpr int64_t kSmallRows = 1024;
// row tiles of max_rows rows over n_local experts: each expert adds at most
// one partial tile; the small-batch launch of both GEMMs keeps a line per
// 32-row chunk there instead
inline int64_t words(int64_t max_rows, int n_local) {
  const int64_t tiles = (max_rows + 255) / 256 + n_local;
  const int64_t chunks = max_rows <= kSmallRows ? (max_rows + 31) / 32 + n_local : 0;
  return kRowDone + (tiles > chunks ? tiles : chunks) * kLine;
}
}  // namespace sched

constexpr int kModeGateUp = 1, kModeDown = 2, kModeBoth = 3;
struct MoeParams {
  const void* x;             // (n_tokens, H)
  void* act;                 // (max_rows, I): GEMM-1's output, GEMM-2's A operand
  void* y;                   // (N*k, H) y_entries
  const int32_t* perm;       // row -> flat entry id
  const int32_t* offsets;    // (n_local + 1) row offsets per local expert
  const int32_t* w_slot;     // (n_local,) slot of local expert j, or NULL: slot j
  const void* w_in;          // (slots, 2I, H)
  const void* w_out;         // (slots, H, I)
  int n_local, top_k, H, I;
  uint32_t x_bytes, act_bytes;   // sizes of x and act in bytes (< 4 GiB)
  uint32_t k_magic;          // entry / top_k == umulhi(entry, k_magic) >> k_shift (k_magic 0: k = 1)
  int k_shift;
  int n_queues;              // queues (XCDs), a power of two <= 8
  int* sched;
  int wait_limit;            // polls of a row counter before a GEMM-2 tile gives up
  int dbg_row;               // row tile whose GEMM-2 tiles wait for one count more (test hook; -1: none)
};

// 16x16x32 bf16 MFMA with the accumulator in VGPRs; src0 = weight
// fragment, src1 = row fragment, so the result is C^T (lane: one row, 4
// consecutive columns).  mfma_first starts a new accumulation (C operand 0).
__device__ __forceinline__ void mfma_acc(f32x4& acc, const u32x4& w, const u32x4& a) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(w), "v"(a));
}
__device__ __forceinline__ void mfma_first(f32x4& acc, const u32x4& w, const u32x4& a) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(w), "v"(a));
}
// Orders later reads of `acc` after every earlier volatile asm (an empty asm
// that claims to rewrite it).  AMDGPU register constraints live in device
// functions only: in a kernel body the host pass parses them as x86 ones.
__device__ __forceinline__ void pin_acc(f32x4& acc) { asm volatile("" : "+v"(acc)); }
// buffer_load_dwordx4 ... lds of one 1 KiB block: lane L's 16 bytes from
// base + voff + soff land at lds + 16 L; an offset at or past `bytes` reads
// zeros instead of faulting.  (A plain device function: inside the kernel
// template the host pass drops the kernel's launch stub.)
// The resource is rebuilt from scalars read with readfirstlane: wherever the
// compiler kept base / bytes, the descriptor is then in SGPRs (a descriptor it
// thinks may be divergent gets a readfirstlane loop around every load).
__device__ __forceinline__ void buffer_lds_16(const unsigned char* base, int bytes, uint32_t voff, int soff,
                                              unsigned char* lds) {
  // readfirstlane returns int: cast each half to uint32_t before widening, or
  // a low word with bit 31 set would sign-extend over the high word
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xFFFFFFFFu)));
  const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | lo;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bs), 0, __builtin_amdgcn_readfirstlane(bytes),
                                        bfk::kBufWord3),
      (__attribute__((address_space(3))) void*)lds, 16, voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

// Grouped GEMM over 256-row tiles of the dispatched rows: GEMM-1 + SwiGLU
// (MODE kModeGateUp), GEMM-2 + scatter (kModeDown), or both in one launch
// (kModeBoth).  Tiles are (row tile, column tile) pairs; a row tile is 256
// consecutive rows of one expert (an expert's last one may be partial).
//
// Queues.  The row tiles are split into n_queues contiguous ranges, one per
// XCD, and the workgroups of an XCD take that range's tiles in order: the
// first without a claim (workgroup b takes item b / n_queues of queue
// b % n_queues; workgroups are dispatched to the XCDs round robin, so that is
// b's XCD's queue, which matters only for L2 locality), the rest one at a
// time through the queue's counter in `sched`, past those fixed slots.  The
// tiles of one expert run on one XCD and share its weights in that XCD's L2,
// and the column tiles of a row tile, taken one after the other, share the
// row tile's A rows there.  The
// XCDs do not run at one speed (the same work takes up to 8 % longer on one
// than on another), so a workgroup whose queue is drained takes the
// remaining tiles of the other queues (a bit per drained queue in `sched`
// spares it the atomics on those).
// In kModeBoth a queue lists GEMM-1's tiles of its row tiles, then GEMM-2's
// (measured: GEMM-2 row tiles 4 or 8 row tiles behind GEMM-1's, to reuse act
// from L2, ran 4-15 % slower than this order).  A GEMM-2 tile needs every GEMM-1 column tile of its row tile
// done (act is its A operand): each GEMM-1 tile, once its stores are
// complete, adds one to its row tile's counter in `sched`, and a GEMM-2 tile
// starts when that counter is full.  GEMM-1 stores act with device scope
// (written through to memory), so a GEMM-2 tile on any XCD reads the final
// rows: its XCD's caches hold no line of them (it reads them only after they
// are final, and every launch starts with clean caches).  The wait is checked
// four steps before the tile in front of it would prefetch the GEMM-2
// tile's first stages; if it is not met there, the workgroup finishes its tile, counts it, and
// waits between tiles with nothing of its own pending: a workgroup that waits
// holds no unfinished tile, and the tiles it waits for come earlier in the
// queue than the one it waits with (fixed slots come before claimed ones),
// so every wait ends.  A wait that still
// exceeds p.wait_limit polls (sched::kWaitLimit) sets sched flag kFlagWait,
// and the tile then stores NaN.
// Which workgroup computes a tile never changes its result, so the bits are
// those of two separate launches.
// Device-scope atomics of a single lane (thread 0 of a workgroup).  The
// offset (and for reads the addend) is an opaque zero: with a uniform
// address the compiler combines the atomic across the wave and reads its
// result back into a scalar right away, which stalls the wave on every
// memory operation it has in flight (the stage DMA included); and it turns
// an add of a known 0 into an atomic load, which may be answered from a
// cache line another XCD has since changed.  With the opaque zero these stay
// one read-modify-write each, performed where every XCD's atomics are.
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}
__device__ __forceinline__ int atomic_add_1(int* p, int v) { return atomicAdd(p + opaque_zero(), v); }
__device__ __forceinline__ int atomic_read(int* p) {
  const int z = opaque_zero();
  return atomicAdd(p + z, z);
}
__device__ __forceinline__ int atomic_or_1(int* p, int v) { return atomicOr(p + opaque_zero(), v); }
// Device-scope 32-bit load (written earlier in this launch, possibly on
// another XCD): what a wait polls, so that the counter's line only sees the
// counting read-modify-writes.
__device__ __forceinline__ int load_dev_i32(const int32_t* q) {
  return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte store with device scope (sc1): written through to memory, where a
// later read from another XCD finds it.  base / bytes as in buffer_lds_16.
__device__ __forceinline__ void store_dev_16(void* base, uint32_t bytes, uint32_t voff, const u32x4& v) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xFFFFFFFFu)));
  const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | lo;
  __builtin_amdgcn_raw_buffer_store_b128(
      v, __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bs), 0,
                                           __builtin_amdgcn_readfirstlane(static_cast<int>(bytes)), bfk::kBufWord3),
      voff, 0, 16 /* sc1: device scope */);
}

// 16-byte load with device scope (sc1): it does not return a line this XCD's
// caches kept from before another XCD rewrote it.  base / bytes as in
// buffer_lds_16.
__device__ __forceinline__ u32x4 load_dev_16(const void* base, uint32_t bytes, uint32_t voff) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xFFFFFFFFu)));
  const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | lo;
  return __builtin_amdgcn_raw_buffer_load_b128(
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bs), 0,
                                        __builtin_amdgcn_readfirstlane(static_cast<int>(bytes)), bfk::kBufWord3),
      voff, 0, 16 /* sc1: device scope */);
}

template <int MODE>
__global__ __launch_bounds__(bfk::NT) void moe_gemm_bf16_kernel(MoeParams p) {
  using namespace bfk;
  constexpr bool BOTH = MODE == kModeBoth;
  __shared__ __attribute__((aligned(16))) unsigned char smem[LDS_BYTES];
  int* const s_prefix = reinterpret_cast<int*>(smem + TABLES);         // [NLMAX + 1] row tiles before expert j
  int* const s_off = s_prefix + NLMAX + 1;                             // [NLMAX + 1] row offsets
  int* const s_rows = s_off + NLMAX + 1;                               // [2][BM] row maps
  int* const s_msg = s_rows + 2 * BM;                                  // [8] answers of thread 0's atomics
  int* const s_slot = s_msg + 8;                                       // [NLMAX] weight slot of expert j
  unsigned char* const s_rt_e = reinterpret_cast<unsigned char*>(s_slot + NLMAX);   // [RT_TAB] expert of row tile R

  const int tid = threadIdx.x;
  // wave index as a scalar: keeps per-wave choices (A or weight rows, buffer
  // resources) in SGPRs
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nl = p.n_local;
  const int n1 = p.I / (BN / 2), n2 = p.H / BN;  // column tiles of a row tile: GEMM-1, GEMM-2
  int* const sched = p.sched;

  // First items need no claim: workgroup b takes item b / nq of queue b % nq.
  // Workgroups are dispatched to the XCDs round robin, so queue b % nq is
  // b's XCD's (which only matters for L2 locality); every other item is
  // claimed from a queue's counter, past the queue's n_static fixed slots.
  const int nq = p.n_queues;
  const int q = static_cast<int>(blockIdx.x) & (nq - 1);
  const int n_static = static_cast<int>(gridDim.x) / nq;   // the grid is a multiple of nq
  const int first_pos = static_cast<int>(blockIdx.x) / nq;
  auto claim = [&](int qq) { return n_static + atomic_add_1(sched + sched::queue_word(qq), 1); };

  // ---- row tiles ------------------------------------------------------------------
  // offsets[nl] < 0: the dispatch gave up (its outputs are poisoned); then no
  // expert has rows, no tile runs and the call is flagged
  {
    const int last = p.offsets[nl];
    for (int j = tid; j <= nl; j += NT) s_off[j] = last < 0 ? 0 : p.offsets[j];
    if (last < 0 && blockIdx.x == 0 && tid == 0) atomic_or_1(sched + sched::kFlags, sched::kFlagInput);
  }
  for (int j = tid; j < nl; j += NT) s_slot[j] = p.w_slot != nullptr ? p.w_slot[j] : j;
  __syncthreads();
  if (tid < 64) scan_units<BM>(s_off, s_prefix, nl, 1);
  __syncthreads();
  const int RT = __builtin_amdgcn_readfirstlane(s_prefix[nl]);
  const bool rt_tab = RT <= RT_TAB;
  if (rt_tab)
    for (int j = tid; j < nl; j += NT)
      for (int r = s_prefix[j]; r < s_prefix[j + 1]; ++r) s_rt_e[r] = static_cast<unsigned char>(j);
  __syncthreads();

  // ---- queues ---------------------------------------------------------------------
  // Queue qq holds row tiles [lo(qq), lo(qq + 1)); a workgroup starts on its
  // XCD's queue and, when that is drained, takes tiles from the others.
  constexpr int kPerRowMode = MODE == kModeGateUp ? 1 : (MODE == kModeDown ? 2 : 3);
  const int per_row = kPerRowMode == 1 ? n1 : (kPerRowMode == 2 ? n2 : n1 + n2);
  auto q_lo = [&](int qq) { return static_cast<int>(static_cast<int64_t>(RT) * qq / nq); };
  auto q_items = [&](int qq) { return (q_lo(qq + 1) - q_lo(qq)) * per_row; };

  // Item `pos` of the queue -> tile.  g1: a GEMM-1 tile; R: global row tile;
  // nt: column tile.  The row tile's expert is the largest j with
  // s_prefix[j] <= R.  act_wm: waves with wm >= act_wm compute nothing (a
  // row tile of at most 128 rows, an expert's last, runs on the 4 waves of
  // rows 0..127, one per SIMD, and sums every output element in the same
  // order as a whole tile).
  struct Tile { int g1, e, slot, row0, row_end, nt, act_wm, R; };
  auto decode = [&](int pos, int qq) {
    const int r_lo = q_lo(qq), nr = q_lo(qq + 1) - r_lo;
    int g1, R, c;
    if constexpr (!BOTH) {
      g1 = MODE == kModeGateUp;
    } else {
      g1 = pos < nr * n1;
      if (!g1) pos -= nr * n1;
    }
    const int w = g1 ? n1 : n2;
    R = pos / w;
    c = pos - R * w;
    R += r_lo;
    int lo = 0;
    if (rt_tab) {
      lo = s_rt_e[R];
    } else {
      int hi = nl - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_prefix[mid] <= R) lo = mid; else hi = mid - 1;
      }
    }
    Tile t;                                        // uniform: keep it in SGPRs
    t.g1 = __builtin_amdgcn_readfirstlane(g1);
    t.e = __builtin_amdgcn_readfirstlane(lo);
    t.slot = __builtin_amdgcn_readfirstlane(s_slot[lo]);
    t.row0 = __builtin_amdgcn_readfirstlane(s_off[lo] + (R - s_prefix[lo]) * BM);
    t.row_end = __builtin_amdgcn_readfirstlane(s_off[lo + 1]);
    t.nt = __builtin_amdgcn_readfirstlane(c);
    t.R = __builtin_amdgcn_readfirstlane(R);
    t.act_wm = (t.row_end - t.row0 <= BM / 2) ? 2 : 4;
    return t;
  };
  // GEMM-1 counts a GEMM-2 tile of row tile R waits for: n1 (one more for
  // the test hook's row tile, which therefore gives up)
  auto need = [&](int R) { return n1 + (R == p.dbg_row ? 1 : 0); };
  // thread 0: until row tile R's GEMM-1 tiles are all counted (bounded);
  // returns 1 if the wait gave up (the tile then stores NaN)
  auto wait_rows = [&](int R) {
    int polls = 0;
    while (load_dev_i32(sched + sched::row_word(R)) < need(R)) {
      if (++polls == p.wait_limit) {
        atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
        return 1;
      }
      __builtin_amdgcn_s_sleep(4);
    }
    return 0;
  };
  // row map: perm[row0 .. row0 + BM) of a tile DMA'd into LDS (clamped to the
  // tile's last row, so every lane reads inside perm).  GEMM-1 gathers its A
  // rows through it, GEMM-2 scatters its output rows.
  static_assert(BM % 64 == 0 && BM / 64 <= NW, "row-map DMA: one 64-row instruction per wave");
  auto rowmap_dma = [&](const Tile& t, int parity) {
    if (wave < BM / 64) {
      const int r = min(t.row0 + wave * 64 + lane, t.row_end - 1);
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(p.perm + r),
                                       (__attribute__((address_space(3))) void*)(s_rows + parity * BM + wave * 64),
                                       4, 0, 0);
    }
  };

  // ---- DMA sources ----------------------------------------------------------------
  // Block q = wave * BPW + i (waves 0-3: A rows 8q .. 8q+7; waves 4-7: weight
  // rows 8(q - 32) ..); lane L moves 16 B of row 8q + L/8 into byte 16 L of
  // the block, i.e. physical chunk L & 7, and fetches logical chunk
  // (L & 7) ^ (row & 7): 128-byte rows XOR-swizzled by r & 7, which makes the
  // fragment reads conflict-free.
  const bool wave_a = wave < 4;
  // Output columns of a weight stage row.  Within each aligned group of 32
  // rows (two 16-column fragments j, j+1), fragment row n of fragment j2 holds
  // column 8 (n / 4) + 4 j2 + n % 4: lane group lg then owns columns
  // 8 lg .. 8 lg + 7 of the group across the two fragments (16 contiguous
  // bytes of bf16 output per lane and store).
  auto pair_cols = [](int rb) { return (rb & ~31) | (((rb & 15) >> 2) << 3) | (((rb >> 4) & 1) << 2) | (rb & 3); };
  // Weight stage rows: wave wn's fragments j < 4 read rows wn*64 + 16 j ..,
  // fragments j >= 4 rows 128 + wn*64 + 16 (j - 4) ..  GEMM-1: rows < 128 are
  // gate rows, rows >= 128 the matching up rows (act columns nt*128 + wn*64
  // + pair_cols(16 j ..)).  GEMM-2: the same rows hold output columns
  // nt*256 + wn*128 + pair_cols(16 j ..), so both read one LDS layout.
  auto weight_row = [&](const Tile& t, int rb0) {
    if (t.g1) return (rb0 < BN / 2 ? 0 : p.I) + t.nt * (BN / 2) + pair_cols(rb0 & (BN / 2 - 1));
    const int l = (rb0 & 63) + (rb0 >= BN / 2 ? 64 : 0);
    return t.nt * BN + ((rb0 & (BN / 2 - 1)) >> 6) * 128 + pair_cols(l);
  };
  // (base, bytes) rather than a buffer resource: a struct member of type
  // __amdgpu_buffer_rsrc_t makes the host pass drop the kernel's launch stub
  struct Src { const unsigned char* base; int bytes; uint32_t off[BPW]; int rot, kd; };
  auto setup = [&](const Tile& t, int parity) {
    // recompute the per-lane row terms here instead of keeping them live across
    // the whole tile loop (hoisted, they outgrow the register budget and spill)
    int lrow = lane >> 3, lchunk = (lane & 7) ^ (lane >> 3);
    asm volatile("" : "+v"(lrow), "+v"(lchunk));
    int wv = wave;                             // opaque here too: no per-block constant is hoisted
    asm volatile("" : "+s"(wv));
    const int K = t.g1 ? p.H : p.I;
    Src s;
    s.kd = K / (2 * KS);
    // GEMM-2 rotates its K order by the column tile (memory channels)
    s.rot = (!t.g1 && s.kd % 4 == 0) ? (t.nt & 3) * (s.kd / 4) : 0;
    if (wave_a) {
      s.base = static_cast<const unsigned char*>(t.g1 ? p.x : p.act);
      s.bytes = static_cast<int>(t.g1 ? p.x_bytes : p.act_bytes);
      // 32-bit offsets: the size checks keep x and act below 4 GiB
      const uint32_t lane_off = static_cast<uint32_t>(lchunk * 16);
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int r0 = (wv * BPW + i) * 8;                  // wave-uniform
        uint32_t src_row;
        if (t.g1) {
          const uint32_t f = static_cast<uint32_t>(s_rows[parity * BM + r0 + lrow]);   // flat entry t*k + s
          src_row = p.k_magic ? (__umulhi(f, p.k_magic) >> p.k_shift) : f;
        } else {
          src_row = static_cast<uint32_t>(min(t.row0 + r0 + lrow, t.row_end - 1));
        }
        s.off[i] = src_row * static_cast<uint32_t>(K * 2) + lane_off;
      }
      // a row half needs only A rows 0..127 (waves 0-1): the other A waves'
      // loads read past a zero-sized buffer, i.e. zeros, without memory traffic
      if (t.act_wm < 4 && wv * BPW * 8 >= t.act_wm * 64) s.bytes = 0;
    } else {
      const int64_t stride = static_cast<int64_t>(t.g1 ? 2 * p.I : p.H) * K;   // elements per expert
      s.base = static_cast<const unsigned char*>(t.g1 ? p.w_in : p.w_out) + static_cast<int64_t>(t.slot) * stride * 2;
      s.bytes = static_cast<int>(stride * 2);
      // weight row of stage row rb0 + lrow (rb0 = the block's first row, a
      // multiple of 8): weight_row(rb0) + lane part, so the row split into a
      // scalar per block and one per-lane term
      const int lp = ((lrow & 4) << 1) | (lrow & 3);
      const uint32_t lane_off = static_cast<uint32_t>((lp * K + lchunk * 8) * 2);
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int rb0 = ((wv - 4) * BPW + i) * 8;          // wave-uniform
        s.off[i] = static_cast<uint32_t>(weight_row(t, rb0) * K * 2) + lane_off;
      }
    }
    return s;
  };
  // stage buffers: A rows of buffer b at b * 32 KiB, weight rows at
  // 64 KiB + b * 32 KiB, so each fragment read is one of four base registers
  // plus an immediate below 64 KiB
  const int lds_blk = wave_a ? wave * BPW * 1024 : BREGION + (wave - 4) * BPW * 1024;
  auto dma_blk = [&](const Src& s, int kd, int buf, int i) {
    int ke = kd + s.rot;
    if (ke >= s.kd) ke -= s.kd;
    // opaque: otherwise the 16 destinations (buffer x block) are hoisted into
    // scalar registers, which the loop does not have to spare
    int lb = lds_blk;
    asm volatile("" : "+s"(lb));
    buffer_lds_16(s.base, s.bytes, s.off[i], ke * RB, smem + lb + buf * HALF + i * 1024);
  };

  // ---- fragments ------------------------------------------------------------------
  // Lane (lr, lg) reads 16 B of row 16 i + lr at logical chunk 4 kk + lg
  // (kk = step parity within the stage), stored at chunk (4 kk + lg) ^ (lr & 7).
  const int lr = lane & 15, lg = lane >> 4;
  uint32_t a_base[2], b_base[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const uint32_t cp = static_cast<uint32_t>(((4 * kk + lg) ^ (lr & 7)) << 4);
    a_base[kk] = static_cast<uint32_t>((wm * 64 + lr) * RB) + cp;
    b_base[kk] = static_cast<uint32_t>(BREGION + (wn * 64 + lr) * RB) + cp;
  }
  // weight fragment j: rows 16 j (j < 4) or 128 + 16 (j - 4) past the wave's first
  auto b_off = [&](int j) { return j < 4 ? j * 16 * RB : (BN / 2 + (j - 4) * 16) * RB; };
  u32x4 fa[2][MF], fb[NF];
  f32x4 acc[MF][NF];

  // One step: MFMAs on fa[SET] / fb.  EVEN steps read the fragments of the
  // step's second half of the stage in buffer rbuf and end with the stage
  // wait + barrier; ODD steps issue the DMA of stage dkd (of the tile `s`
  // describes) into buffer dbuf, one block per MFMA group, and read the next
  // stage's first-step fragments from rbuf (unless !RD).  ZERO starts the
  // accumulation.  An idle wave of a row-half tile only moves its DMA blocks.
  auto step = [&](auto set_c, auto zero_c, auto odd_c, auto rd_c, const Src& s, int dkd, int dbuf, int rbuf,
                  bool act) {
    constexpr int SET = decltype(set_c)::value;
    constexpr bool ZERO = decltype(zero_c)::value, ODD = decltype(odd_c)::value, RD = decltype(rd_c)::value;
    constexpr int RKK = ODD ? 0 : 1;                 // which half of the stage the read fragments are
    const unsigned char* R = smem + rbuf * HALF;
    if (!act) {
      if constexpr (ODD) {
#pragma unroll
        for (int i = 0; i < BPW; ++i) dma_blk(s, dkd, dbuf, i);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NF; ++j) {
        if constexpr (ODD) dma_blk(s, dkd, dbuf, j);
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          if constexpr (ZERO) mfma_first(acc[i][j], fb[j], fa[SET][i]);
          else mfma_acc(acc[i][j], fb[j], fa[SET][i]);
        }
        if constexpr (RD) {
          // the next step's first group needs all four row fragments: read
          // them in the first four groups (their own register set is free)
          if (j < MF) fa[SET ^ 1][j] = *reinterpret_cast<const u32x4*>(R + a_base[RKK] + j * 16 * RB);
          fb[j] = *reinterpret_cast<const u32x4*>(R + b_base[RKK] + b_off(j));
        }
        asm volatile("" ::: "memory");
        // a wave two groups into its step goes ahead of the other wave of
        // its SIMD until the step ends: the pair drifts apart instead of
        // issuing its DMA blocks and fragment reads in lockstep (same box:
        // GEMM-1 -1.6 us, GEMM-2 -2 us; raised from the first group, or
        // later, it gains less)
        if (j == 1) __builtin_amdgcn_s_setprio(1);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (!ODD) {
      // the stage DMA'd during the previous step has landed (nothing else this
      // wave issued since is a load), every fragment read of this step is done
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      lds_barrier();
    }
  };
  // fragments of a tile's first step (stage 0 = buffer 0, first half): read at
  // the tile start, after the previous epilogue, so no fragment registers are
  // live across an epilogue
  auto first_frags = [&]() {
#pragma unroll
    for (int g = 0; g < MF; ++g) fa[0][g] = *reinterpret_cast<const u32x4*>(smem + a_base[0] + g * 16 * RB);
#pragma unroll
    for (int j = 0; j < NF; ++j) fb[j] = *reinterpret_cast<const u32x4*>(smem + b_base[0] + b_off(j));
    __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  };

  // ---- epilogues ------------------------------------------------------------------------
  // From the accumulators: with the weight rows permuted per 32-column group
  // (pair_cols), lane (lr, lg) of the fragment pair (2 jp, 2 jp + 1) in row
  // fragment i holds 8 consecutive output columns of one row.  GEMM-1 stores
  // them directly (16 rows x 64 contiguous bytes per instruction; its SiLU
  // keeps the VALU busier than the stores); GEMM-2 regroups them into whole
  // lines through a per-wave LDS slice.  No workgroup barrier: the stores
  // drain while the next tile's MFMAs run.
  typedef uint16_t T;
  auto epilogue = [&](const Tile& t, int parity, int poison) {
    if (wm >= t.act_wm) return;
    // the last MFMAs' results must be written before they are read (the
    // asm hides the MFMAs from the hazard recognizer): pad, then tie every
    // accumulator to an (empty) asm after the padding so no read moves above it
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) pin_acc(acc[i][j]);
    // a GEMM-2 tile whose wait for its rows gave up stores NaN
    if (poison) {
      const float nan = __builtin_nanf("");
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc[i][j] = f32x4{nan, nan, nan, nan};
    }
    // per-lane terms from an opaque copy of the thread index, so the compiler
    // cannot hoist them out of the tile loop (they would be spilled there)
    int et = tid;
    asm volatile("" : "+v"(et));
    const int elr = et & 15, elg = (et >> 4) & 3;
    if (MODE == kModeGateUp || (BOTH && t.g1)) {
      // act columns: lane (elr, elg) of fragment pair jp holds 8 of them
      T* const C = static_cast<T*>(p.act);
      const int col = t.nt * (BN / 2) + wn * 64 + elg * 8;                // first column of fragment pair 0
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const int r = wm * 64 + i * 16 + elr;
        T* const dst = C + static_cast<int64_t>(t.row0 + r) * p.I + col;
        const bool ok = t.row0 + r < t.row_end;
#pragma unroll
        for (int jp = 0; jp < NF / 4; ++jp) {                               // fragment pairs (2 jp, 2 jp + 1)
          float v[8];
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              v[4 * h + q4] = silu_f(acc[i][2 * jp + h][q4]) * acc[i][2 * jp + h + NF / 2][q4];
          u32x4 w;
#pragma unroll
          for (int h = 0; h < 4; ++h) w[h] = pack_bf16x2(v[2 * h], v[2 * h + 1]);
          if (ok) {
            if constexpr (BOTH)
              store_dev_16(p.act, p.act_bytes, static_cast<uint32_t>((t.row0 + r) * p.I + col + jp * 32) * 2u, w);
            else
              *reinterpret_cast<u32x4*>(dst + jp * 32) = w;
          }
        }
      }
    } else {
      // GEMM-2: lane (elr, elg) holds 16-byte chunk 4 jp + elg of row elr of
      // each row fragment, i.e. 64 bytes of a row per store instruction.  The
      // rows go through this wave's LDS slice instead (8 rows at a time,
      // chunk c of row r at (c ^ r) * 16: conflict-free both ways) and leave
      // as 4 rows x 256 contiguous bytes per store: whole 128-byte lines,
      // which the memory system takes about twice as fast as half lines.
      // The slice is private to the wave and a wave's LDS accesses complete
      // in issue order, so no barrier or wait is needed around it: round k
      // (rows 8k .. 8k+7 of the wave's 64) writes the slice before round
      // k-1's stores go out and reads it back after them, so the wait for a
      // round's reads overlaps the next round's writes (the row map's
      // destination cells are read with the round's data).  The output base
      // is held in scalar registers (a kernel argument reloaded mid-epilogue
      // is a scalar load, whose wait also waits for every LDS access in
      // flight).
      const int lrow = (et >> 4) & 3, lchunk = et & 15;                    // read-back: row lrow (+4), chunk lchunk
      unsigned char* const stg = smem + STG + wave * STG_WAVE;
      uint64_t ybase = reinterpret_cast<uint64_t>(static_cast<T*>(p.y) + t.nt * BN + wn * 128);
      uint32_t ystride = static_cast<uint32_t>(p.H) * 2u;
      asm volatile("" : "+s"(ybase), "+s"(ystride));
      constexpr int NR = 2 * MF;                                           // rounds of 8 rows
      const int n_ok = t.row_end - t.row0 - wm * 64;                       // rows of this wave's 64 that exist
      const int* const rmap = s_rows + parity * BM + wm * 64 + lrow;
      u32x4 w[NF / 2], d[2];
      int cell[2];                                                         // (token, slot) cells of the stores
#pragma unroll
      for (int k = 0; k <= NR; ++k) {
        if (k < NR) {
          const int i = k >> 1, half = k & 1;
          // packed again for each half (the VALU is otherwise idle here):
          // holding the packed row fragment across both halves costs the
          // registers that the read-back of the previous round needs (the
          // empty asm keeps the compiler from reusing the first packing)
          if (half == 1)
#pragma unroll
            for (int j = 0; j < NF; ++j) pin_acc(acc[i][j]);
#pragma unroll
          for (int jp = 0; jp < NF / 2; ++jp)
#pragma unroll
            for (int h = 0; h < 4; ++h)
              w[jp][h] = pack_bf16x2(acc[i][2 * jp + h / 2][2 * (h & 1)], acc[i][2 * jp + h / 2][2 * (h & 1) + 1]);
          if ((elr >> 3) == half) {
#pragma unroll
            for (int jp = 0; jp < NF / 2; ++jp)
              *reinterpret_cast<u32x4*>(stg + (elr & 7) * 256 + (((4 * jp + elg) ^ (elr & 7)) << 4)) = w[jp];
          }
          asm volatile("" ::: "memory");
        }
        if (k > 0) {
          const int kp = k - 1;
#pragma unroll
          for (int sr = 0; sr < 2; ++sr) {
            // non-temporal: y (N*k rows, 268 MB at T=16384) is larger than
            // the MALL and read once by the combine (non-temporal loads as
            // well); kept out of it, it no longer evicts act, x and the
            // weights, which this and the next layer step read again
            if (8 * kp + 4 * sr + lrow < n_ok)
              __builtin_nontemporal_store(
                  d[sr], reinterpret_cast<__attribute__((address_space(1))) u32x4*>(
                             ybase + static_cast<uint64_t>(static_cast<uint32_t>(cell[sr])) * ystride + lchunk * 16));
          }
          asm volatile("" ::: "memory");
        }
        if (k < NR) {
#pragma unroll
          for (int sr = 0; sr < 2; ++sr) {
            const int rr = 4 * sr + lrow;                                  // row of the slice
            d[sr] = *reinterpret_cast<const u32x4*>(stg + rr * 256 + ((lchunk ^ rr) << 4));
            cell[sr] = rmap[8 * k + 4 * sr];
          }
          asm volatile("" ::: "memory");
        }
      }
    }
  };

  // ---- persistent tile loop ---------------------------------------------------------
  // Rounds: a workgroup takes one or two items from a queue (its own first;
  // once that is drained, the next queue with items left) and runs the
  // pipelined tile loop over that queue's items, claiming the next ones as
  // it goes (see the claims below), until the queue runs dry.
  std::integral_constant<int, 0> S0;
  std::integral_constant<int, 1> S1;
  std::integral_constant<bool, false> NO;
  std::integral_constant<bool, true> YES;
  int n_done = 0;
  int sig_r = -1;                                  // row tile of a GEMM-1 tile not yet counted
  int cq = q;                                      // the queue of the items in hand
  bool first_round = true;
  for (;;) {
    // every wave waited for its stores (vmcnt(0)) before leaving the tile
    // loop: count the last GEMM-1 tile, then take two items
    __syncthreads();
    if (tid == 0) {
      if (BOTH && sig_r >= 0) atomic_add_1(sched + sched::row_word(sig_r), 1);
      int a = INT_MAX, b = INT_MAX, qq = cq;
      bool claimed = false;
      if (first_round) {
        // the fixed first item, and a second one as below; without one
        // (n_static > n) the queue has nothing left to claim
        const int n = q_items(q);
        qq = q;
        if (first_pos < n) {
          a = first_pos;
          const bool g2 = MODE == kModeDown || (BOTH && a >= (q_lo(q + 1) - q_lo(q)) * n1);
          if (!g2) {
            b = claim(q);
            if (b >= n) atomic_or_1(sched + sched::kDrained, 1 << q);
          }
          claimed = true;
        } else {
          atomic_or_1(sched + sched::kDrained, 1 << q);
        }
      }
      const int drained = claimed ? 0 : atomic_read(sched + sched::kDrained);
      for (int v = 0; v < nq && !claimed; ++v) {
        qq = (cq + v) & (nq - 1);
        if ((drained >> qq) & 1) continue;
        const int n = q_items(qq);
        a = claim(qq);
        if (a < n) {
          // a second item only while this one is a GEMM-1 tile (see the claims below)
          const bool g2 = MODE == kModeDown || (BOTH && a >= (q_lo(qq + 1) - q_lo(qq)) * n1);
          if (!g2) {
            b = claim(qq);
            if (b >= n) atomic_or_1(sched + sched::kDrained, 1 << qq);
          }
          break;
        }
        atomic_or_1(sched + sched::kDrained, 1 << qq);
        a = INT_MAX;
      }
      s_msg[0] = a;
      s_msg[1] = b;
      s_msg[3] = qq;
    }
    sig_r = -1;
    first_round = false;
    __syncthreads();
    const int i0 = __builtin_amdgcn_readfirstlane(s_msg[0]), i1 = __builtin_amdgcn_readfirstlane(s_msg[1]);
    cq = __builtin_amdgcn_readfirstlane(s_msg[3]);
    const int n_items = q_items(cq);
    if (i0 >= n_items) break;                      // every queue is drained

    Tile cur = decode(i0, cq);
    bool has_next = i1 < n_items;
    Tile nxt = has_next ? decode(i1, cq) : cur;
    // the weight waves load their first two stages at once (weight rows need
    // neither the row map nor GEMM-1's rows); the A waves after the row map
    // has landed (and, for a GEMM-2 tile, its rows are done)
    Src sc;
    if (!wave_a) {
      sc = setup(cur, 0);
#pragma unroll
      for (int i = 0; i < BPW; ++i) dma_blk(sc, 0, 0, i);
#pragma unroll
      for (int i = 0; i < BPW; ++i) dma_blk(sc, 1, 1, i);
    }
    if (tid == 0) s_msg[4] = (BOTH && !cur.g1) ? wait_rows(cur.R) : 0;
    rowmap_dma(cur, 0);
    if (has_next) rowmap_dma(nxt, 1);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    int poison = __builtin_amdgcn_readfirstlane(s_msg[4]);   // cur's wait gave up
    if (wave_a) {
      sc = setup(cur, 0);
#pragma unroll
      for (int i = 0; i < BPW; ++i) dma_blk(sc, 0, 0, i);
#pragma unroll
      for (int i = 0; i < BPW; ++i) dma_blk(sc, 1, 1, i);
    }
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    lds_barrier();

    // Invariant at a tile's start: its stages 0 and 1 are in buffers 0 and 1
    // (landed, published).  Steps are unrolled by four (two stages), so every
    // buffer index is an immediate.
    bool open = true;                              // no claim on queue cq has come back empty yet
    for (int it = 0;; ++it) {
      const bool act = wm < cur.act_wm;
      const int KT = (cur.g1 ? p.H : p.I) / KS;     // MFMA steps of this tile
      // Claims, at step KT-8 (step 0 in tiles too short for that): while the
      // next tile is a GEMM-1 tile, the one after it (a GEMM-1 tile's row map
      // must be in LDS before the tile in front of it prefetches its first
      // stages); with no next tile, the next one itself, decoded at step
      // KT-4 (a GEMM-2 tile needs its row map only in its epilogue).  A
      // workgroup thus holds at most one unstarted GEMM-2 tile when the queues
      // run dry.
      const bool early = KT - 8 < 4;
      const bool ahead2 = open && has_next && nxt.g1;
      const bool ahead1 = open && !has_next;
      // a GEMM-2 tile next: poll its row tile's counter at steps KT-8 .. KT-6
      // (at step 0 for short tiles), read it at step KT-4
      const bool poll = BOTH && has_next && !nxt.g1;
      if (act) first_frags();
      step(S0, YES, NO, YES, sc, 0, 0, 0, act);          // step 0 (stage 0)
      // every wave is past its previous epilogue (barrier above), so the row
      // map buffer that epilogue read can take the next tile's row map; the
      // wait at the end of step 2 covers it, setup() reads it at step KT-3
      if (it > 0 && has_next) rowmap_dma(nxt, (it + 1) & 1);
      // every wave waited for its stores (vmcnt(0)) before the barrier that
      // ended step 0: the previous GEMM-1 tile's act rows are complete
      if (BOTH && tid == 0 && sig_r >= 0) atomic_add_1(sched + sched::row_word(sig_r), 1);
      sig_r = -1;
      int got = INT_MAX, dep = 0;
      if (tid == 0 && early) {
        if (ahead2 || ahead1) got = claim(cq);
        if (poll) dep = load_dev_i32(sched + sched::row_word(nxt.R));
      }
      step(S1, NO, YES, YES, sc, 2, 0, 1, act);          // step 1: DMA stage 2 -> buffer 0
      step(S0, NO, NO, YES, sc, 0, 0, 1, act);           // step 2 (stage 1)
      if (tid == 0 && early) {
        s_msg[0] = got;
        s_msg[2] = dep;
      }
      step(S1, NO, YES, YES, sc, 3, 1, 0, act);          // step 3: DMA stage 3 -> buffer 1
      // steady state: steps k4 .. k4+3 (stages k4/2, k4/2 + 1) DMA stages k4/2 + 2, + 3
      for (int k4 = 4; k4 < KT - 4; k4 += 4) {
        const bool late = k4 == KT - 8;
        if (tid == 0 && late) {
          if (ahead2 || ahead1) got = claim(cq);
          if (poll) dep = load_dev_i32(sched + sched::row_word(nxt.R));
        }
        step(S0, NO, NO, YES, sc, 0, 0, 0, act);
        // the claim came back before the barrier of step KT-8: a GEMM-2 tile
        // claimed for next polls its row tile (the row tile is arithmetic)
        if (BOTH && tid == 0 && late && ahead1) {
          const int nr = q_lo(cq + 1) - q_lo(cq);
          if (got < n_items && got >= nr * n1) dep = load_dev_i32(sched + sched::row_word(q_lo(cq) + (got - nr * n1) / n2));
        }
        step(S1, NO, YES, YES, sc, k4 / 2 + 2, 0, 1, act);
        step(S0, NO, NO, YES, sc, 0, 0, 1, act);
        if (tid == 0 && late) {
          s_msg[0] = got;
          s_msg[2] = dep;
        }
        step(S1, NO, YES, YES, sc, k4 / 2 + 3, 1, 0, act);
      }
      // last two stages: their odd steps DMA the next tile's stages 0 and 1.
      // Without a next tile, or with one whose first stages cannot stream in
      // yet (a GEMM-2 tile whose rows are not ready, a GEMM-1 tile claimed
      // without its row map), they re-read this tile's (in bounds, never
      // consumed) so the code has no branch here.
      step(S0, NO, NO, YES, sc, 0, 0, 0, act);           // step KT-4
      bool ready;
      if (ahead1) {
        const int g = __builtin_amdgcn_readfirstlane(s_msg[0]);
        ready = false;
        if (g < n_items) {
          nxt = decode(g, cq);
          has_next = true;
          ready = !nxt.g1 && (!BOTH || (!early && __builtin_amdgcn_readfirstlane(s_msg[2]) >= need(nxt.R)));
          if (ready) rowmap_dma(nxt, (it + 1) & 1);     // read by its epilogue, many barriers on
        } else {
          open = false;
          if (tid == 0) atomic_or_1(sched + sched::kDrained, 1 << cq);
        }
      } else {
        ready = has_next && (!poll || __builtin_amdgcn_readfirstlane(s_msg[2]) >= need(nxt.R));
      }
      sc = ready ? setup(nxt, (it + 1) & 1) : setup(cur, it & 1);
      step(S1, NO, YES, YES, sc, 0, 0, 1, act);          // step KT-3: next stage 0 -> buffer 0
      step(S0, NO, NO, YES, sc, 0, 0, 1, act);           // step KT-2
      step(S1, NO, YES, NO, sc, 1, 1, 0, act);           // step KT-1: next stage 1 -> buffer 1
      epilogue(cur, it & 1, poison);
      ++n_done;
      if (BOTH && cur.g1) sig_r = cur.R;
      if (!has_next) {
        // no DMA may still be writing this workgroup's LDS when its waves end
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        break;
      }
      cur = nxt;
      poison = 0;
      has_next = false;
      if (ahead2) {
        const int g = __builtin_amdgcn_readfirstlane(s_msg[0]);
        has_next = g < n_items;
        if (has_next) {
          nxt = decode(g, cq);
        } else {
          open = false;
          if (tid == 0) atomic_or_1(sched + sched::kDrained, 1 << cq);
        }
      }
      if (!ready) {
        // cur's first stages did not stream in: count the tile just
        // finished, wait between tiles for cur's rows if it is a GEMM-2
        // tile, then load its row map and first stages
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __syncthreads();
        if (tid == 0) {
          if (BOTH && sig_r >= 0) atomic_add_1(sched + sched::row_word(sig_r), 1);
          s_msg[4] = (BOTH && !cur.g1) ? wait_rows(cur.R) : 0;
        }
        sig_r = -1;
        rowmap_dma(cur, (it + 1) & 1);
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __syncthreads();
        poison = __builtin_amdgcn_readfirstlane(s_msg[4]);
        sc = setup(cur, (it + 1) & 1);
#pragma unroll
        for (int i = 0; i < BPW; ++i) dma_blk(sc, 0, 0, i);
#pragma unroll
        for (int i = 0; i < BPW; ++i) dma_blk(sc, 1, 1, i);
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        lds_barrier();
      }
    }
  }
  // Count this workgroup's items, then arrive; the count is complete
  // (vmcnt(0)) before the arrival, so the last workgroup to arrive sees every
  // count.  It checks that every queue was drained and returns every word it
  // used to zero for the next launch.
  if (tid == 0) {
    atomic_add_1(sched + sched::kItems, n_done);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    s_msg[3] = atomic_add_1(sched + sched::kDone, 1);
  }
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(s_msg[3]) == static_cast<int>(gridDim.x) - 1) {
    if (tid == 0) {
      if (atomic_read(sched + sched::kItems) != RT * per_row) atomic_or_1(sched + sched::kFlags, sched::kFlagDrain);
      for (int j = 0; j < 8; ++j) atomicExch(sched + sched::queue_word(j), 0);
      atomicExch(sched + sched::kItems, 0);
      atomicExch(sched + sched::kDrained, 0);
      atomicExch(sched + sched::kDone, 0);
    }
    if (BOTH)
      for (int r = tid; r < RT; r += NT) atomicExch(sched + sched::row_word(r), 0);
  }
}

// ============================================================================
// bf16 path for few rows per expert (decode, small batches): one workgroup
// per (chunk of at most 32 rows of one local expert, column block), 4 waves,
// each wave two 16-column weight fragments (GEMM-1: 16 gate + the matching 16
// up columns; GEMM-2: 32 output columns) against the chunk's two row
// fragments.  There the time goes to streaming the weights from HBM, so each
// wave keeps DEPTH K-steps of weight and row fragments in flight, straight
// from global memory into VGPRs (no barriers), and an expert with no rows has
// no chunk, so its weights are never read.  K is walked in exactly
// the main kernel's order (GEMM-2: its column tile's rotation of the K stages; the
// same MFMA with the weight fragment as src0), so every output element gets
// the same fp32 accumulation sequence and the same bits as from
// moe_gemm_bf16_kernel, whichever kernel the launch size selects.
namespace skinny {
constexpr int NW = 4, NT = NW * 64;
constexpr int MFC = 2;                        // row fragments per pass (32 rows)
constexpr int DEPTH = 8;                      // K-steps of loads in flight
// GEMM-2 of the fused launch: weight K-steps DEPTH .. DEPTH + LSTEPS - 1 of
// each wave go to LDS before the wait (1 KiB per step and fragment: 64 KiB
// per workgroup, so two workgroups fit on a CU)
constexpr int LSTEPS = 8;
// fused launch: GEMM-2's workgroups start streaming their weights once every
// GEMM-1 workgroup of the chunk is this many blocks of DEPTH steps from the
// end of its K loop
constexpr int SIG_BLOCKS = 2;
constexpr int LDS_W = NW * LSTEPS * 2 * 1024;
// use this path when N * k is at most this (measured crossover against the
// tiled kernel: GEMM-1 between 1024 and 2048 entries, GEMM-2 past 2048)
constexpr int64_t kMaxEntries1 = 1024, kMaxEntries2 = 2048;
static_assert(kMaxEntries1 == sched::kSmallRows, "schedule words of the small-batch launch");
static_assert(LSTEPS == DEPTH, "the K loop's first block reads all the LDS steps");

// The K loop of a small-batch workgroup with DEPTH K-steps of loads in
// flight (KT steps, a multiple of DEPTH; the caller has loaded block 0):
// block b of DEPTH steps runs its MFMAs and issues block b + 1's loads --
// block 1's with `first` (from LDS where the caller staged them), the later
// ones with `next` -- and the last block runs only its MFMAs.  No load sits
// under a run-time condition inside a block: the compiler then counts the
// loads in flight exactly and each step waits only for its own operands.  (A
// conditional load makes it wait for every load in flight at the end of each
// block, and the pipeline drains every DEPTH steps: the loop then runs at
// one memory latency per block.)  Block 1 is peeled too, so that the loop
// is entered with the loads in flight that it has at every iteration and
// its waits are the steady state's.  at_block(b) runs before block b.
template <class Mfma, class First, class Next, class AtBlock>
__device__ __forceinline__ void k_pipeline(int KT, Mfma mfma, First first, Next next, AtBlock at_block) {
  const int NB = KT / DEPTH;
  auto block = [&](int b, auto load) {
    at_block(b);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      mfma(d);
      load((b + 1) * DEPTH + d, d);
    }
  };
  if (NB > 1) {
    block(0, first);
    if (NB > 2) {
      block(1, next);
      for (int b = 2; b < NB - 1; ++b) block(b, next);
    }
  }
  at_block(NB - 1);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) mfma(d);
}
}  // namespace skinny

// The combine that ends a small-batch launch (moe_gemm_skinny_both_kernel
// with COMB): top-8, bf16, the (token, slot) layout of y_entries.
struct CombineParams {
  const uint16_t* gate;            // (n_tokens, 8)
  const int32_t* row_of_entry;     // (n_tokens * 8), -1: cell not computed
  const uint8_t* valid;            // (n_tokens,) or NULL
  uint16_t* out;                   // (n_tokens, hidden)
  int64_t n_tokens;
  int hidden;
  int n_g2, n_comb;                // GEMM-2 and combine workgroups of the launch
  uint32_t y_bytes;                // bytes of y_entries (< 4 GiB)
  int wait_limit;                  // polls before a combine workgroup's wait gives up
  int dbg_comb;                    // combine workgroup that waits for one more (test hook; -1: none)
};

// One workgroup's share of a small-batch GEMM: a (chunk, column block) pair
// (the mapping is below).  FUSED (both GEMMs in one launch, GEMM-1's
// workgroups first in the grid): each GEMM-1 workgroup adds one to its
// chunk's counter in `sched` twice, when it is SIG_BLOCKS blocks of DEPTH
// steps from the end of its K loop (most of its weights are in) and when its
// act stores (device scope) are complete.  A GEMM-2 workgroup reads its
// destination cells, waits (thread 0, bounded) until the chunk's count
// reaches the number of GEMM-1 column blocks (normally their first counts; a
// mix of first and second counts meets it too, harmlessly: this wait only
// orders the weight streams), then loads its first DEPTH weight steps into
// registers and the next LSTEPS into LDS (`s_w`: each lane fetches exactly
// the 16 bytes it later feeds the MFMA, so a step's fragment is read back at
// byte 16 * lane of its 1 KiB block), waits until the count is twice the
// column blocks (each adds exactly two, so every act store of the chunk is
// complete), and only then loads act's rows.  GEMM-1's weights thus stream first, with the whole
// memory bandwidth (measured on the 32-token decode layer: GEMM-1's K loops
// end at 13.4 us instead of 16.3 us with both weight streams overlapping, the
// launch takes 22.4-22.8 us instead of 25.9 us; counting at the last block
// instead of two before the end: 23.5 us, three before: 23.3 us).  The
// workgroups are dispatched in grid order, so every GEMM-1 workgroup is
// resident before any GEMM-2 workgroup can wait, GEMM-1 never waits, and
// every wait ends.  The last GEMM-2 workgroup of a chunk to pass the second
// wait takes the chunk's counts back out (the amounts every workgroup adds),
// so they return to zero once every workgroup has finished, in any order.
// A wait gives up after p.wait_limit polls: the wait flag is set and the
// workgroup stores NaN.
// COMB (GEMM-2 of a launch that ends with the combine): y is stored with
// device scope, and every GEMM-2 workgroup, with rows or without, counts
// itself done in `sched` once its stores are complete.
template <bool GEMM1, bool FUSED, bool COMB = false>
__device__ __forceinline__ void skinny_body(const GemmParams& p, int block, int n_cb_other, int* sched,
                                            int* s_pre, int* s_off, unsigned char* s_w, int* s_gave) {
  static_assert(!COMB || (FUSED && !GEMM1), "the combine follows the fused launch's GEMM-2");
  using namespace skinny;
  typedef uint16_t T;
  constexpr int CH = 16 * MFC;                                // rows per workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = p.n_local;
  // offsets[nl] < 0: the dispatch gave up (its outputs are poisoned); then no
  // expert has rows and the call is flagged
  {
    const int last = p.offsets[nl];
    for (int j = tid; j <= nl; j += NT) s_off[j] = last < 0 ? 0 : p.offsets[j];
    if (last < 0 && block == 0 && tid == 0 && p.flags != nullptr) atomic_or_1(p.flags, sched::kFlagInput);
  }
  // chunk table: expert j owns ceil(rows_j / CH) chunks of CH rows.  The
  // grid (sized for the worst case, a multiple of 8 chunks; workgroups past
  // the last chunk return) runs chunk q's column blocks on workgroups
  // b == q (mod 8): workgroups are dispatched to the 8 XCDs round robin, so a
  // chunk's A rows are fetched into one XCD's L2 and shared there by all its
  // column blocks (and in the fused launch GEMM-2 finds act where GEMM-1 of
  // the same chunk wrote it)
  __syncthreads();
  if (tid < 64) scan_units<CH>(s_off, s_pre, nl, 1);
  __syncthreads();
  const int n_cb = GEMM1 ? p.N / 64 : p.N / 128;             // column blocks per expert
  const int q = (block >> 3) / n_cb * 8 + (block & 7), cb = (block >> 3) % n_cb;
  const int n_chunks = s_pre[nl];
  if (q >= n_chunks) {
    if (COMB && tid == 0) atomic_add_1(sched + sched::kG2Done, 1);
    return;
  }
  int lo = 0, hi = nl - 1;                                    // largest j with s_pre[j] <= q
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pre[mid] <= q) lo = mid; else hi = mid - 1;
  }
  const int e = __builtin_amdgcn_readfirstlane(lo);
  const int row_lo = __builtin_amdgcn_readfirstlane(s_off[e] + (q - s_pre[e]) * CH);
  const int row_hi = __builtin_amdgcn_readfirstlane(min(s_off[e + 1], row_lo + CH));
  const int lr = lane & 15, lg = lane >> 4;
  const int K = p.K, KT = K / 32, KD = K / 64;
  // the main kernel's column tile of this block and its K rotation (in steps)
  const int nt = cb / 2;
  const int rot = (!GEMM1 && KD % 4 == 0) ? 2 * (nt & 3) * (KD / 4) : 0;
  // weight rows of this wave's two fragments
  const int slot = p.w_slot != nullptr ? p.w_slot[e] : e;
  const T* W = static_cast<const T*>(p.W) + static_cast<int64_t>(slot) * p.w_expert_stride;
  int wrow[2];
  if constexpr (GEMM1) {
    const int g0 = cb * 64 + wave * 16;
    wrow[0] = g0 + lr;                       // gate column
    wrow[1] = p.N + g0 + lr;                 // its up column
  } else {
    const int c0 = cb * 128 + wave * 32;
    wrow[0] = c0 + lr;
    wrow[1] = c0 + 16 + lr;
  }
  const T* wp0 = W + static_cast<int64_t>(wrow[0]) * K + 8 * lg;
  const T* wp1 = W + static_cast<int64_t>(wrow[1]) * K + 8 * lg;
  const T* A = static_cast<const T*>(p.A);
  T* const C = static_cast<T*>(p.C);
  // chunk counters of the fused launch: GEMM-1 workgroups done, GEMM-2 workgroups past the wait
  int* const done1 = FUSED ? sched + sched::row_word(q) : nullptr;
  int* const seen2 = FUSED ? done1 + 1 : nullptr;

  {
    const int r0 = row_lo;
    u32x4 wq[DEPTH][2], aq[DEPTH][MFC];
    auto k_off = [&](int t) {
      int ks = t + rot;
      if (ks >= KT) ks -= KT;
      return static_cast<int64_t>(ks) * 32;
    };
    // steps held in LDS (fused GEMM-2 only): [DEPTH, DEPTH + n_lds)
    constexpr bool LDS_STEPS = FUSED && !GEMM1;
    const int n_lds = LDS_STEPS ? min(LSTEPS, KT - DEPTH) : 0;
    unsigned char* const w_lds = LDS_STEPS ? s_w + wave * (LSTEPS * 2 * 1024) : nullptr;
    auto load_w = [&](int t, int slot) {
      const int64_t off = k_off(t);
      wq[slot][0] = *reinterpret_cast<const u32x4*>(wp0 + off);
      wq[slot][1] = *reinterpret_cast<const u32x4*>(wp1 + off);
    };
    auto load_w_lds = [&](int t, int slot) {             // a step staged in LDS: [DEPTH, DEPTH + n_lds)
      const unsigned char* b = w_lds + (t - DEPTH) * 2048 + 16 * lane;
      wq[slot][0] = *reinterpret_cast<const u32x4*>(b);
      wq[slot][1] = *reinterpret_cast<const u32x4*>(b + 1024);
    };
    if constexpr (!LDS_STEPS) {
      // the weights need only the chunk's expert: their first steps go out
      // before the row map is read
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) load_w(d, d);
    }
    // GEMM-2's destination cells, read now rather than after the K loop
    // (in the fused launch the read overlaps the wait for GEMM-1)
    int cell[MFC];
    if constexpr (!GEMM1) {
#pragma unroll
      for (int f = 0; f < MFC; ++f) cell[f] = p.perm[min(r0 + 16 * f + lr, row_hi - 1)];
    }
    // thread 0: until the chunk's counter reaches `target` (one more for the
    // test hook's chunk); a give-up sets the wait flag and *s_gave.  Polled
    // with read-modify-writes: polled with device-scope loads (here and in
    // the combine's wait below) the two-launch decode layer took 38.6 us
    // instead of 33.6 (same box, alternating builds)
    auto wait_count = [&](int target) {
      if (q == p.dbg_chunk) ++target;
      int polls = 0;
      while (atomic_read(done1) < target) {
        if (++polls == p.wait_limit) {
          atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
          *s_gave = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    };
    if constexpr (LDS_STEPS) {
      // GEMM-1 streams its weights first: every GEMM-1 workgroup of the
      // chunk counts once SIG_BLOCKS blocks before the end of its K loop, so
      // GEMM-2's weights do not take memory bandwidth from GEMM-1's until
      // then (the chunk's act is ready when the count is twice the blocks)
      if (tid == 0) {
        *s_gave = 0;
        wait_count(n_cb_other);
      }
      __syncthreads();
      // the weights do not depend on GEMM-1's results: their first DEPTH
      // steps go to registers and the next n_lds steps to LDS before the wait
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) load_w(d, d);
      const unsigned char* wb = reinterpret_cast<const unsigned char*>(W);
      const int wbytes = static_cast<int>(p.w_expert_stride * 2);
      const uint32_t lo0 = static_cast<uint32_t>((wp0 - W) * 2), lo1 = static_cast<uint32_t>((wp1 - W) * 2);
      for (int t = DEPTH; t < DEPTH + n_lds; ++t) {
        const uint32_t ko = static_cast<uint32_t>(k_off(t) * 2);
        buffer_lds_16(wb, wbytes, lo0 + ko, 0, w_lds + (t - DEPTH) * 2048);
        buffer_lds_16(wb, wbytes, lo1 + ko, 0, w_lds + (t - DEPTH) * 2048 + 1024);
      }
      if (tid == 0) {
        wait_count(2 * n_cb_other);
        // the last GEMM-2 workgroup of the chunk past its wait takes out what
        // every workgroup adds (GEMM-1: two counts each; GEMM-2: one), so a
        // count that arrives after a give-up still leaves both at zero
        if (atomic_add_1(seen2, 1) == n_cb - 1) {
          atomic_add_1(done1, -2 * n_cb_other);
          atomic_add_1(seen2, -n_cb);
        }
      }
      // this wave's LDS steps have landed (its own lanes read them back)
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      __syncthreads();
    }
    // A rows of the pass (rows past row_hi read the last row; never stored)
    const T* ap[MFC];
#pragma unroll
    for (int f = 0; f < MFC; ++f) {
      const int r = min(r0 + 16 * f + lr, row_hi - 1);
      int64_t src;
      if constexpr (GEMM1) src = p.perm[r] / p.top_k;      // token row of x
      else src = r;                                        // act row
      ap[f] = A + src * K + 8 * lg;
    }
    auto load_a = [&](int t, int slot) {
      const int64_t off = k_off(t);
#pragma unroll
      for (int f = 0; f < MFC; ++f) aq[slot][f] = *reinterpret_cast<const u32x4*>(ap[f] + off);
    };
    // accumulators start at +0.0, which is what the main kernel's first MFMA
    // adds (C operand 0), so the sums are the same bit for bit
    f32x4 acc[MFC][2];
#pragma unroll
    for (int f = 0; f < MFC; ++f)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[f][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_a(d, d);
    auto mfma_step = [&](int d) {
#pragma unroll
      for (int f = 0; f < MFC; ++f)
#pragma unroll
        for (int j = 0; j < 2; ++j) mfma_acc(acc[f][j], wq[d][j], aq[d][f]);
    };
    auto next = [&](int t, int slot) {
      load_w(t, slot);
      load_a(t, slot);
    };
    auto first = [&](int t, int slot) {
      if constexpr (LDS_STEPS) load_w_lds(t, slot);
      else load_w(t, slot);
      load_a(t, slot);
    };
    // fused GEMM-1: the first count of the chunk, SIG_BLOCKS blocks of DEPTH
    // steps before the end of the K loop (at its start when shorter)
    const int nb = KT / DEPTH, b_sig = nb > SIG_BLOCKS ? nb - SIG_BLOCKS : 0;
    auto at_block = [&](int b) {
      if (FUSED && GEMM1 && b == b_sig && tid == 0) atomic_add_1(done1, 1);
    };
    k_pipeline(KT, mfma_step, first, next, at_block);
    // results: lane (lr, lg) of fragment j holds columns 4 lg .. 4 lg + 3 of
    // the fragment for row lr of each row fragment
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int f = 0; f < MFC; ++f)
#pragma unroll
      for (int j = 0; j < 2; ++j) pin_acc(acc[f][j]);
    // a fused GEMM-2 workgroup whose wait for act gave up stores NaN
    if constexpr (LDS_STEPS) {
      if (__builtin_amdgcn_readfirstlane(*s_gave)) {
        const float nan = __builtin_nanf("");
#pragma unroll
        for (int f = 0; f < MFC; ++f)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[f][j] = f32x4{nan, nan, nan, nan};
      }
    }
#pragma unroll
    for (int f = 0; f < MFC; ++f) {
      const int r = r0 + 16 * f + lr;
      if (r >= row_hi) continue;
      if constexpr (GEMM1) {
        const int col = cb * 64 + wave * 16 + 4 * lg;
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
          w[h] = pack_bf16x2(silu_f(acc[f][0][2 * h]) * acc[f][1][2 * h],
                             silu_f(acc[f][0][2 * h + 1]) * acc[f][1][2 * h + 1]);
        uint64_t* const dst = reinterpret_cast<uint64_t*>(C + static_cast<int64_t>(r) * p.N + col);
        const uint64_t v = (static_cast<uint64_t>(w[1]) << 32) | w[0];
        // fused: device scope, so GEMM-2 on any XCD reads the final rows
        if constexpr (FUSED) __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else *dst = v;
      } else {
        const int64_t row = cell[f];                       // (token, slot) cell
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = cb * 128 + wave * 32 + 16 * j + 4 * lg;
          const uint2 w = make_uint2(pack_bf16x2(acc[f][j][0], acc[f][j][1]), pack_bf16x2(acc[f][j][2], acc[f][j][3]));
          if constexpr (COMB)   // device scope: the combine may run on another XCD
            __hip_atomic_store(reinterpret_cast<uint64_t*>(C + row * p.N + col),
                               (static_cast<uint64_t>(w.y) << 32) | w.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            *reinterpret_cast<uint2*>(C + row * p.N + col) = w;
        }
      }
    }
  }
  if constexpr (FUSED && GEMM1) {
    // every wave's act stores are complete before the chunk's count goes up
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    if (tid == 0) atomic_add_1(done1, 1);
  }
  if constexpr (COMB) {
    // every wave's y stores are complete before the count goes up
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    if (tid == 0) atomic_add_1(sched + sched::kG2Done, 1);
  }
}

// Combine workgroup `cb` of a launch that ends with the combine: thread 0
// waits (bounded) until every GEMM-2 workgroup has counted its y stores
// complete; the last combine workgroup past the wait returns both counters
// to zero.  Then each thread sums one 16-byte chunk of a token's output row
// (combine8_chunk: the order of combine8_kernel, so the same bits), reading y
// with device-scope loads.
__device__ void skinny_combine(const CombineParams& cp, const uint16_t* y, int cb, int* sched, int* s_gave) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    int polls = 0, gave = 0;
    const int target = cp.n_g2 + (cb == cp.dbg_comb ? 1 : 0);
    while (atomic_read(sched + sched::kG2Done) < target) {
      if (++polls == cp.wait_limit) {
        atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
        gave = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    *s_gave = gave;
    // the last combine workgroup past its wait takes out what every
    // workgroup adds, so a GEMM-2 count that arrives after a give-up still
    // leaves both words at zero
    if (atomic_add_1(sched + sched::kCombDone, 1) == cp.n_comb - 1) {
      atomic_add_1(sched + sched::kG2Done, -cp.n_g2);
      atomic_add_1(sched + sched::kCombDone, -cp.n_comb);
    }
  }
  __syncthreads();
  const int cpr = cp.hidden / 8;                              // 16-byte chunks per row
  const uint32_t q = static_cast<uint32_t>(cb) * skinny::NT + tid;
  const int64_t t = q / static_cast<uint32_t>(cpr);
  const int c = static_cast<int>(q - static_cast<uint32_t>(t) * cpr);
  if (t >= cp.n_tokens) return;
  if (__builtin_amdgcn_readfirstlane(*s_gave)) {             // the wait gave up: NaN outputs
    const uint32_t nan2 = pack_bf16x2(__builtin_nanf(""), __builtin_nanf(""));
    *reinterpret_cast<u32x4*>(cp.out + t * cp.hidden + c * 8) = u32x4{nan2, nan2, nan2, nan2};
    return;
  }
  combine8_chunk<MEP_DTYPE_BF16>(y, cp.gate, cp.row_of_entry, cp.valid, t, c, cp.hidden, cp.out,
                                 [&](const uint16_t* ptr) {
                                   return load_dev_16(y, cp.y_bytes, static_cast<uint32_t>((ptr - y) * 2));
                                 });
}

template <bool GEMM1>
__global__ __launch_bounds__(skinny::NT) void moe_gemm_skinny_kernel(GemmParams p) {
  __shared__ int s_pre[bfk::NLMAX + 1];                       // chunks before expert j
  __shared__ int s_off[bfk::NLMAX + 1];
  skinny_body<GEMM1, false>(p, blockIdx.x, 0, nullptr, s_pre, s_off, nullptr, nullptr);
}

// Both small-batch GEMMs in one launch: workgroups [0, g1_blocks) are GEMM-1's,
// the rest GEMM-2's (see skinny_body); with COMB the last cp.n_comb
// workgroups then combine the tokens' rows (skinny_combine).  Workgroups are
// dispatched in grid order, so every workgroup a combine workgroup waits for
// is resident or done before it is.
template <bool COMB>
__global__ __launch_bounds__(skinny::NT) void moe_gemm_skinny_both_kernel(GemmParams p1, GemmParams p2,
                                                                          int g1_blocks, int* sched,
                                                                          CombineParams cp) {
  __shared__ int s_pre[bfk::NLMAX + 1];
  __shared__ int s_off[bfk::NLMAX + 1];
  __shared__ __attribute__((aligned(16))) unsigned char s_w[skinny::LDS_W];
  __shared__ int s_gave;                                      // a wait of this workgroup gave up
  const int b = blockIdx.x;
  if (b < g1_blocks) skinny_body<true, true>(p1, b, p2.N / 128, sched, s_pre, s_off, s_w, &s_gave);
  else if (!COMB || b < g1_blocks + cp.n_g2)
    skinny_body<false, true, COMB>(p2, b - g1_blocks, p1.N / 64, sched, s_pre, s_off, s_w, &s_gave);
  else skinny_combine(cp, static_cast<const uint16_t*>(p2.C), b - g1_blocks - cp.n_g2, sched, &s_gave);
}

// chunks of the small-batch grids: the worst case (each expert adds at most
// one partial chunk), rounded up to a multiple of 8 (one per XCD, see
// skinny_body), so GEMM-1's block count is a multiple of 8 as well
inline int64_t skinny_chunks(int64_t max_rows, int n_local) {
  const int64_t c = (max_rows + 16 * skinny::MFC - 1) / (16 * skinny::MFC) + n_local;
  return (c + 7) / 8 * 8;
}

template <bool GEMM1>
hipError_t launch_skinny(const GemmParams& p, int64_t max_rows, hipStream_t stream) {
  // few rows per expert: stream each expert's weights once (same results)
  const int n_cb = GEMM1 ? p.N / 64 : p.N / 128;
  const int64_t chunks = skinny_chunks(max_rows, p.n_local);
  const int64_t blocks = chunks * n_cb;
  if (blocks == 0) return hipSuccess;
  moe_gemm_skinny_kernel<GEMM1><<<dim3(static_cast<unsigned>(blocks)), skinny::NT, 0, stream>>>(p);
  return hipGetLastError();
}

// comb: NULL, or the combine that ends the launch (its n_g2 / n_comb are set here)
hipError_t launch_skinny_both(const GemmParams& p1, const GemmParams& p2, int64_t max_rows, int* sched,
                              const CombineParams* comb, hipStream_t stream) {
  const int64_t chunks = skinny_chunks(max_rows, p1.n_local);
  const int64_t b1 = chunks * (p1.N / 64), b2 = chunks * (p2.N / 128);
  if (b1 + b2 == 0) return hipSuccess;
  if (comb == nullptr) {
    moe_gemm_skinny_both_kernel<false><<<dim3(static_cast<unsigned>(b1 + b2)), skinny::NT, 0, stream>>>(
        p1, p2, static_cast<int>(b1), sched, CombineParams{});
  } else {
    CombineParams cp = *comb;
    cp.n_g2 = static_cast<int>(b2);
    cp.n_comb = static_cast<int>((cp.n_tokens * (cp.hidden / 8) + skinny::NT - 1) / skinny::NT);
    moe_gemm_skinny_both_kernel<true><<<dim3(static_cast<unsigned>(b1 + b2 + cp.n_comb)), skinny::NT, 0, stream>>>(
        p1, p2, static_cast<int>(b1), sched, cp);
  }
  return hipGetLastError();
}

// ============================================================================
// The decode layer in one launch (mep_moe_layer): router + dispatch, GEMM-1 +
// SwiGLU, GEMM-2 and the combine, for bf16, 32 experts, top-8 and at most 32
// tokens (every expert then has at most one 32-row chunk).
//
// Workgroup 0 routes the batch (router + one-block dispatch, the same
// instructions as mep_route_dispatch's one-workgroup path, so the same bits),
// stores everything, writes its XCD's L2 back to memory (release at device
// scope) and then publishes one routing record per expert: a 64-bit word
// (written once, so read whole) holding a written bit, the expert's first
// row and its tokens as a bit mask.  Workgroups are dispatched in grid
// order, so it is resident before anyone waits for it.  The GEMM workgroups
// that follow are expert-major: (expert e, column block cb), all column
// blocks of expert e on XCD (e + 1) mod 8 for both GEMMs (act stays in one
// L2).  GEMM-1 does not wait for the routing: a batch has at most 32 tokens,
// one MFMA row block, so each GEMM-1 workgroup computes its expert's
// gate/up columns for every token while workgroup 0 routes -- the weight
// stream, not the MFMAs, sets its time, and that stream is the same -- and
// then reads its expert's record (one load, issued before its last block of
// K-steps; the routing is done by then) to store the act rows of the tokens
// routed to e: token t's row is the first row plus the routed tokens before
// t (the block lists its entries in token order).  A row's MFMA result
// depends only on that row, in the same K order and with the same MFMAs as
// skinny_body, so act has the two-call path's bits.  Each GEMM-1 workgroup
// then adds 2 to its expert's count.  GEMM-2 workgroups stream their
// weights (all of K = 512: registers + LDS) up front, wait for their
// expert's record and read its rows and destination cells (written before
// the records), then wait for that count to reach twice the GEMM-1 column
// blocks and read act.  The last user of a record clears it for the next
// launch.  The combine has
// no wait of its own: the last GEMM-2 workgroup of a column block to finish
// (one per expert with rows) combines that column block for every token
// (combine8_chunk, the same slot-order sum as mep_combine), reading y, the
// gates and row_of_entry with device-scope loads.  A wait that gives up sets
// the wait flag; the routing wait also poisons the launch (schedule word
// dec::kPoison: every output NaN); every counter is taken back out by the
// last workgroup that uses it.
namespace dec {
constexpr int kMaxTokens = 32;
constexpr int E = 32;
// Schedule words.  Counters that many workgroups update each sit in a
// 256-byte block of their own: device-scope atomics on one line are
// performed one after another where that line lives, and a few hundred of
// them on one line put microseconds of queueing in front of every count
// behind them.
constexpr int kPoison = sched::kRowDone;                // a routing wait gave up
constexpr int kCombined = kPoison + 1;                  // column blocks combined
constexpr int kBlock = 2 * sched::kLine;                // ints per counter block
// expert e's block: GEMM-1 count, GEMM-2 workgroups past their wait, users
// done with the routing record, and the record itself (one 64-bit word: bit
// 63 set once written, bits 32..47 the expert's first row, bits 0..31 its
// tokens, bit t for token t)
__host__ __device__ constexpr int kExp(int e) { return sched::kRowDone + kBlock * (1 + e); }
constexpr int kDone1 = 0, kSeen2 = 1, kUsers = 2, kRecWord = 4;
// column block cb's block: GEMM-2 workgroups done with it
__host__ __device__ constexpr int kColBlk(int cb) { return sched::kRowDone + kBlock * (1 + E + cb); }
constexpr uint64_t kRecValid = 1ull << 63;
constexpr int kRouterLds = E * kRowStride32 + kWaves * kRowsPerWave * (E + 1) * 4 + kWaves * E * 4 + 2 * E * 4;
constexpr int kLds = kRouterLds > skinny::LDS_W ? kRouterLds : skinny::LDS_W;
inline int64_t words(int hidden) { return kColBlk(hidden / 128); }
__device__ __forceinline__ uint64_t* rec_word(int* sched, int e) {
  return reinterpret_cast<uint64_t*>(sched + kExp(e) + kRecWord);
}
}  // namespace dec

struct DecodeParams {
  const uint16_t* x;             // (n, H)
  const uint16_t* w_router;      // (E, H)
  const uint8_t* valid;          // (n,) or NULL
  int64_t n_tokens;
  int64_t* topk_idx;             // (n, 8)
  uint16_t* gate;                // (n, 8)
  float* logits;                 // (n, E) or NULL
  int32_t* counts;               // (E,)
  int32_t* offsets;              // (E + 1,)
  int32_t* perm;                 // (n * 8,)
  int32_t* row_of_entry;         // (n * 8,)
  int64_t* route_counts;         // (E,) or NULL
  uint32_t* ws_header;           // dispatch workspace: header word 0 and the two status words
  uint32_t* ws_flags;
  GemmParams g1, g2;             // GEMM-1: x -> act; GEMM-2: act -> y_entries
  uint16_t* out;                 // (n, H)
  int n_g1, n_g2;                // GEMM-1 / GEMM-2 workgroups (E x column blocks each)
  int* sched;
  int wait_limit;                // polls before GEMM-2's wait for act gives up
  int route_wait_limit;          // polls before GEMM-1's wait for its routing record gives up
  int dbg_routed;                // GEMM-1 workgroup whose routing wait cannot end (test hook; -1: none)
};


// A user of expert e's routing record is done with it (workgroup 0 after
// writing it, every GEMM-1 and GEMM-2 workgroup of the expert after reading
// it): the last of them clears it for the next launch.
__device__ __forceinline__ void decode_rec_done(const DecodeParams& p, int e) {
  int* const users = p.sched + dec::kExp(e) + dec::kUsers;
  const int n = 1 + p.g1.N / 64 + p.g2.N / 128;
  if (atomic_add_1(users, 1) == n - 1) {
    __hip_atomic_store(dec::rec_word(p.sched, e), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    atomic_add_1(users, -n);
  }
}

// A GEMM-2 workgroup of expert e is done with the expert's GEMM-1 count
// (past its wait, at its end): the last of the expert's GEMM-2 workgroups
// takes the counts back out, so a count that arrives after a give-up still
// leaves both at zero.  Counted at the end, next to the column block's
// count, so that its round trip is not one more between GEMM-1's last count
// and GEMM-2's K loop.
__device__ __forceinline__ void decode_seen2(const DecodeParams& p, int e) {
  int* const seen2 = p.sched + dec::kExp(e) + dec::kSeen2;
  const int n_cb = p.g2.N / 128;
  if (atomic_add_1(seen2, 1) == n_cb - 1) {
    atomic_add_1(p.sched + dec::kExp(e) + dec::kDone1, -2 * (p.g1.N / 64));
    atomic_add_1(seen2, -n_cb);
  }
}

// Workgroup 0: route the batch (router32_logits, router_tail: the fused
// router's code), dispatch it as one block (flat order, stable by expert:
// modeling.py:94-96), then publish the routing.
template <int NSEG>
__device__ void decode_route(const DecodeParams& p, unsigned char* lds) {
  constexpr int E = dec::E, KC = 8;
  unsigned char* const ws = lds;
  float (*lg)[kRowsPerWave][E + 1] = reinterpret_cast<float (*)[kRowsPerWave][E + 1]>(lds + E * kRowStride32);
  int (*s_wcnt)[E] = reinterpret_cast<int (*)[E]>(lds + E * kRowStride32 + kWaves * kRowsPerWave * (E + 1) * 4);
  int* const s_base = reinterpret_cast<int*>(lds + E * kRowStride32 + kWaves * kRowsPerWave * (E + 1) * 4 +
                                             kWaves * E * 4);
  uint32_t* const s_mask = reinterpret_cast<uint32_t*>(s_base + E);   // tokens of each expert
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  if (tid < kWaves * E) s_wcnt[tid / E][tid % E] = 0;   // published by the first barrier of router32_logits
  if (tid < E) s_mask[tid] = 0u;
  const int64_t t0 = static_cast<int64_t>(wave) * kRowsPerWave;
  f32x4 acc[2];
  router32_logits<NSEG>(p.x, p.w_router, p.n_tokens, t0, ws, acc);
  RouterHist hist{};
  hist.valid = p.valid;
  int sel[2];                                     // experts of this lane's two slots, -1: not dispatched
  router_tail<MEP_DTYPE_BF16, E, KC>(acc, lg[wave], nullptr, nullptr, nullptr, nullptr, nullptr, t0, p.n_tokens, KC,
                                      p.topk_idx, p.gate, p.logits, hist, sel);
  // rank of each entry among the wave's entries of its expert (lane order =
  // token order; a lane's two slots hold different experts)
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
    if (e >= 0) atomicOr(s_mask + e, 1u << static_cast<int>(t0 + (lane >> 2)));   // token < 32
  }
  __syncthreads();
  if (tid < E) {
    int tot = 0;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) tot += s_wcnt[ww][tid];
    int incl = tot;                                // inclusive prefix over experts (lanes 0..31 of wave 0)
#pragma unroll
    for (int d = 1; d < E; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    const int off = incl - tot;
    s_base[tid] = off;
    p.counts[tid] = tot;
    p.offsets[tid] = off;
    if (tid == E - 1) p.offsets[E] = incl;
    if (p.route_counts != nullptr) p.route_counts[tid] += tot;
  }
  __syncthreads();
  const int t = lane >> 2, g = lane & 3;
  if (t0 + t < p.n_tokens) {
    const int64_t f = (t0 + t) * KC + g * 2;
    int row[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = sel[h];
      row[h] = -1;
      if (e >= 0) {
        int r = s_base[e] + rank[h];
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) r += ww < wave ? s_wcnt[ww][e] : 0;
        row[h] = r;
        p.perm[r] = static_cast<int32_t>(f + h);
      }
    }
    p.row_of_entry[f] = row[0];
    p.row_of_entry[f + 1] = row[1];
  }
  if (tid == 0) {
    p.ws_flags[0] = 0u;
    p.ws_flags[1] = 0u;
    p.ws_header[0] = 1u;
  }
  // every wave's stores are in this XCD's L2; write them back to memory,
  // then publish the records (device scope: written through to memory)
  __syncthreads();
  if (wave == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (lane < E) {
      const uint64_t rec = dec::kRecValid | (static_cast<uint64_t>(s_base[lane]) << 32) | s_mask[lane];
      __hip_atomic_store(dec::rec_word(p.sched, lane), rec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // workgroup 0 is one of the record's users: its count follows the
      // record, so that whoever clears it does so after it landed
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
      decode_rec_done(p, lane);
    }
  }
}

// The last GEMM-2 workgroup of column block cb: out[t, cb*128 .. +128) for
// every token, combine8's slot-order sum with device-scope reads of y, the
// gates and row_of_entry; NaN everywhere if a routing wait gave up (the
// poison word is read with the other loads, after this workgroup's count of
// the column block returned, so after every GEMM-2 count it follows).  It then
// counts the column block combined; the last column block returns the
// poison and its own counter to zero.
__device__ void decode_combine(const DecodeParams& p, int cb, int n_cb2) {
  const int tid = threadIdx.x;
  const uint16_t* const y = static_cast<const uint16_t*>(p.g2.C);
  const int H = p.g2.N;
  const uint32_t y_bytes = static_cast<uint32_t>(p.n_tokens * 8 * H * 2);
  for (int q = tid; q < p.n_tokens * 16; q += skinny::NT) {
    const int64_t t = q >> 4;
    const int c = cb * 16 + (q & 15);
    auto ld = [&](const uint16_t* ptr) { return load_dev_16(y, y_bytes, static_cast<uint32_t>((ptr - y) * 2)); };
    combine8_chunk<MEP_DTYPE_BF16, decltype(ld), true>(y, p.gate, p.row_of_entry, p.valid, t, c, H, p.out, ld,
                                                       p.sched + dec::kPoison);
  }
  if (tid == 0 && atomic_add_1(p.sched + dec::kCombined, 1) == n_cb2 - 1) {
    atomic_add_1(p.sched + dec::kCombined, -n_cb2);
    atomicExch(p.sched + dec::kPoison, 0);
  }
}

// GEMM workgroup u of the decode launch: expert e, column block cb (see above).
template <bool GEMM1>
__device__ void decode_gemm(const DecodeParams& p, int u, unsigned char* lds, int* s_msg) {
  using namespace skinny;
  typedef uint16_t T;
  const GemmParams& g = GEMM1 ? p.g1 : p.g2;
  int* const sched = p.sched;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_cb = GEMM1 ? g.N / 64 : g.N / 128;
  const int n_cb1 = p.g1.N / 64, n_cb2 = p.g2.N / 128;
  const int e = __builtin_amdgcn_readfirstlane(((u >> 3) / n_cb) * 8 + (u & 7));
  const int cb = __builtin_amdgcn_readfirstlane((u >> 3) % n_cb);
  const int n = static_cast<int>(p.n_tokens);
  const int max_entries = n * 8;
  const int lr = lane & 15, lg = lane >> 4;
  const int K = g.K, KT = K / 32, KD = K / 64;
  const int nt = cb / 2;
  const int rot = (!GEMM1 && KD % 4 == 0) ? 2 * (nt & 3) * (KD / 4) : 0;
  const T* W = static_cast<const T*>(g.W) + static_cast<int64_t>(e) * g.w_expert_stride;
  int wrow[2];
  if constexpr (GEMM1) {
    const int g0 = cb * 64 + wave * 16;
    wrow[0] = g0 + lr;
    wrow[1] = g.N + g0 + lr;
  } else {
    const int c0 = cb * 128 + wave * 32;
    wrow[0] = c0 + lr;
    wrow[1] = c0 + 16 + lr;
  }
  const T* wp0 = W + static_cast<int64_t>(wrow[0]) * K + 8 * lg;
  const T* wp1 = W + static_cast<int64_t>(wrow[1]) * K + 8 * lg;
  int* const done1 = sched + dec::kExp(e) + dec::kDone1;
  uint64_t rec = 0;                                      // the expert's routing record
  auto load_rec = [&]() {
    return __hip_atomic_load(dec::rec_word(sched, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  u32x4 wq[DEPTH][2], aq[DEPTH][MFC];
  auto k_off = [&](int tt) {
    int ks = tt + rot;
    if (ks >= KT) ks -= KT;
    return static_cast<int64_t>(ks) * 32;
  };
  const int n_lds = min(LSTEPS, KT - DEPTH);
  unsigned char* const w_lds = lds + wave * (LSTEPS * 2 * 1024);
  auto load_w = [&](int tt, int slot) {
    const int64_t off = k_off(tt);
    wq[slot][0] = *reinterpret_cast<const u32x4*>(wp0 + off);
    wq[slot][1] = *reinterpret_cast<const u32x4*>(wp1 + off);
  };
  auto load_w_lds = [&](int tt, int slot) {               // a step staged in LDS: [DEPTH, DEPTH + n_lds)
    const unsigned char* b = w_lds + (tt - DEPTH) * 2048 + 16 * lane;
    wq[slot][0] = *reinterpret_cast<const u32x4*>(b);
    wq[slot][1] = *reinterpret_cast<const u32x4*>(b + 1024);
  };
  // the first DEPTH K-steps of this wave's weights to registers (each lane
  // fetches the 16 bytes it later feeds the MFMA); GEMM-2 also stages the
  // next n_lds steps in LDS, since it waits before its K loop.  The weights
  // need only the expert, so this runs before any wait.
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_w(d, d);
  if constexpr (!GEMM1) {
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(W);
    const int wbytes = static_cast<int>(g.w_expert_stride * 2);
    const uint32_t lo0 = static_cast<uint32_t>((wp0 - W) * 2), lo1 = static_cast<uint32_t>((wp1 - W) * 2);
    for (int tt = DEPTH; tt < DEPTH + n_lds; ++tt) {
      const uint32_t ko = static_cast<uint32_t>(k_off(tt) * 2);
      buffer_lds_16(wb, wbytes, lo0 + ko, 0, w_lds + (tt - DEPTH) * 2048);
      buffer_lds_16(wb, wbytes, lo1 + ko, 0, w_lds + (tt - DEPTH) * 2048 + 1024);
    }
  }
  const T* A = static_cast<const T*>(g.A);
  const T* ap[MFC];
  int r0 = 0, row_hi = 0, n_active = 0;
  int cell[MFC];
  if constexpr (!GEMM1) {
    if (tid == 0) {
      s_msg[3] = 0;
      // the routing is complete once the expert's record is written (after
      // workgroup 0's other stores reached memory), so the rows are read
      // while GEMM-1 still runs; bounded: a give-up flags and NaNs this
      // workgroup's rows
      int polls = 0;
      while ((load_rec() & dec::kRecValid) == 0) {
        if (++polls == p.wait_limit) {
          atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
          s_msg[3] = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      decode_rec_done(p, e);                             // done with the record
    }
    __syncthreads();
    // this expert's rows (at most 32), checked so that whatever a workgroup
    // reads after a give-up stays in bounds
    int lo = load_dev_i32(p.offsets + e), hi = load_dev_i32(p.offsets + e + 1);
    if (lo < 0 || hi < lo || hi - lo > 16 * MFC || hi > max_entries) hi = lo = 0;
    lo = __builtin_amdgcn_readfirstlane(lo);
    hi = __builtin_amdgcn_readfirstlane(hi);
    // experts with rows: one GEMM-2 workgroup each per column block
    const int o0 = lane < dec::E ? load_dev_i32(p.offsets + lane) : 0;
    const int o1 = lane < dec::E ? load_dev_i32(p.offsets + lane + 1) : 0;
    n_active = __builtin_amdgcn_readfirstlane(static_cast<int>(__popcll(__ballot(lane < dec::E && o1 > o0))));
    r0 = lo;
    row_hi = hi;
    if (hi > lo) {
#pragma unroll
      for (int f = 0; f < MFC; ++f) {
        const int r = min(r0 + 16 * f + lr, row_hi - 1);
        const int c = load_dev_i32(p.perm + r);
        cell[f] = c < 0 ? 0 : (c >= max_entries ? max_entries - 1 : c);
        ap[f] = A + static_cast<int64_t>(r) * K + 8 * lg;   // act row
      }
    }
    if (tid == 0) {
      // until every GEMM-1 workgroup of the expert has stored its act rows
      // (each adds 2 after them); bounded as above
      const int target = 2 * n_cb1 + (e == g.dbg_chunk ? 1 : 0);
      int polls = 0;
      while (load_dev_i32(done1) < target) {
        if (++polls == p.wait_limit) {
          atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
          s_msg[3] = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
    if (hi == lo) {
      // no rows: nothing to compute (every token masked: expert 0's GEMM-2
      // workgroups write the zero outputs)
      __builtin_amdgcn_s_waitcnt(kVmcnt0);        // no DMA may still be writing LDS when the waves end
      if (tid == 0) decode_seen2(p, e);
      if (n_active == 0 && e == 0) decode_combine(p, cb, n_cb2);
      return;
    }
  }
  f32x4 acc[MFC][2];
#pragma unroll
  for (int f = 0; f < MFC; ++f)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[f][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (GEMM1) {
    // x, every token of the batch (row 16 f + lr of the MFMA is token
    // 16 f + lr; rows past the batch repeat its last token), is the same for
    // the four waves: it goes through an LDS ring of two blocks of DEPTH
    // steps, laid out in MFMA lane order (step s, row fragment f: lane L's
    // 16 bytes at (s MFC + f) KiB + 16 L).  Wave w copies rows 8 w .. 8 w + 7
    // of a block, whole 128-byte lines (8 rows per load), into registers one
    // block ahead and writes them after the block's MFMAs.  Read by each wave
    // from memory instead, x would be fetched four times over in half lines
    // and take most of the requests a CU keeps in flight, which is what
    // bounds this loop; the weights stream into registers DEPTH steps ahead.
    // (Plain loads and LDS writes, not LDS DMA: the compiler waits for every
    // load in flight before reading LDS that a DMA may have written.)
    static_assert(DEPTH == 8 && MFC == 2 && NW == 4, "a block of x is 32 rows x 4 lines, 4 loads per wave");
    static_assert(16 * MFC == dec::kMaxTokens, "one row block holds the batch");
    constexpr int kSlot = DEPTH * MFC * 1024;
    unsigned char* const a_lds = lds;                    // [2][DEPTH][MFC][1 KiB]
    const int xrow = 8 * wave + (lane >> 3), xc = lane & 7;   // row of the block, 16-byte chunk of a line
    const unsigned char* const xsrc =
        reinterpret_cast<const unsigned char*>(A) + static_cast<int64_t>(min(xrow, n - 1)) * K * 2 + 16 * xc;
    // LDS offset of this lane's chunk of line i (steps 2 i, 2 i + 1)
    const int xdst = ((xc >> 2) * MFC + (xrow >> 4)) * 1024 + ((xrow & 15) + 16 * (xc & 3)) * 16;
    u32x4 xr[4];
    auto load_x = [&](int b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xr[i] = *reinterpret_cast<const u32x4*>(xsrc + b * (DEPTH * 64) + i * 128);
    };
    auto write_x = [&](int b) {
      unsigned char* const dst = a_lds + (b & 1) * kSlot + xdst;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(dst + i * (2 * MFC * 1024)) = xr[i];
    };
    auto block = [&](int b, bool next) {
      const unsigned char* const src = a_lds + (b & 1) * kSlot + 16 * lane;
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        u32x4 a[MFC];
#pragma unroll
        for (int f = 0; f < MFC; ++f) a[f] = *reinterpret_cast<const u32x4*>(src + (d * MFC + f) * 1024);
#pragma unroll
        for (int f = 0; f < MFC; ++f)
#pragma unroll
          for (int j = 0; j < 2; ++j) mfma_acc(acc[f][j], wq[d][j], a[f]);
        if (next) load_w((b + 1) * DEPTH + d, d);
      }
    };
    // block b + 1 of x is loaded during block b and written after it; its
    // slot last held block b - 1, which every wave finished before the
    // barrier that ended block b - 1
    const int NB = KT / DEPTH;                           // at least 4 (K = hidden >= 1024)
    load_x(0);
    write_x(0);
    lds_barrier();
    for (int b = 0; b < NB - 1; ++b) {
      load_x(b + 1);
      block(b, true);
      write_x(b + 1);
      lds_barrier();
    }
    // the expert's routing record, read before the last block (the routing
    // is done by then; it is checked after the block)
    rec = load_rec();
    block(NB - 1, false);
  } else {
    // this wave's LDS steps have landed (its own lanes read them back)
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    auto load_a = [&](int tt, int slot) {
      const int64_t off = k_off(tt);
#pragma unroll
      for (int f = 0; f < MFC; ++f) aq[slot][f] = *reinterpret_cast<const u32x4*>(ap[f] + off);
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_a(d, d);
    k_pipeline(
        KT,
        [&](int d) {
#pragma unroll
          for (int f = 0; f < MFC; ++f)
#pragma unroll
            for (int j = 0; j < 2; ++j) mfma_acc(acc[f][j], wq[d][j], aq[d][f]);
        },
        [&](int tt, int slot) {
          load_w_lds(tt, slot);
          load_a(tt, slot);
        },
        [&](int tt, int slot) {
          load_w(tt, slot);
          load_a(tt, slot);
        },
        [](int) {});
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int f = 0; f < MFC; ++f)
#pragma unroll
    for (int j = 0; j < 2; ++j) pin_acc(acc[f][j]);
  T* const C = static_cast<T*>(g.C);
  if constexpr (GEMM1) {
    // the record read before the last block, else until it is written
    // (bounded, each wave on its own; a give-up flags and poisons the launch,
    // and the wave stores nothing)
    if ((rec & dec::kRecValid) == 0 || u == p.dbg_routed) {
      int polls = 0;
      while ((rec & dec::kRecValid) == 0 || u == p.dbg_routed) {
        if (++polls == p.route_wait_limit) {
          if (lane == 0) {
            atomic_or_1(sched + sched::kFlags, sched::kFlagWait);
            atomic_or_1(sched + dec::kPoison, 1);
          }
          rec = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        rec = load_rec();
      }
    }
    // token t's act row: the expert's first row plus the routed tokens
    // before t (checked, so that a record read after a give-up stays in bounds)
    uint32_t mask = static_cast<uint32_t>(rec) & (n >= 32 ? ~0u : (1u << n) - 1u);
    const int first = static_cast<int>((rec >> 32) & 0xFFFFu);
    if (first + static_cast<int>(__popc(mask)) > max_entries) mask = 0u;
#pragma unroll
    for (int f = 0; f < MFC; ++f) {
      const int t = 16 * f + lr;
      if (((mask >> t) & 1u) == 0u) continue;
      const int r = first + __popc(mask & ((1u << t) - 1u));
      const int col = cb * 64 + wave * 16 + 4 * lg;
      uint32_t w[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        w[h] = pack_bf16x2(silu_f(acc[f][0][2 * h]) * acc[f][1][2 * h],
                           silu_f(acc[f][0][2 * h + 1]) * acc[f][1][2 * h + 1]);
      uint64_t* const dst = reinterpret_cast<uint64_t*>(C + static_cast<int64_t>(r) * g.N + col);
      __hip_atomic_store(dst, (static_cast<uint64_t>(w[1]) << 32) | w[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    // a GEMM-2 wait for act that gave up: NaN rows
    if (__builtin_amdgcn_readfirstlane(s_msg[3])) {
      const float nan = __builtin_nanf("");
#pragma unroll
      for (int f = 0; f < MFC; ++f)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[f][j] = f32x4{nan, nan, nan, nan};
    }
#pragma unroll
    for (int f = 0; f < MFC; ++f) {
      const int r = r0 + 16 * f + lr;
      if (r >= row_hi) continue;
      const int64_t row = cell[f];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = cb * 128 + wave * 32 + 16 * j + 4 * lg;
        const uint2 w = make_uint2(pack_bf16x2(acc[f][j][0], acc[f][j][1]), pack_bf16x2(acc[f][j][2], acc[f][j][3]));
        __hip_atomic_store(reinterpret_cast<uint64_t*>(C + row * g.N + col), (static_cast<uint64_t>(w.y) << 32) | w.x,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // every wave's stores are complete before the counts go up
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  __syncthreads();
  if constexpr (GEMM1) {
    if (tid == 0) {
      atomic_add_1(done1, 2);
      decode_rec_done(p, e);
    }
  } else {
    // the last GEMM-2 workgroup of the column block combines it
    if (tid == 0) {
      int* const col = sched + dec::kColBlk(cb);
      const int c = atomic_add_1(col, 1);
      decode_seen2(p, e);                                  // its round trip overlaps the count's
      s_msg[1] = c == n_active - 1;
      if (c == n_active - 1) atomic_add_1(col, -n_active);
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(s_msg[1])) decode_combine(p, cb, n_cb2);
  }
}

template <int NSEG>
__global__ __launch_bounds__(skinny::NT) void moe_decode_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[dec::kLds];
  __shared__ int s_msg[4];
  const int b = blockIdx.x;
  if (b == 0) {
    // the routing, then the last GEMM-2 unit (its weights are needed only
    // once GEMM-1 is done): the grid is then one workgroup smaller, and at
    // hidden 1024 every workgroup is resident from the start (two per CU)
    decode_route<NSEG>(p, lds);
    __syncthreads();                                 // the router's LDS is free
    decode_gemm<false>(p, p.n_g2 - 1, lds, s_msg);
  } else if (b <= p.n_g1) {
    decode_gemm<true>(p, b - 1, lds, s_msg);
  } else {
    decode_gemm<false>(p, b - 1 - p.n_g1, lds, s_msg);
  }
}

// XCD queues of a device with n_cu compute units: one per 32 CUs (8 on a
// whole MI355X), a power of two.
int queues_for(int n_cu) {
  int nq = n_cu / 32;
  nq = nq < 1 ? 1 : (nq > 8 ? 8 : nq);
  return pow2_floor(nq);
}

// One persistent workgroup per CU (at most one item's worth), a multiple of
// the queue count so that every XCD runs the same number.
template <int MODE>
hipError_t launch_tiled(const MoeParams& p, int64_t max_rows, hipStream_t stream) {
  const int n1 = p.I / (bfk::BN / 2), n2 = p.H / bfk::BN;
  const int per_row = MODE == kModeGateUp ? n1 : (MODE == kModeDown ? n2 : n1 + n2);
  const int64_t items = ((max_rows + bfk::BM - 1) / bfk::BM + p.n_local) * per_row;
  if (items == 0) return hipSuccess;
  const int nq = p.n_queues;
  const int64_t cap = device_cu_count() / nq * nq;
  int64_t grid = items < cap ? items : cap;
  grid = (grid + nq - 1) / nq * nq;
  moe_gemm_bf16_kernel<MODE><<<dim3(static_cast<unsigned>(grid)), bfk::NT, 0, stream>>>(p);
  return hipGetLastError();
}

MoeParams moe_params(const void* x, int64_t n_tokens, int top_k, const int32_t* perm, const int32_t* offsets,
                     int n_local, int64_t max_rows, const void* w_in, const void* w_out, const int32_t* w_slot,
                     int hidden, int inter, void* act, void* y, int32_t* sched) {
  MoeParams p;
  p.x = x; p.act = act; p.y = y; p.perm = perm; p.offsets = offsets; p.w_slot = w_slot;
  p.w_in = w_in; p.w_out = w_out;
  p.n_local = n_local; p.top_k = top_k; p.H = hidden; p.I = inter;
  p.x_bytes = static_cast<uint32_t>(n_tokens * hidden * 2);
  p.act_bytes = static_cast<uint32_t>(max_rows * inter * 2);
  div_magic(static_cast<uint32_t>(top_k), &p.k_magic, &p.k_shift);
  p.n_queues = queues_for(device_cu_count());
  p.sched = sched;
  const GiveupTest gt = giveup_test();
  p.wait_limit = gt.site == MEP_GIVEUP_ROWS ? gt.polls : sched::kWaitLimit;
  p.dbg_row = gt.site == MEP_GIVEUP_ROWS ? 0 : -1;
  return p;
}

// The schedule-buffer fields of the small-batch and generic kernels' params.
void set_sched(GemmParams& g, int32_t* sched) {
  g.flags = sched != nullptr ? sched + sched::kFlags : nullptr;
  const GiveupTest gt = giveup_test();
  g.wait_limit = gt.site == MEP_GIVEUP_CHUNK ? gt.polls : sched::kWaitLimit;
  g.dbg_chunk = gt.site == MEP_GIVEUP_CHUNK ? 0 : -1;
}

// The bf16 tiled kernels need K a multiple of 256 (whole four-step rounds,
// GEMM-2's stage rotation) and more rows than the small-batch kernels take.
bool tiled_gate_up(int dtype, int64_t max_rows) {
  return dtype == MEP_DTYPE_BF16 && max_rows > skinny::kMaxEntries1;
}
bool tiled_down(int dtype, int64_t max_rows, int inter) {
  return dtype == MEP_DTYPE_BF16 && inter % 256 == 0 && max_rows > skinny::kMaxEntries2;
}

// Tile shapes of the generic kernel (fp32, and bf16 GEMM-2 with I % 256 != 0):
// bf16 256x256 on 8 waves (4 x 2), fp32 128x128 on 4 waves.
typedef TileCfg<256, 256, 4, 2> CfgBf16;
typedef TileCfg<128, 128, 2, 2> CfgF32;

// GEMM-1 / GEMM-2 parameters of the small-batch and generic kernels
template <int DT, class Cfg>
GemmParams gemm1_params(const void* x, int64_t n_tokens, int top_k, const int32_t* perm, const int32_t* offsets,
                        int n_local, const void* w_in, const int32_t* w_slot, int hidden, int inter, void* act) {
  GemmParams g1;
  g1.A = x; g1.perm = perm; g1.offsets = offsets; g1.W = w_in; g1.C = act;
  g1.w_slot = w_slot;
  g1.w_expert_stride = static_cast<int64_t>(2) * inter * hidden;
  g1.n_local = n_local; g1.top_k = top_k; g1.K = hidden; g1.N = inter;
  g1.n_tiles_n = inter / (Cfg::BN / 2);
  g1.a_bytes = static_cast<uint32_t>(n_tokens * hidden * dtype_bytes(DT));
  div_magic(static_cast<uint32_t>(top_k), &g1.k_magic, &g1.k_shift);
  set_sched(g1, nullptr);
  return g1;
}
template <int DT, class Cfg>
GemmParams gemm2_params(const void* act, int top_k, const int32_t* perm, const int32_t* offsets, int n_local,
                        int64_t max_rows, const void* w_out, const int32_t* w_slot, int hidden, int inter, void* y) {
  GemmParams g2;
  g2.A = act; g2.perm = perm; g2.offsets = offsets; g2.W = w_out; g2.C = y;
  g2.w_slot = w_slot;
  g2.w_expert_stride = static_cast<int64_t>(hidden) * inter;
  g2.n_local = n_local; g2.top_k = top_k; g2.K = inter; g2.N = hidden;
  g2.n_tiles_n = hidden / Cfg::BN;
  g2.a_bytes = static_cast<uint32_t>(max_rows * inter * dtype_bytes(DT));
  div_magic(static_cast<uint32_t>(top_k), &g2.k_magic, &g2.k_shift);
  set_sched(g2, nullptr);
  return g2;
}

template <int DT, class Cfg>
int run_gate_up(const void* x, int64_t n_tokens, int top_k, const int32_t* perm, const int32_t* offsets,
                int n_local, int64_t max_rows, const void* w_in, const int32_t* w_slot, int hidden, int inter,
                void* act, int32_t* sched, hipStream_t stream) {
  hipError_t e;
  if (tiled_gate_up(DT, max_rows)) {
    const MoeParams p = moe_params(x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, nullptr, w_slot,
                                   hidden, inter, act, nullptr, sched);
    e = launch_tiled<kModeGateUp>(p, max_rows, stream);
  } else {
    GemmParams g1 = gemm1_params<DT, Cfg>(x, n_tokens, top_k, perm, offsets, n_local, w_in, w_slot, hidden,
                                          inter, act);
    set_sched(g1, sched);
    if (DT == MEP_DTYPE_BF16) e = launch_skinny<true>(g1, max_rows, stream);
    else e = launch<DT, Cfg, true>(g1, max_rows, stream);
  }
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_swiglu_gate_up: %s", hipGetErrorString(e));
  return MEP_OK;
}

template <int DT, class Cfg>
int run_down(const void* act, int top_k, const int32_t* perm, const int32_t* offsets, int n_local,
             int64_t max_rows, const void* w_out, const int32_t* w_slot, int hidden, int inter, void* y,
             int32_t* sched, hipStream_t stream) {
  hipError_t e;
  if (tiled_down(DT, max_rows, inter)) {
    MoeParams p = moe_params(nullptr, 0, top_k, perm, offsets, n_local, max_rows, nullptr, w_out, w_slot, hidden,
                             inter, const_cast<void*>(act), y, sched);
    e = launch_tiled<kModeDown>(p, max_rows, stream);
  } else {
    GemmParams g2 = gemm2_params<DT, Cfg>(act, top_k, perm, offsets, n_local, max_rows, w_out, w_slot, hidden,
                                          inter, y);
    set_sched(g2, sched);
    if (DT == MEP_DTYPE_BF16 && inter % 256 == 0) e = launch_skinny<false>(g2, max_rows, stream);
    else e = launch<DT, Cfg, false>(g2, max_rows, stream);
  }
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


namespace mep {
namespace {

// The schedule buffer a launch needs: non-null, and at least
// mep_experts_queue_ints(max_rows, n_local) words when a tiled kernel runs.
int check_queue(const char* fn, bool tiled, int32_t* tile_queue, size_t tile_queue_ints, int64_t max_rows,
                int n_local) {
  MEP_REQUIRE(tile_queue != nullptr, MEP_ERR_INVALID_ARG, "%s: null tile_queue", fn);
  if (tiled) {
    const int64_t need = sched::words(max_rows, n_local);
    MEP_REQUIRE(static_cast<int64_t>(tile_queue_ints) >= need, MEP_ERR_WORKSPACE,
                "%s: tile_queue has %zu ints < required %lld", fn, tile_queue_ints, (long long)need);
  }
  return MEP_OK;
}

int gate_up_impl(const char* fn, const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                 const int32_t* offsets, int32_t n_local, int64_t max_rows, const void* w_in,
                 const int32_t* w_slot, int32_t hidden, int32_t inter, int32_t dtype, void* act,
                 size_t act_bytes, int32_t* tile_queue, size_t tile_queue_ints, void* stream) {
  int rc = check_expert_args(fn, n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(x && perm && offsets && w_in && act, MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
  rc = check_queue(fn, tiled_gate_up(dtype, max_rows), tile_queue, tile_queue_ints, max_rows, n_local);
  if (rc != MEP_OK) return rc;
  const size_t need = static_cast<size_t>(max_rows) * inter * dtype_bytes(dtype);
  MEP_REQUIRE(act_bytes >= need, MEP_ERR_WORKSPACE, "%s: act %zu B < required %zu B", fn, act_bytes, need);
  MEP_REQUIRE(aligned16(x) && aligned16(w_in) && aligned16(act), MEP_ERR_INVALID_ARG,
              "%s: buffers must be 16-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MEP_DTYPE_BF16)
    return run_gate_up<MEP_DTYPE_BF16, CfgBf16>(x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_slot,
                                                hidden, inter, act, tile_queue, s);
  return run_gate_up<MEP_DTYPE_F32, CfgF32>(x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_slot,
                                            hidden, inter, act, tile_queue, s);
}

int down_impl(const char* fn, const void* act, int64_t n_tokens, int32_t top_k, const int32_t* perm,
              const int32_t* offsets, int32_t n_local, int64_t max_rows, const void* w_out, const int32_t* w_slot,
              int32_t hidden, int32_t inter, int32_t dtype, void* y_entries, int32_t* tile_queue,
              size_t tile_queue_ints, void* stream) {
  int rc = check_expert_args(fn, n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(act && perm && offsets && w_out && y_entries, MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
  rc = check_queue(fn, tiled_down(dtype, max_rows, inter), tile_queue, tile_queue_ints, max_rows, n_local);
  if (rc != MEP_OK) return rc;
  MEP_REQUIRE(aligned16(act) && aligned16(w_out) && aligned16(y_entries), MEP_ERR_INVALID_ARG,
              "%s: buffers must be 16-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MEP_DTYPE_BF16)
    return run_down<MEP_DTYPE_BF16, CfgBf16>(act, top_k, perm, offsets, n_local, max_rows, w_out, w_slot, hidden,
                                             inter, y_entries, tile_queue, s);
  return run_down<MEP_DTYPE_F32, CfgF32>(act, top_k, perm, offsets, n_local, max_rows, w_out, w_slot, hidden,
                                         inter, y_entries, tile_queue, s);
}

// Both GEMMs: one launch of the tiled kernel when both would run tiled, else
// the two launches.
// comb: NULL, or a combine that the small-batch launch may end with; then
// *combined tells whether it did (otherwise the caller runs the combine).
int grouped_impl(const char* fn, const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                 const int32_t* offsets, int32_t n_local, int64_t max_rows, const void* w_in, const void* w_out,
                 const int32_t* w_slot, int32_t hidden, int32_t inter, int32_t dtype, void* y_entries,
                 void* workspace, size_t workspace_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                 void* stream, const CombineParams* comb = nullptr, bool* combined = nullptr) {
  if (combined != nullptr) *combined = false;
  int rc = check_expert_args(fn, n_tokens, top_k, n_local, max_rows, hidden, inter, dtype);
  if (rc != MEP_OK) return rc;
  if (max_rows == 0 || n_local == 0) return MEP_OK;
  MEP_REQUIRE(workspace != nullptr, MEP_ERR_INVALID_ARG, "%s: null workspace", fn);
  const size_t need = mep_experts_workspace_size(max_rows, inter, dtype);
  MEP_REQUIRE(workspace_bytes >= need, MEP_ERR_WORKSPACE, "%s: workspace %zu B < required %zu B", fn,
              workspace_bytes, need);
  if (tiled_gate_up(dtype, max_rows) && tiled_down(dtype, max_rows, inter)) {
    MEP_REQUIRE(x && perm && offsets && w_in && w_out && y_entries, MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
    rc = check_queue(fn, true, tile_queue, tile_queue_ints, max_rows, n_local);
    if (rc != MEP_OK) return rc;
    MEP_REQUIRE(aligned16(x) && aligned16(w_in) && aligned16(w_out) && aligned16(workspace) && aligned16(y_entries),
                MEP_ERR_INVALID_ARG, "%s: buffers must be 16-byte aligned", fn);
    const MoeParams p = moe_params(x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_out, w_slot,
                                   hidden, inter, workspace, y_entries, tile_queue);
    const hipError_t e = launch_tiled<kModeBoth>(p, max_rows, static_cast<hipStream_t>(stream));
    MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
    return MEP_OK;
  }
  if (dtype == MEP_DTYPE_BF16 && inter % 256 == 0 && !tiled_gate_up(dtype, max_rows) &&
      !tiled_down(dtype, max_rows, inter)) {
    // both small-batch GEMMs in one launch (GEMM-2's weights stream while GEMM-1 runs)
    MEP_REQUIRE(x && perm && offsets && w_in && w_out && y_entries, MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
    rc = check_queue(fn, true, tile_queue, tile_queue_ints, max_rows, n_local);
    if (rc != MEP_OK) return rc;
    MEP_REQUIRE(aligned16(x) && aligned16(w_in) && aligned16(w_out) && aligned16(workspace) && aligned16(y_entries),
                MEP_ERR_INVALID_ARG, "%s: buffers must be 16-byte aligned", fn);
    GemmParams g1 = gemm1_params<MEP_DTYPE_BF16, CfgBf16>(x, n_tokens, top_k, perm, offsets, n_local, w_in, w_slot,
                                                          hidden, inter, workspace);
    GemmParams g2 = gemm2_params<MEP_DTYPE_BF16, CfgBf16>(workspace, top_k, perm, offsets, n_local, max_rows, w_out,
                                                          w_slot, hidden, inter, y_entries);
    set_sched(g1, tile_queue);
    set_sched(g2, tile_queue);
    const hipError_t e = launch_skinny_both(g1, g2, max_rows, tile_queue, comb, static_cast<hipStream_t>(stream));
    MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
    if (combined != nullptr) *combined = comb != nullptr;
    return MEP_OK;
  }
  rc = gate_up_impl(fn, x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_slot, hidden, inter, dtype,
                    workspace, workspace_bytes, tile_queue, tile_queue_ints, stream);
  if (rc != MEP_OK) return rc;
  return down_impl(fn, workspace, n_tokens, top_k, perm, offsets, n_local, max_rows, w_out, w_slot, hidden, inter,
                   dtype, y_entries, tile_queue, tile_queue_ints, stream);
}

}  // namespace
}  // namespace mep

extern "C" size_t mep_experts_queue_ints(int64_t max_rows, int32_t n_local) {
  if (max_rows < 0 || n_local < 0) return 0;
  return static_cast<size_t>(mep::sched::words(max_rows, n_local));
}

extern "C" int mep_experts_check(const int32_t* tile_queue, void* stream) {
  clear_error();
  MEP_REQUIRE(tile_queue != nullptr, MEP_ERR_INVALID_ARG, "mep_experts_check: null tile_queue");
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_experts_check: %s", hipGetErrorString(e));
  int32_t flags = 0;
  e = hipMemcpy(&flags, tile_queue + mep::sched::kFlags, sizeof(flags), hipMemcpyDeviceToHost);
  MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_experts_check: %s", hipGetErrorString(e));
  if (flags != 0) {
    // reported once: the flags are cleared for the launches that follow
    const int32_t zero = 0;
    e = hipMemcpy(const_cast<int32_t*>(tile_queue) + mep::sched::kFlags, &zero, sizeof(zero), hipMemcpyHostToDevice);
    MEP_REQUIRE(e == hipSuccess, MEP_ERR_HIP, "mep_experts_check: %s", hipGetErrorString(e));
  }
  MEP_REQUIRE(!(flags & mep::sched::kFlagInput), MEP_ERR_HIP,
              "mep_experts_check: offsets[n_local] < 0, the dispatch gave up; no tile ran (results invalid)");
  MEP_REQUIRE(!(flags & mep::sched::kFlagWait), MEP_ERR_HIP,
              "mep_experts_check: a workgroup gave up waiting (GEMM-2 for its GEMM-1 rows, or the combine for "
              "GEMM-2's rows; its outputs are NaN)");
  MEP_REQUIRE(!(flags & mep::sched::kFlagDrain), MEP_ERR_HIP,
              "mep_experts_check: a tile queue was not drained (results invalid)");
  return MEP_OK;
}

extern "C" int mep_swiglu_gate_up(const void* x, int64_t n_tokens, int32_t top_k,
                                  const int32_t* perm, const int32_t* offsets, int32_t n_local,
                                  int64_t max_rows, const void* w_in, int32_t hidden, int32_t inter,
                                  int32_t dtype, void* act, size_t act_bytes, int32_t* tile_queue,
                                  size_t tile_queue_ints, void* stream) {
  clear_error();
  return gate_up_impl("mep_swiglu_gate_up", x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, nullptr,
                      hidden, inter, dtype, act, act_bytes, tile_queue, tile_queue_ints, stream);
}

extern "C" int mep_swiglu_down(const void* act, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                               const int32_t* offsets, int32_t n_local, int64_t max_rows,
                               const void* w_out, int32_t hidden, int32_t inter, int32_t dtype,
                               void* y_entries, int32_t* tile_queue, size_t tile_queue_ints, void* stream) {
  clear_error();
  return down_impl("mep_swiglu_down", act, n_tokens, top_k, perm, offsets, n_local, max_rows, w_out, nullptr,
                   hidden, inter, dtype, y_entries, tile_queue, tile_queue_ints, stream);
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
                                  void* workspace, size_t workspace_bytes, int32_t* tile_queue,
                                  size_t tile_queue_ints, void* stream) {
  clear_error();
  return grouped_impl("mep_grouped_swiglu", x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_out,
                      nullptr, hidden, inter, dtype, y_entries, workspace, workspace_bytes, tile_queue,
                      tile_queue_ints, stream);
}

extern "C" int mep_grouped_swiglu_slots(const void* x, int64_t n_tokens, int32_t top_k,
                                        const int32_t* perm, const int32_t* offsets, int32_t n_local,
                                        int64_t max_rows, const void* w_in, const void* w_out,
                                        const int32_t* w_slot, int32_t hidden, int32_t inter, int32_t dtype,
                                        void* y_entries, void* workspace, size_t workspace_bytes,
                                        int32_t* tile_queue, size_t tile_queue_ints, void* stream) {
  clear_error();
  MEP_REQUIRE(w_slot != nullptr || n_local == 0 || max_rows == 0, MEP_ERR_INVALID_ARG,
              "mep_grouped_swiglu_slots: null w_slot");
  return grouped_impl("mep_grouped_swiglu_slots", x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in,
                      w_out, w_slot, hidden, inter, dtype, y_entries, workspace, workspace_bytes, tile_queue,
                      tile_queue_ints, stream);
}

extern "C" int mep_grouped_swiglu_combine(const void* x, int64_t n_tokens, int32_t top_k, const int32_t* perm,
                                          const int32_t* offsets, const int32_t* row_of_entry,
                                          const void* topk_gate, const uint8_t* valid_mask, int32_t n_local,
                                          int64_t max_rows, const void* w_in, const void* w_out, int32_t hidden,
                                          int32_t inter, int32_t dtype, void* y_entries, void* workspace,
                                          size_t workspace_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                                          void* out, void* stream) {
  clear_error();
  const char* fn = "mep_grouped_swiglu_combine";
  MEP_REQUIRE(max_rows == n_tokens * static_cast<int64_t>(top_k), MEP_ERR_INVALID_ARG,
              "%s: max_rows %lld must be n_tokens * top_k (every (token, slot) cell)", fn,
              static_cast<long long>(max_rows));
  MEP_REQUIRE(n_tokens == 0 || (row_of_entry && topk_gate && out), MEP_ERR_INVALID_ARG,
              "%s: null row_of_entry / topk_gate / out", fn);
  // the small-batch launch ends with the combine for bf16 top-8 (the other
  // sizes run the experts and mep_combine as two launches, same results)
  CombineParams cp{};
  const bool fuse = dtype == MEP_DTYPE_BF16 && top_k == 8 && n_tokens > 0 && aligned16(out) &&
                    aligned16(y_entries) && max_rows * hidden * 2 < (int64_t(1) << 32);
  if (fuse) {
    cp.gate = static_cast<const uint16_t*>(topk_gate);
    cp.row_of_entry = row_of_entry;
    cp.valid = valid_mask;
    cp.out = static_cast<uint16_t*>(out);
    cp.n_tokens = n_tokens;
    cp.hidden = hidden;
    cp.y_bytes = static_cast<uint32_t>(max_rows * hidden * 2);
    const GiveupTest gt = giveup_test();
    cp.wait_limit = gt.site == MEP_GIVEUP_COMBINE ? gt.polls : sched::kWaitLimit;
    cp.dbg_comb = gt.site == MEP_GIVEUP_COMBINE ? 0 : -1;
  }
  bool combined = false;
  int rc = grouped_impl(fn, x, n_tokens, top_k, perm, offsets, n_local, max_rows, w_in, w_out, nullptr, hidden,
                        inter, dtype, y_entries, workspace, workspace_bytes, tile_queue, tile_queue_ints, stream,
                        fuse ? &cp : nullptr, &combined);
  if (rc != MEP_OK || combined) return rc;
  return mep_combine(y_entries, topk_gate, row_of_entry, valid_mask, n_tokens, top_k, hidden, dtype, out, stream);
}

namespace mep {
namespace {

// The decode layer's one launch, if it applies: bf16, 32 experts, top-8,
// 1..32 tokens, hidden 1024 / 2048 / 4096, inter a multiple of 256, and a
// schedule buffer of dec::words(hidden) ints; otherwise hipErrorNotSupported
// with nothing enqueued.
hipError_t launch_decode(const void* x, const void* w_router, const uint8_t* valid, int64_t n_tokens, int hidden,
                         int E, int k, int dtype, const void* w_in, const void* w_out, int inter, int64_t* topk_idx,
                         void* gate, float* logits, int32_t* counts, int32_t* offsets, int32_t* perm,
                         int32_t* row_of_entry, int64_t* route_counts, void* y_entries, void* dispatch_ws,
                         void* act, int32_t* tile_queue, size_t tile_queue_ints, void* out, hipStream_t stream) {
  if (dtype != MEP_DTYPE_BF16 || E != dec::E || k != 8 || n_tokens < 1 || n_tokens > dec::kMaxTokens ||
      inter % 256 != 0 || static_cast<int64_t>(tile_queue_ints) < dec::words(hidden))
    return hipErrorNotSupported;
  if (hidden != 1024 && hidden != 2048 && hidden != 4096) return hipErrorNotSupported;
  DecodeParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.w_router = static_cast<const uint16_t*>(w_router);
  p.valid = valid;
  p.n_tokens = n_tokens;
  p.topk_idx = topk_idx;
  p.gate = static_cast<uint16_t*>(gate);
  p.logits = logits;
  p.counts = counts;
  p.offsets = offsets;
  p.perm = perm;
  p.row_of_entry = row_of_entry;
  p.route_counts = route_counts;
  p.ws_header = static_cast<uint32_t*>(dispatch_ws);
  p.ws_flags = reinterpret_cast<uint32_t*>(static_cast<char*>(dispatch_ws) + kWsHeaderBytes);
  const int64_t max_rows = n_tokens * k;
  p.g1 = gemm1_params<MEP_DTYPE_BF16, CfgBf16>(x, n_tokens, k, perm, offsets, E, w_in, nullptr, hidden, inter, act);
  p.g2 = gemm2_params<MEP_DTYPE_BF16, CfgBf16>(act, k, perm, offsets, E, max_rows, w_out, nullptr, hidden, inter,
                                               y_entries);
  set_sched(p.g1, tile_queue);
  set_sched(p.g2, tile_queue);
  p.out = static_cast<uint16_t*>(out);
  p.n_g1 = E * (inter / 64);
  p.n_g2 = E * (hidden / 128);
  p.sched = tile_queue;
  const GiveupTest gt = giveup_test();
  p.wait_limit = gt.site == MEP_GIVEUP_CHUNK ? gt.polls : sched::kWaitLimit;
  p.route_wait_limit = gt.site == MEP_GIVEUP_ROUTED ? gt.polls : sched::kWaitLimit;
  p.dbg_routed = gt.site == MEP_GIVEUP_ROUTED ? 0 : -1;
  const dim3 grid(static_cast<unsigned>(p.n_g1 + p.n_g2));   // workgroup 0 also runs GEMM-2 unit n_g2 - 1
  switch (hidden) {
    case 1024: moe_decode_kernel<1><<<grid, skinny::NT, 0, stream>>>(p); break;
    case 2048: moe_decode_kernel<2><<<grid, skinny::NT, 0, stream>>>(p); break;
    default: moe_decode_kernel<4><<<grid, skinny::NT, 0, stream>>>(p); break;
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace mep

extern "C" size_t mep_moe_layer_queue_ints(int64_t n_tokens, int32_t n_experts, int32_t hidden) {
  if (n_tokens < 0 || n_experts <= 0 || hidden <= 0) return 0;
  const int64_t a = mep::sched::words(n_tokens * 8, n_experts), b = mep::dec::words(hidden);
  return static_cast<size_t>(a > b ? a : b);
}

extern "C" int mep_moe_layer(const void* x, const void* w_router, const uint8_t* valid_mask, int64_t n_tokens,
                             int32_t hidden, int32_t n_experts, int32_t top_k, int32_t dtype, const void* w_in,
                             const void* w_out, int32_t inter, int64_t* topk_idx, void* topk_gate, float* logits,
                             int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* row_of_entry,
                             int64_t* route_counts, void* y_entries, void* dispatch_ws, size_t dispatch_ws_bytes,
                             void* experts_ws, size_t experts_ws_bytes, int32_t* tile_queue, size_t tile_queue_ints,
                             void* out, void* stream) {
  clear_error();
  const char* fn = "mep_moe_layer";
  MEP_REQUIRE(n_tokens >= 0, MEP_ERR_INVALID_ARG, "%s: n_tokens < 0", fn);
  MEP_REQUIRE(dispatch_ws != nullptr && experts_ws != nullptr && tile_queue != nullptr, MEP_ERR_INVALID_ARG,
              "%s: null workspace or tile_queue", fn);
  MEP_REQUIRE(dispatch_ws_bytes >= mep_route_dispatch_workspace_size(n_tokens, n_experts), MEP_ERR_WORKSPACE,
              "%s: dispatch workspace %zu B < required %zu B", fn, dispatch_ws_bytes,
              mep_route_dispatch_workspace_size(n_tokens, n_experts));
  const int64_t max_rows = n_tokens * top_k;
  MEP_REQUIRE(experts_ws_bytes >= mep_experts_workspace_size(max_rows, inter, dtype), MEP_ERR_WORKSPACE,
              "%s: experts workspace %zu B < required %zu B", fn, experts_ws_bytes,
              mep_experts_workspace_size(max_rows, inter, dtype));
  if (n_tokens > 0) {
    MEP_REQUIRE(x && w_router && w_in && w_out && topk_idx && topk_gate && counts && offsets && perm &&
                    row_of_entry && y_entries && out,
                MEP_ERR_INVALID_ARG, "%s: null pointer", fn);
    MEP_REQUIRE(aligned16(x) && aligned16(w_in) && aligned16(w_out) && aligned16(experts_ws) &&
                    aligned16(y_entries) && aligned16(out) && aligned16(topk_gate),
                MEP_ERR_INVALID_ARG, "%s: buffers must be 16-byte aligned", fn);
    const hipError_t e = launch_decode(x, w_router, valid_mask, n_tokens, hidden, n_experts, top_k, dtype, w_in, w_out,
                                       inter, topk_idx, topk_gate, logits, counts, offsets, perm, row_of_entry,
                                       route_counts, y_entries, dispatch_ws, experts_ws, tile_queue, tile_queue_ints,
                                       out, static_cast<hipStream_t>(stream));
    if (e == hipSuccess) return MEP_OK;
    MEP_REQUIRE(e == hipErrorNotSupported, MEP_ERR_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  }
  // the two calls: router + dispatch, then the experts ending with the combine
  int rc = mep_route_dispatch(x, w_router, valid_mask, n_tokens, hidden, n_experts, top_k, dtype, topk_idx, topk_gate,
                              logits, counts, offsets, perm, row_of_entry, route_counts, dispatch_ws,
                              dispatch_ws_bytes, stream);
  if (rc != MEP_OK) return rc;
  if (n_tokens == 0) return MEP_OK;
  return mep_grouped_swiglu_combine(x, n_tokens, top_k, perm, offsets, row_of_entry, topk_gate, valid_mask, n_experts,
                                    max_rows, w_in, w_out, hidden, inter, dtype, y_entries, experts_ws,
                                    experts_ws_bytes, tile_queue, tile_queue_ints, out, stream);
}
