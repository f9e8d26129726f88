// MXFP4 matmuls on the gfx950 scaled MFMA: the grouped expert GEMMs g_moe_ggu_mxfp4s[_fused]_k{H} /
// g_moe_gdn_mxfp4s_k{FE} of the reference's MoE prefill chain (S/gen_moe.py:1126-1228), and the dense prefill GEMM
// g_gemm_mxfp4s_{store|swiglu}_f8_m256 (S/gen_mxfp4s.py:50-101, the gfx12 fp8 WMMA counterpart), which is the same
// kernel over dense 64-row tiles of one weight matrix (qmm_gemm_mxfp4):
//
//   gu   act[r, c] = act_fast(sum_k X8[t, k] Wg[e][c, k] + bg[e, c], sum_k X8[t, k] Wu[e][c, k] + bu[e, c]),
//                    t = rowmap[r] / KU
//   dn   ys[r, c]  = sum_k A8[r, k] Wd[e][c, k] + bd[e, c]                             (rows already sorted)
//
// for every row r of every 64-row tile with expert e = tile_info[tile, 0] >= 0 (rows with rowmap[r] < 0 are not
// written; the MXFP8 output of the fused gate/up writes them as codes 0, scale 0); the expert biases are optional (gpt-oss, S/gen_moe.py:958-1007). W is MXFP4 in split planes: nibbles [E, rows, K/2] ("pairs": byte j holds elements 2j, 2j+1) and
// E8M0 scales [E, rows, K/32]. X8 / A8 are MXFP8 activations from qmm_quant_mxfp8: E4M3 codes [rows, K] with one
// E8M0 scale per 32 values along K. fp32 accumulation.
//
// One v_mfma_scale_f32_32x32x64_f8f6f4 per 32 x 32 x 64 block, A = E4M3 activations (format 0), B = E2M1 weights
// (format 4), both with E8M0 block scales applied by the MFMA itself (measured lane layouts on gfx950, half
// h = lane / 32): the E2M1 operand of lane h holds K values 32h .. 32h+31 of the 64-value chunk as 16 bytes, low
// nibble first, which is exactly one 32-value block of the split nibble plane, so weights go from HBM to the MFMA
// without any unpacking, and its scale is that block's E8M0 byte. The E4M3 operand of lane h holds K values
// 16h .. 16h+15 in bytes 0..15 and 32+16h .. 32+16h+15 in bytes 16..31, and its scale is the one of block h; both
// operands therefore see the same two 32-value blocks per chunk.
//
// Weight layouts. kSplit reads the split planes as they are: one load instruction then touches 32 weight rows
// (1440 bytes apart at K = 2880), 32 bytes each, which streams at about 4.5-5 TB/s. kTiled reads the MFMA-tiled
// planes of qmm_tile_mxfp4: the 1 KB tile (row block rb of 32 rows, chunk c of 64 values) holds at bytes
// 16 l .. 16 l + 15 exactly lane l's E2M1 operand (row 32 rb + l % 32, values 64 c + 32 (l / 32) ..), tiles ordered
// (rb, c), so a wave streams one contiguous run of 1 KB loads over K (about 7.4 TB/s for the same bytes); the E8M0
// plane holds per (rb, group of four chunks) 256 bytes, lane l's four scale bytes at 4 l, so one dword load per
// lane brings the scales of four chunks.
//
// Tiling: a workgroup of four waves owns one 64-row expert tile; each wave computes its 64 rows x CB output column
// blocks of 32 over all of K. gu: wave w owns output columns 32 CB w .. 32 CB (w + 1) - 1 of a 128 CB-column block,
// its weight blocks being those columns of the gate and of the up matrix (2 CB x 2 MFMA blocks), so the activation
// is applied in registers. dn: the same columns of the one matrix (CB x 2 MFMA blocks). Wide tiles (tiled planes,
// many rows an expert: gu CB = 2, dn CB = 4, four weight blocks a wave either way) halve or quarter the activation
// bytes a weight byte meets; CB = 1 keeps more workgroups on the weight stream when the experts hold few rows.
// Workgroup b runs on XCD b % 8;
// the live tiles (those with an expert) are cut into eight contiguous ranges, one per XCD, and each XCD walks its
// range in groups of twelve tiles, tile-fastest: the workgroups resident together on an XCD are then the tiles of one
// or two experts on a few column blocks, so an expert's weights come from HBM about once and its other tiles read
// them from that XCD's L2, and a group's activation rows are read by all column blocks while still in L2.
//
// Steps. The E8M0 scales of the tile's 64 activation rows (and, for kSplit, of its 128 + 128 or 128 weight columns),
// K / 32 bytes each, are staged in LDS once; per-step byte loads of split-plane scales through the vector memory
// path cost more than the weight stream (kTiled streams its scales as one dword per four chunks instead). A
// super-step covers kSub 64-value chunks: the tile's activation codes for it are staged in LDS (double-buffered, one
// barrier per super-step) and the weights stream straight into registers DEPTH super-steps ahead.
#include <type_traits>

#include "bfly.hpp"
#include "common.hpp"

using namespace qmm;

namespace {

// Pipeline shape per kernel: DEPTH super-steps of weight loads in flight, SUB 64-value chunks per super-step (one
// barrier each). The down GEMM streams one weight column block per wave (the gate/up GEMM two), so its super-steps
// are twice as long for as many bytes per barrier. Both epilogues store their outputs nontemporally: every
// workgroup stores at its very end, and streamed stores drain during the epilogue instead of as dirty L2 lines at the
// end of the kernel (gate/up -1 us, down -2 us at the gpt-oss-20b shape, T = 256).
#ifndef QMM_MX_DEPTH_GU
#define QMM_MX_DEPTH_GU 2
#endif
#ifndef QMM_MX_SUB_GU
#define QMM_MX_SUB_GU 2
#endif
#ifndef QMM_MX_DEPTH_DN
#define QMM_MX_DEPTH_DN 2
#endif
#ifndef QMM_MX_SUB_DN
#define QMM_MX_SUB_DN 4
#endif
#ifndef QMM_MX_WAVES
#define QMM_MX_WAVES 3            // minimum waves per SIMD the register allocation must allow (3 workgroups per CU)
#endif

constexpr int BM = 64, KC = 64;
constexpr int kTileGroup = 12;   // tiles of a range walked together over the column blocks

enum Kind { kGU = 1, kDN = 2, kGU8 = 3 };   // kGU8: gu with its output quantized to MXFP8
enum Layout { kSplit = 0, kTiled = 1 };
// where the output goes: the grouped GEMMs' sorted f32 rows, or a dense GEMM's y (f32 / bf16, stored or added to);
// a dense kGU is the swiglu GEMM silu(X Wg^T) (X Wu^T) over rows 0 .. M - 1 of x
enum Out { kOutGrouped = 0, kOutF32 = 1, kOutF32Acc = 2, kOutBF16 = 3, kOutBF16Acc = 4 };
typedef __attribute__((ext_vector_type(4))) u32 v4u;   // a native vector: the register rings stay in VGPRs

struct MArgs {
  int N, K;
  int M;                        // dense: rows of x and y
  const u8 *x8, *xs;            // activation codes [rows, K], scales [rows, K/32]
  int x_rows;
  const u8 *wn, *wsc;           // gate (or down) nibbles / scales of expert 0
  const u8 *wn2, *wsc2;         // up nibbles / scales (gu, not fused) or NULL
  int64_t nib_ebytes, sc_ebytes;   // bytes of one expert's nibble / scale plane
  int64_t up_nib_off, up_sc_off;   // fused gu: offset of the up rows inside an expert
  const int32_t *tile_info, *rowmap;
  const float *bias, *bias2;       // per-expert output biases [E, N] (gu: gate, up; dn: bias only) or NULL
  int KU, E, act;
  float *y;
  u8 *y8, *ys8;                    // kGU8: E4M3 codes [rows, N] and E8M0 scales [rows, N/32] of the activation
  int n_blocks, max_tiles;
};

// The sigmoid as v_exp_f32 and v_rcp_f32 (each about 1 ulp; exp overflow gives rcp(inf) = 0, as the division would):
// the epilogue runs once per output at the very end of every workgroup, where an IEEE division and a range-reduced
// expf per value are a measurable tail. The outputs are MXFP8-quantized next (3 mantissa bits).
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

__device__ __forceinline__ float act_fast(int act, float g, float u) {
  if (act == QMM_ACT_SWIGLU_OAI) {
    const float xg = fminf(g, 7.0f);
    const float yu = fminf(fmaxf(u, -7.0f), 7.0f);
    return xg * sigmoid_fast(1.702f * xg) * (yu + 1.0f);
  }
  return g * sigmoid_fast(g) * u;
}

// f(integral_constant<I>) for I = 0 .. N-1, in order: ring slots as compile-time constants
template <class F, int... I>
__device__ __forceinline__ void for_slots(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <class F, int... I>
__device__ __forceinline__ void for_steps(F &&f, int c0, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}, c0), ...);
}

// Element i of an n-element copy into LDS, for every i, 256 threads: kBatch loads in flight per thread before
// their stores (a plain loop would wait for each load before the next). get(i) loads element i (i < n).
template <int kBatch = 8, class T, class G>
__device__ __forceinline__ void batched_copy(T *dst, int64_t n, int tid, G &&get) {
  for (int64_t b = 0; b < n; b += kBatch * 256) {
    T v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int64_t i = b + tid + 256 * q;
      v[q] = get(i < n ? i : n - 1);
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int64_t i = b + tid + 256 * q;
      if (i < n) dst[i] = v[q];
    }
  }
}

// copies n bytes from global memory to LDS with the widest loads the alignment of both allows
__device__ __forceinline__ void copy_to_lds(u8 *dst, const u8 *src, int64_t n, int tid) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | (uintptr_t)n;
  if ((al & 15) == 0) {
    const v4u *s = reinterpret_cast<const v4u *>(src);
    batched_copy(reinterpret_cast<v4u *>(dst), n / 16, tid, [&](int64_t i) { return s[i]; });
  } else if ((al & 3) == 0) {
    const u32 *s = reinterpret_cast<const u32 *>(src);
    batched_copy(reinterpret_cast<u32 *>(dst), n / 4, tid, [&](int64_t i) { return s[i]; });
  } else {
    batched_copy(dst, n, tid, [&](int64_t i) { return src[i]; });
  }
}

template <int KIND, int LAYOUT, int DEPTH, int kSub, int OUT, int CB, int WAVES>
__global__ __launch_bounds__(256, WAVES) void mxfp4_grouped_kernel(MArgs a) {
  constexpr bool DENSE = OUT != kOutGrouped;
  static_assert(!(DENSE && KIND == kGU8), "the MXFP8 epilogue writes the grouped activation");
  static_assert(CB == 1 || LAYOUT == kTiled, "several column blocks a wave on the tiled planes only");
  constexpr int APITCH = kSub * KC + 16;     // activation bytes per LDS row (16-byte aligned rows)
  constexpr bool GU = KIND != kDN;
  // CB output column blocks of 32 per wave; its 32-column weight blocks: gu the CB gate blocks, then the same CB
  // blocks of the up matrix; dn the CB blocks
  constexpr int NJ = GU ? 2 * CB : CB;
  constexpr int WC = 32 * CB;                // output columns per wave
  constexpr int BN = 4 * WC;                 // output columns per workgroup
  // the activation double buffer; kGU8 reuses it after the loop for its f32 output, 32 rows at a time
  constexpr int OPITCH = BN + 4;   // floats per output row: the 4-float skew spreads a column's rows over the banks
  constexpr int kStage = 2 * BM * APITCH, kOut = KIND == kGU8 ? 32 * OPITCH * 4 : 0;
  __shared__ __align__(16) u8 smem[kStage > kOut ? kStage : kOut];
  auto As = reinterpret_cast<u8 (*)[BM][APITCH]>(smem);
  __shared__ int src_row[BM];
  __shared__ int live_end;
  // E8M0 scales staged once: the tile's 64 activation rows and, for kSplit, the block's weight columns (gu: 128 gate
  // then 128 up columns; dn: 128 columns), K / 32 bytes each.
  extern __shared__ __align__(16) u8 dyn_lds[];
  u8 *Asc = dyn_lds, *Wsc = dyn_lds + BM * (a.K / 32);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- which tile and column block: the live tiles [0, L) (L = 1 + the last tile with an expert) in eight
  //      contiguous ranges, range x on XCD x, walked in groups of kTileGroup tiles (below)
  int L = a.max_tiles;   // dense: every 64-row tile of x
  if constexpr (!DENSE) {
    if (tid == 0) live_end = 0;
    __syncthreads();
    {
      int last = 0;
      for (int t = tid; t < a.max_tiles; t += 256)
        if (a.tile_info[2 * t] >= 0) last = t + 1;
      if (last) atomicMax(&live_end, last);
    }
    __syncthreads();
    L = live_end;
  }
  const int xcd = (int)(blockIdx.x & 7), xi = (int)(blockIdx.x >> 3);
  const int t_begin = (int)(((int64_t)xcd * L) >> 3), t_end = (int)(((int64_t)(xcd + 1) * L) >> 3);
  const int cnt = t_end - t_begin;
  if (cnt <= 0 || xi >= cnt * a.n_blocks) return;
  // the range in groups of kTileGroup tiles, each group walked tile-fastest over every column block before the next:
  // a group's activation rows (12 x 64 rows) are then read by its column blocks while they are still in the XCD's
  // L2, where one sweep of all the range's tiles per column block lets the weight stream evict them in between
  // (gpt-oss-20b at T = 4096, HBM reads a launch: gate/up 878 -> 727 MB, down 454 -> 386 MB; times within 2 %)
  int tile, cbk;
  if (cnt > kTileGroup) {
    const int per = kTileGroup * a.n_blocks, g = xi / per, r = xi - g * per, gt0 = g * kTileGroup;
    const int gn = cnt - gt0 < kTileGroup ? cnt - gt0 : kTileGroup;
    tile = t_begin + gt0 + r % gn;
    cbk = r / gn;
  } else {
    tile = t_begin + xi % cnt;
    cbk = xi / cnt;
  }
  const int N = a.N, K = a.K, C = K / KC;
  const int n0 = cbk * BN, m0 = tile * BM;
  // the tile's expert and row map are loaded together; the weight stream starts as soon as the expert is known,
  // before the row map, the activation rows and their scales (every workgroup starts at once, so each dependent
  // round trip before the first weight load is time the HBM idles)
  int rm, expert = 0;
  if constexpr (DENSE) {
    rm = tid < BM && m0 + tid < a.M ? m0 + tid : -1;
  } else {
    rm = tid < BM ? a.rowmap[m0 + tid] : -1;
    expert = a.tile_info[2 * tile];
    if (expert < 0) return;
    expert = expert >= a.E ? a.E - 1 : expert;
  }

  auto clampc = [&](int c) __attribute__((always_inline)) { return c < C ? c : C - 1; };
  const int SK = K / 32;           // scale bytes per row
  const int C4 = (C + 3) >> 2;     // kTiled: groups of four chunks per row block

  // ---- weights: this lane's two columns (gu: one column of the gate and of the up matrix) and K half
  const int h = lane >> 5, lc = lane & 31;
  const int col = n0 + WC * wave + lc;       // the lane's output column (dn: of its first block)
  // a wave whose columns all lie past N (the last column block of a matrix whose N is not a multiple of the
  // block) keeps its loads and barriers but issues no MFMA: its outputs are never stored
  const bool wlive = n0 + WC * wave < N;
  const u8 *nbj[NJ], *sbj[NJ];   // the matrix of weight block j
  {
    const u8 *gn = a.wn + (int64_t)expert * a.nib_ebytes, *gs = a.wsc + (int64_t)expert * a.sc_ebytes;
    const u8 *un = gn, *us = gs;
    if constexpr (GU) {
      if (a.wn2) { un = a.wn2 + (int64_t)expert * a.nib_ebytes; us = a.wsc2 + (int64_t)expert * a.sc_ebytes; }
      else { un = gn + a.up_nib_off; us = gs + a.up_sc_off; }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      nbj[j] = j < CB ? gn : un;
      sbj[j] = j < CB ? gs : us;
    }
  }
  // the lane's weight stream: split -- its column's row at K half h; tiled -- lane slot of the wave's row block
  // (waves past the last column read the last block and store nothing)
  const u8 *wcn[NJ];
  const u8 *wcs[NJ];
  int wrow[NJ];   // kSplit: the lane's weight columns as rows of Wsc (gu: the gate block, then the up block)
  if constexpr (LAYOUT == kTiled) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      int rb = (n0 >> 5) + CB * wave + j % CB;
      rb = rb < (N >> 5) ? rb : (N >> 5) - 1;
      wcn[j] = nbj[j] + (int64_t)rb * C * 1024 + 16 * lane;
      wcs[j] = sbj[j] + (int64_t)rb * C4 * 256 + 4 * lane;
      wrow[j] = 0;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      wcn[j] = nbj[j] + (int64_t)(col < N ? col : N - 1) * (K / 2) + 16 * h;
      wcs[j] = nullptr;
      wrow[j] = 128 * j + 32 * wave + lc;
    }
  }
  constexpr int CSTRIDE = LAYOUT == kTiled ? 1024 : 32;   // bytes between consecutive chunks of the lane's stream

  f32x16 acc[2][NJ];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Rings DEPTH super-steps deep. kTiled also streams the weight blocks' scale dwords, one per group of four chunks
  // (kSub divides four): with four chunks a super-step, one a ring slot; with fewer (SPG = 4 / kSub super-steps a
  // dword), each dword is loaded once, SPG super-steps ahead of its group, into one of two group slots, and the loop
  // runs 2 SPG super-steps an iteration so that every slot index is a constant (one dword load per weight block and
  // super-step was a sixth of the bytes the workgroup moves through its vector memory path, and measurably slower).
  constexpr int SPG = LAYOUT == kTiled && kSub < 4 ? 4 / kSub : 0;
  constexpr int U = SPG ? 2 * SPG : DEPTH;   // super-steps per loop iteration
  static_assert(U % DEPTH == 0, "an iteration holds whole turns of the rings");
  v4u aring[DEPTH][kSub], bring[DEPTH][kSub][NJ];
  u32 sring[SPG ? 2 : DEPTH][NJ];
  auto load_s = [&](int slot, int g) __attribute__((always_inline)) {
    g = g < C4 ? g : C4 - 1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) sring[slot][j] = *reinterpret_cast<const u32 *>(wcs[j] + (int64_t)g * 256);
  };
  auto load_b = [&](int slot, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < kSub; ++i)
        bring[slot][i][j] = *reinterpret_cast<const v4u *>(wcn[j] + (int64_t)clampc(kSub * st + i) * CSTRIDE);
    if constexpr (LAYOUT == kTiled && !SPG) load_s(slot, st);
  };
  // the weight stream: the first super-step (the others follow the activation staging, below)
  load_b(0, 0);
  if constexpr (SPG) load_s(0, 0);

  int my_src = -1;
  if (tid < BM) {
    int src;
    if constexpr (DENSE) {
      src = rm;
    } else if constexpr (GU) {
      src = rm >= 0 ? rm / a.KU : -1;
      src = src < a.x_rows ? src : -1;
    } else {
      src = rm >= 0 ? m0 + tid : -1;
    }
    src_row[tid] = src;
    my_src = src;
  }
  // whether rows 32..63 hold a live row: if not, the upper 32-row MFMA blocks are skipped (their outputs are the
  // zeros of dead rows) -- expert tiles of prefill batches are often less than half full
  const bool upper = __syncthreads_or(tid >= 32 && my_src >= 0) != 0;

  // ---- activation staging: per super-step (kSub chunks of 64 values) thread tid carries 16 bytes of every chunk of
  //      row tid / 4 (piece tid % 4 of each chunk)
  const int arow_i = tid >> 2, apart = tid & 3;
  // a buffer resource over the activation codes: a dead row's offset lies past the end (0x80000000) and loads
  // zeros without touching memory, so a tile of few live rows fetches only those
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<u8 *>(a.x8), (short)0, (int)((int64_t)a.x_rows * K), 0x00020000);
  const u32 aoff = src_row[arow_i] >= 0 ? (u32)((int64_t)src_row[arow_i] * K + 16 * apart) : 0x80000000u;
  auto load_a = [&](int slot, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSub; ++i)
      aring[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)(aoff + (u32)(clampc(kSub * st + i) * KC)), 0, 0);
  };
  auto stage = [&](int slot, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSub; ++i) *reinterpret_cast<v4u *>(&As[buf][arow_i][KC * i + 16 * apart]) = aring[slot][i];
  };
  // the first activation chunk and the activation rows' scales (a gathered row each; up to K = 4096 one batch of
  // loads) are issued together and land one round trip after the first weights; then the chunk is staged and the
  // next ones go into the ring. kSplit also stages the weight column blocks' scales.
  //
  // The loads still in flight when the loop starts are issued in the order one loop iteration issues them
  // (activations of super-step j + 1 + DEPTH, then weights of super-step j + DEPTH, for j = -DEPTH + 1 .. -1). The
  // compiler places one s_waitcnt per wait point, valid on both paths into the loop header; a prologue whose last
  // loads came in another order would make the loop's waits stricter than the loop itself needs (in the extreme,
  // every weight load of the previous super-step waited on before the activations are staged).
  load_a(0, 0);
  if constexpr (DEPTH > 1) load_a(1, 1);
  {
    // the rows' scales: four threads a row (BM x 4 = 256), each every fourth 2-byte piece of its row (K / 32 is
    // even), eight loads in flight before their stores; no division per piece (a 64-bit one took about 130
    // instructions a piece, some 2000 a thread in every workgroup's prologue)
    static_assert(BM * 4 == 256, "four threads a scale row");
    const int r = tid >> 2, q0 = tid & 3, n2 = SK / 2;
    const u16 *sp = reinterpret_cast<const u16 *>(a.xs + (int64_t)(src_row[r] >= 0 ? src_row[r] : 0) * SK);
    u16 *dp = reinterpret_cast<u16 *>(Asc + r * SK);
    for (int b = q0; b < n2; b += 32) {
      u16 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = sp[b + 4 * q < n2 ? b + 4 * q : n2 - 1];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (b + 4 * q < n2) dp[b + 4 * q] = v[q];
    }
  }
  if constexpr (LAYOUT == kSplit) {
    const int cols = N - n0 < BN ? N - n0 : BN;   // columns past N are never stored
#pragma unroll
    for (int m = 0; m < NJ; ++m) copy_to_lds(Wsc + m * BN * SK, sbj[m] + (int64_t)n0 * SK, (int64_t)cols * SK, tid);
  }
  stage(0, 0);
  if constexpr (DEPTH == 1) load_a(0, 1);
  for_slots([&](auto uc) {
    constexpr int j = decltype(uc)::value;
    if constexpr (j > 0) {
      load_a((j + 1) % DEPTH, j + 1);
      load_b(j, j);
    }
  }, std::make_integer_sequence<int, DEPTH>{});
  __syncthreads();

  // The super-step count is rounded up to a multiple of DEPTH. A padding chunk (c >= C) runs with both E8M0 scales
  // 0: its products are at most 448 * 6 * 2^-254, far below the smallest f32 subnormal, so they add exactly zero.
  // Each super-step is instantiated with its ring slots as constants (integral_constant), so the rings stay in
  // registers; the super-steps past the last chunk that rounding the count up to U adds skip their MFMAs (a uniform
  // branch) but keep their loads and barrier, so the waits are the same in every iteration.
  const int S = (C + kSub - 1) / kSub;
  const int SP = (S + U - 1) / U * U;
  auto step = [&](auto uc, int s0) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    constexpr int ub = u % DEPTH;              // ring slot
    constexpr int nx = (u + 1) % DEPTH;
    constexpr int us = SPG ? u / SPG : ub;     // scale slot
    const int st = s0 + u;
    const int buf = st & 1;
#pragma unroll
    for (int i = 0; i < kSub && st < S && wlive; ++i) {
      const int c = kSub * st + i;
      const bool live = c < C;
      const int sc_off = 2 * clampc(c) + h;   // the lane's E8M0 byte of this chunk in a scale row
      auto afrag = [&](int ii, i32x8 &af, int &sa) __attribute__((always_inline)) {
        const v4u v0 = *reinterpret_cast<const v4u *>(&As[buf][32 * ii + lc][KC * i + 16 * h]);
        const v4u v1 = *reinterpret_cast<const v4u *>(&As[buf][32 * ii + lc][KC * i + 32 + 16 * h]);
        af = i32x8{(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
        sa = live ? Asc[(32 * ii + lc) * SK + sc_off] : 0;
      };
      i32x8 bf[NJ];
      int sb[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const v4u bv = bring[ub][i][j];
        bf[j] = i32x8{(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w, 0, 0, 0, 0};
        if constexpr (LAYOUT == kTiled) sb[j] = live ? (int)((sring[us][j] >> (8 * (c & 3))) & 255u) : 0;
        else sb[j] = live ? Wsc[wrow[j] * SK + sc_off] : 0;
      }
      {
        i32x8 af;
        int sa;
        afrag(0, af, sa);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[0][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af, bf[j], acc[0][j], 0, 4, 0, sa, 0, sb[j]);
      }
      if (upper) {
        i32x8 af;
        int sa;
        afrag(1, af, sa);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[1][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af, bf[j], acc[1][j], 0, 4, 0, sa, 0, sb[j]);
      }
    }
    // Vector loads complete in issue order for the s_waitcnt counter, so a wait on a load also waits on every load
    // issued before it. The activation chunk staged here (issued DEPTH super-steps ago, ahead of that super-step's
    // weights) is therefore waited on before this super-step's loads are issued, and its own activation load goes
    // out ahead of its weight load: that wait never covers the weights of the last DEPTH - 1 super-steps, which stay
    // in flight across it.
    stage(nx, buf ^ 1);
    load_a(nx, st + 1 + DEPTH);
    load_b(ub, st + DEPTH);
    if constexpr (SPG && u % SPG == 0) load_s((us + 1) % 2, st / SPG + 1);   // the next group's dwords
    __syncthreads();
  };
  for (int s0 = 0; s0 < SP; s0 += U)
    for_steps(step, s0, std::make_integer_sequence<int, U>{});

  if constexpr (KIND == kGU8) {
    // The activation quantized to MXFP8 as qmm_quant_mxfp8 quantizes it. Per 32-row half of the tile, the f32
    // activations go to LDS (the activation buffers are free after the loop's last barrier); then threads 2 b and
    // 2 b + 1 own 32-value block b of a row (BN / 32 blocks a row), 16 values each: their maximum is one lane
    // exchange, and each thread's 16 E4M3 codes leave as one 16-byte store. Dead rows quantize zeros: codes 0, scale
    // byte 0.
    float *Of = reinterpret_cast<float *>(smem);
    float bg[CB], bu[CB];
#pragma unroll
    for (int cc = 0; cc < CB; ++cc) {
      const int64_t bo = (int64_t)expert * N + (col + 32 * cc < N ? col + 32 * cc : N - 1);
      bg[cc] = a.bias ? a.bias[bo] : 0.f;
      bu[cc] = a.bias2 ? a.bias2[bo] : 0.f;
    }
    const int cols = N - n0 < BN ? N - n0 : BN;   // a multiple of 32
    constexpr int QT = BN / 16, QR = 256 / QT;    // threads per row, rows per round
    const int blk = (tid % QT) >> 1, part = tid & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i) __syncthreads();   // the first half's reads are done before the second half overwrites them
#pragma unroll
      for (int cc = 0; cc < CB; ++cc)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int lr = 8 * (r >> 2) + 4 * h + (r & 3);
          Of[lr * OPITCH + WC * wave + 32 * cc + lc] =
              src_row[32 * i + lr] >= 0 ? act_fast(a.act, acc[i][cc][r] + bg[cc], acc[i][CB + cc][r] + bu[cc]) : 0.f;
        }
      __syncthreads();
#pragma unroll
      for (int q0 = 0; q0 < 32; q0 += QR) {
        const int qrow = q0 + tid / QT;
        const f32x4 *src = reinterpret_cast<const f32x4 *>(Of + qrow * OPITCH + 32 * blk + 16 * part);
        f32x4 v[4];
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = src[q];
          m = fmaxf(m, fmaxf(fmaxf(fabsf(v[q][0]), fabsf(v[q][1])), fmaxf(fabsf(v[q][2]), fabsf(v[q][3]))));
        }
        m = fmaxf(m, xshfl<1>(m));
        const int sx = mxfp8_exponent(m);
        v4u code;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          code[q] = (u32)e4m3_pack2<true>(v[q][2], v[q][3], sx, e4m3_pack2<false>(v[q][0], v[q][1], sx, 0));
        const int64_t orow = m0 + 32 * i + qrow;
        if (32 * blk < cols) {
          __builtin_nontemporal_store(code, reinterpret_cast<v4u *>(a.y8 + orow * N + n0 + 32 * blk + 16 * part));
          if (!part) a.ys8[orow * (N / 32) + n0 / 32 + blk] = (u8)(sx + 127);
        }
      }
    }
    return;
  }
  if (col >= N) return;
  if constexpr (DENSE) {
#pragma unroll
    for (int cc = 0; cc < CB; ++cc) {
      const int cj = col + 32 * cc;
      if (cj >= N) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
          if (row >= a.M) continue;
          float v;
          if constexpr (GU) v = act_fast(QMM_ACT_SILU, acc[i][cc][r], acc[i][CB + cc][r]);
          else v = acc[i][cc][r];
          const int64_t o = (int64_t)row * N + cj;
          if constexpr (OUT == kOutF32 || OUT == kOutF32Acc) {
            if constexpr (OUT == kOutF32Acc) v += a.y[o];
            a.y[o] = v;
          } else {
            u16 *yb = reinterpret_cast<u16 *>(a.y);
            if constexpr (OUT == kOutBF16Acc) v += bf16_to_f32(yb[o]);
            yb[o] = (u16)f32_to_bf16_rne(v);
          }
        }
    }
    return;
  }
  float bg[CB], bu[CB];
#pragma unroll
  for (int cc = 0; cc < CB; ++cc) {
    const int64_t bo = (int64_t)expert * N + (col + 32 * cc < N ? col + 32 * cc : N - 1);
    bg[cc] = a.bias ? a.bias[bo] : 0.f;
    bu[cc] = (GU && a.bias2) ? a.bias2[bo] : 0.f;
  }
  // the bias loads complete here, once: otherwise every store below, each behind its own row branch, waits for
  // them with vmcnt(0), which also waits for the stores before it
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
#pragma unroll
  for (int cc = 0; cc < CB; ++cc) {
    const int cj = col + 32 * cc;
    if (cj >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (src_row[lr] < 0) continue;   // a row without an assignment is not written
        float v;
        if constexpr (GU) v = act_fast(a.act, acc[i][cc][r] + bg[cc], acc[i][CB + cc][r] + bu[cc]);
        else v = acc[i][cc][r] + bg[cc];
        __builtin_nontemporal_store(v, a.y + (int64_t)(m0 + lr) * N + cj);
      }
  }
}

constexpr int kMaxK = 12288;   // the workgroup stages (64 + 256) x K / 32 scale bytes in LDS

// CB output column blocks of 32 per wave (CB > 1: tiled planes): 128 CB output columns a workgroup. The register
// allocation allows three workgroups a CU while the accumulators take at most two weight blocks a wave, else two.
template <int KIND, int LAYOUT, int OUT = kOutGrouped, int CB = 1>
int launch(const MArgs &a0, hipStream_t s) {
  MArgs a = a0;
  a.n_blocks = (a.N + 128 * CB - 1) / (128 * CB);
  constexpr int NJ = KIND == kDN ? CB : 2 * CB;
  constexpr int kWaves = NJ <= 2 ? QMM_MX_WAVES : 2;
  constexpr int kDepth = KIND == kDN ? QMM_MX_DEPTH_DN : QMM_MX_DEPTH_GU;
  // several weight blocks a wave shorten the super-steps to keep the bytes per barrier
  constexpr int kSub0 = (KIND == kDN ? QMM_MX_SUB_DN : QMM_MX_SUB_GU) / CB;
  constexpr int kSub = kSub0 > 0 ? kSub0 : 1;
  constexpr int kRows = BM + (LAYOUT == kSplit ? (KIND != kDN ? 256 : 128) : 0);   // scale rows staged in LDS
  const dim3 grid((unsigned)(8 * a.n_blocks * ((a.max_tiles + 7) / 8)));
  const size_t dyn = (size_t)kRows * (a.K / 32);
  const void *fn = reinterpret_cast<const void *>(&mxfp4_grouped_kernel<KIND, LAYOUT, kDepth, kSub, OUT, CB, kWaves>);
  if constexpr ((size_t)kRows * (kMaxK / 32) > 32768) {
    // beyond the default dynamic LDS limit: raised once per device to the largest K this kernel takes, so the order
    // of calls with different K does not matter
    if (dyn > 32768) {
      static std::atomic<unsigned> raised{0};
      if (int st = raise_dyn_lds(fn, kRows * (kMaxK / 32), raised)) return st;
    }
  }
  mxfp4_grouped_kernel<KIND, LAYOUT, kDepth, kSub, OUT, CB, kWaves><<<grid, 256, dyn, s>>>(a);
  return launch_status();
}

// Column blocks a wave of the grouped GEMMs on tiled planes: four weight blocks a wave (gate/up two column blocks of
// each matrix, down four of its one; two workgroups a CU instead of three) once the table holds, on average, at
// least kWideRows rows an expert (the down GEMM; kWideRowsGU the gate/up GEMM). max_tiles - E tiles hold the
// assignments: the bucket sizes max_tiles as A / 64 + E. Below that the one-block kernels keep more workgroups in
// flight on the weight stream. (gpt-oss-20b at T = 1024, 128 rows an expert: gate/up 111 µs wide, 117 with one
// block; down with four blocks 60 / 184 µs at T = 1024 / 4096, with two 67 / 191.)
constexpr int kWideRows = 64, kWideRowsGU = 128;
inline bool wide_tiles(int64_t max_tiles, int E, int rows) { return (max_tiles - E) * BM >= (int64_t)rows * E; }

// MFMA-tiled planes from split planes (a byte permutation): one thread per 16-byte lane slot of a 1 KB tile, and
// per (row block, chunk group) the 64 lanes' four scale bytes. Chunks past K in the last group get scale 0.
__global__ void tile_mxfp4_kernel(const u8 *__restrict__ nib, const u8 *__restrict__ sc, int64_t rows, int K,
                                  u8 *__restrict__ nib_t, u8 *__restrict__ sc_t) {
  const int C = K / KC, C4 = (C + 3) >> 2;
  const int64_t slots = rows / 32 * C * 64;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < slots) {
    const int l = (int)(i & 63);
    const int64_t tile = i >> 6, rb = tile / C;
    const int c = (int)(tile % C);
    const int64_t row = 32 * rb + (l & 31);
    const uint4 v = *reinterpret_cast<const uint4 *>(nib + row * (K / 2) + 32 * c + 16 * (l >> 5));
    *reinterpret_cast<uint4 *>(nib_t + 16 * i) = v;
  }
  const int64_t sslots = rows / 32 * C4 * 64;
  if (i < sslots) {
    const int l = (int)(i & 63);
    const int64_t grp = i >> 6, rb = grp / C4;
    const int g = (int)(grp % C4);
    const int64_t row = 32 * rb + (l & 31);
    u32 w = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = 4 * g + q;
      if (c < C) w |= (u32)sc[row * (K / 32) + 2 * c + (l >> 5)] << (8 * q);
    }
    *reinterpret_cast<u32 *>(sc_t + 4 * i) = w;
  }
}

// f32 values of MFMA-tiled planes, one thread per 32-value block (row r, block b): its 16 bytes sit in lane slot
// 32 (b % 2) + r % 32 of tile (r / 32, b / 2), its E8M0 byte at byte (b / 2) % 4 of that lane's scale dword.
__global__ void dequant_mxfp4t_kernel(const u8 *__restrict__ nib_t, const u8 *__restrict__ sc_t, int64_t rows, int K,
                                      float *__restrict__ out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) {
    const float m[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    lut[threadIdx.x] = threadIdx.x < 8 ? m[threadIdx.x] : -m[threadIdx.x - 8];
  }
  __syncthreads();
  const int C = K / KC, C4 = (C + 3) >> 2, NB = K / 32;
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= rows * NB) return;
  const int64_t r = gi / NB;
  const int b = (int)(gi % NB), c = b >> 1, l = 32 * (b & 1) + (int)(r & 31);
  const int64_t rb = r >> 5;
  const u8 *q = nib_t + ((rb * C + c) * 64 + l) * 16;
  const float s = e8m0_scale(sc_t[((rb * C4 + (c >> 2)) * 64 + l) * 4 + (c & 3)]);
  float *o = out + gi * 32;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const u32 v = q[j];
    o[2 * j] = lut[v & 15u] * s;
    o[2 * j + 1] = lut[v >> 4] * s;
  }
}

}  // namespace

int64_t qmm_mxfp4t_scale_bytes(int64_t rows, int64_t k) {
  if (rows <= 0 || rows % 32 || k <= 0 || k % 64) return 0;
  return rows / 32 * ((k / 64 + 3) / 4) * 256;
}

// The MXFP4 paths of qmm_moe_grouped: split planes (tiled = 0) or MFMA-tiled planes (tiled = 1).
int qmm_grouped_mxfp4(int tiled, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E, int KU,
                      const int32_t *tile_info, const int32_t *rowmap, const void *x, const void *x_scales,
                      int64_t x_rows, const void *w, const void *ws, const void *w2, const void *ws2,
                      const float *bias, const float *bias2, float *y, uint8_t *y8, uint8_t *ys8, hipStream_t s) {
  if (k % 64 || k > kMaxK) return QMM_ERR_SHAPE;   // the workgroup stages (64 + 256) x K / 32 scale bytes in LDS
  if (tiled && n % 32) return QMM_ERR_SHAPE;       // tiled planes hold whole 32-row blocks
  if (x_rows * k >= (1ll << 31)) return QMM_ERR_SHAPE;   // activation rows are addressed by a 32-bit buffer offset
  if (!x_scales || !ws) return QMM_ERR_NULL;
  if (!aligned(x_scales, 2)) return QMM_ERR_ALIGN;
  if (!aligned(x, 16) || !aligned(w, 16) || (w2 && !aligned(w2, 16))) return QMM_ERR_ALIGN;
  if (tiled && (!aligned(ws, 4) || (ws2 && !aligned(ws2, 4)))) return QMM_ERR_ALIGN;
  const bool out8 = y8 != nullptr;   // gu with the activation quantized to MXFP8 in the epilogue
  if (out8 && (mode != 0 || n % 32 || !ys8)) return mode != 0 ? QMM_ERR_RANGE : (ys8 ? QMM_ERR_SHAPE : QMM_ERR_NULL);
  if (out8 && !aligned(y8, 16)) return QMM_ERR_ALIGN;
  if (mode == 0 && !fused && (!w2 || !ws2)) return QMM_ERR_NULL;
  MArgs a{};
  a.N = (int)n; a.K = (int)k;
  a.x8 = static_cast<const u8 *>(x); a.xs = static_cast<const u8 *>(x_scales); a.x_rows = (int)x_rows;
  a.wn = static_cast<const u8 *>(w); a.wsc = static_cast<const u8 *>(ws);
  a.tile_info = tile_info; a.rowmap = rowmap; a.KU = KU; a.E = E; a.act = act; a.y = y; a.y8 = y8; a.ys8 = ys8;
  a.bias = bias; a.bias2 = mode == 0 ? bias2 : nullptr;
  a.max_tiles = (int)max_tiles;
  const bool wide = tiled && wide_tiles(max_tiles, E, mode == 0 ? kWideRowsGU : kWideRows);
  const int64_t nrow = k / 2;                                        // nibble bytes per row (both layouts)
  const int64_t srow = tiled ? qmm_mxfp4t_scale_bytes(32, k) / 32 : k / 32;   // scale bytes per row
  if (mode == 0) {
    if (!fused && (!w2 || !ws2)) return QMM_ERR_NULL;
    a.nib_ebytes = nrow * n * (fused ? 2 : 1);
    a.sc_ebytes = srow * n * (fused ? 2 : 1);
    a.up_nib_off = fused ? nrow * n : 0;
    a.up_sc_off = fused ? srow * n : 0;
    a.wn2 = fused ? nullptr : static_cast<const u8 *>(w2);
    a.wsc2 = fused ? nullptr : static_cast<const u8 *>(ws2);
    if (wide) return out8 ? launch<kGU8, kTiled, kOutGrouped, 2>(a, s) : launch<kGU, kTiled, kOutGrouped, 2>(a, s);
    if (out8) return tiled ? launch<kGU8, kTiled>(a, s) : launch<kGU8, kSplit>(a, s);
    return tiled ? launch<kGU, kTiled>(a, s) : launch<kGU, kSplit>(a, s);
  }
  a.nib_ebytes = nrow * n;
  a.sc_ebytes = srow * n;
  if (wide) return launch<kDN, kTiled, kOutGrouped, 4>(a, s);
  return tiled ? launch<kDN, kTiled>(a, s) : launch<kDN, kSplit>(a, s);
}

// The dense prefill GEMM on MXFP4 weights (split planes or MFMA-tiled planes): the grouped kernels over dense
// 64-row tiles of x, one weight matrix (store / acc) or a gate and an up matrix (swiglu).
extern "C" int qmm_gemm_mxfp4(int fmt, int mode, int64_t rows, int64_t k, int64_t n, const void *x,
                              const void *x_scales, const void *w, const void *ws, const void *w2, const void *ws2,
                              void *y, int y_dtype, qmm_stream_t stream) {
  if (fmt != QMM_MXFP4S && fmt != QMM_MXFP4T) return QMM_ERR_FORMAT;
  if (mode != QMM_GEMM_STORE && mode != QMM_GEMM_ACC && mode != QMM_GEMM_SWIGLU) return QMM_ERR_RANGE;
  if (y_dtype != QMM_F32 && y_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (!x || !x_scales || !w || !ws || !y || (mode == QMM_GEMM_SWIGLU && (!w2 || !ws2))) return QMM_ERR_NULL;
  if (rows <= 0 || k <= 0 || n <= 0 || k % 64 || k > kMaxK || rows > (1 << 24) || n > (1 << 24)) return QMM_ERR_SHAPE;
  const bool tiled = fmt == QMM_MXFP4T;
  if (tiled && n % 32) return QMM_ERR_SHAPE;        // tiled planes hold whole 32-row blocks
  if (rows * k >= (1ll << 31)) return QMM_ERR_SHAPE;   // activation rows are addressed by a 32-bit buffer offset
  if (!aligned(x, 16) || !aligned(x_scales, 2) || !aligned(w, 16) || (w2 && !aligned(w2, 16)) || !aligned(y, 4))
    return QMM_ERR_ALIGN;
  if (tiled && (!aligned(ws, 4) || (ws2 && !aligned(ws2, 4)))) return QMM_ERR_ALIGN;
  MArgs a{};
  a.N = (int)n; a.K = (int)k; a.M = (int)rows;
  a.x8 = static_cast<const u8 *>(x); a.xs = static_cast<const u8 *>(x_scales); a.x_rows = (int)rows;
  a.wn = static_cast<const u8 *>(w); a.wsc = static_cast<const u8 *>(ws);
  a.wn2 = static_cast<const u8 *>(w2); a.wsc2 = static_cast<const u8 *>(ws2);
  a.E = 1; a.KU = 1; a.act = QMM_ACT_SILU; a.y = static_cast<float *>(y);
  a.max_tiles = (int)((rows + BM - 1) / BM);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = y_dtype == QMM_BF16;
  if (mode == QMM_GEMM_SWIGLU) {
    if (bf) return tiled ? launch<kGU, kTiled, kOutBF16>(a, s) : launch<kGU, kSplit, kOutBF16>(a, s);
    return tiled ? launch<kGU, kTiled, kOutF32>(a, s) : launch<kGU, kSplit, kOutF32>(a, s);
  }
  if (mode == QMM_GEMM_ACC) {
    if (bf) return tiled ? launch<kDN, kTiled, kOutBF16Acc>(a, s) : launch<kDN, kSplit, kOutBF16Acc>(a, s);
    return tiled ? launch<kDN, kTiled, kOutF32Acc>(a, s) : launch<kDN, kSplit, kOutF32Acc>(a, s);
  }
  if (bf) return tiled ? launch<kDN, kTiled, kOutBF16>(a, s) : launch<kDN, kSplit, kOutBF16>(a, s);
  return tiled ? launch<kDN, kTiled, kOutF32>(a, s) : launch<kDN, kSplit, kOutF32>(a, s);
}

extern "C" int qmm_tile_mxfp4(const void *nibbles, const void *scales, int64_t rows, int64_t k, void *nib_t,
                              void *sc_t, qmm_stream_t stream) {
  if (!nibbles || !scales || !nib_t || !sc_t) return QMM_ERR_NULL;
  if (rows <= 0 || rows % 32 || k <= 0 || k % 64 || k > (1 << 30)) return QMM_ERR_SHAPE;
  if (!aligned(nibbles, 16) || !aligned(nib_t, 16) || !aligned(sc_t, 4)) return QMM_ERR_ALIGN;
  const int64_t slots = rows / 32 * (k / 64) * 64;   // >= the scale slots (C4 <= C)
  tile_mxfp4_kernel<<<(unsigned)((slots + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const u8 *>(nibbles), static_cast<const u8 *>(scales), rows, (int)k, static_cast<u8 *>(nib_t),
      static_cast<u8 *>(sc_t));
  return launch_status();
}

int qmm_dequant_mxfp4t(const void *w, const void *ws, int64_t rows, int64_t k, float *out, hipStream_t s) {
  if (rows % 32 || k % 64) return QMM_ERR_SHAPE;
  if (!aligned(ws, 4)) return QMM_ERR_ALIGN;
  const int64_t groups = rows * (k / 32);
  dequant_mxfp4t_kernel<<<(unsigned)((groups + 255) / 256), 256, 0, s>>>(static_cast<const u8 *>(w),
                                                                         static_cast<const u8 *>(ws), rows, (int)k, out);
  return launch_status();
}
