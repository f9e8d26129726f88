// MXFP4 grouped expert GEMMs on the gfx950 scaled MFMA, the g_moe_ggu_mxfp4s[_fused]_k{H} / g_moe_gdn_mxfp4s_k{FE}
// kernels of the reference's MoE prefill chain (S/gen_moe.py:1126-1228; its fp8 MXFP4 GEMM, S/gen_mxfp4s.py:1-21,
// is the gfx12 WMMA counterpart):
//
//   gu   act[r, c] = act_fn(sum_k X8[t, k] Wg[e][c, k], sum_k X8[t, k] Wu[e][c, k]),  t = rowmap[r] / KU
//   dn   ys[r, c]  = sum_k A8[r, k] Wd[e][c, k]                                        (rows already sorted)
//
// for every row r of every 64-row tile with expert e = tile_info[tile, 0] >= 0 (rows with rowmap[r] < 0 are written
// as zeros). W is MXFP4 in split planes: nibbles [E, rows, K/2] ("pairs": byte j holds elements 2j, 2j+1) and
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
// Tiling: a workgroup of four waves owns one 64-row expert tile; each wave computes 64 rows x 64 weight columns
// (2 x 2 MFMA blocks) over all of K. gu: wave w owns output columns 32 w .. 32 w + 31 of a 128-column block, its
// two column blocks being those columns of the gate and of the up matrix, so the activation is applied in
// registers. dn: wave w owns the 32 columns 32 w .. 32 w + 31 of a 128-column block. Tiles are dealt to the eight XCDs round-robin
// (workgroup b runs on XCD b % 8): the bucket writes the live tiles first, and a tile-major order would leave
// the XCDs that get the trailing, unused tiles idle; a tile's column blocks stay on one XCD, sharing its
// activation rows in that L2.
//
// Steps. All E8M0 scales of the workgroup (its 64 activation rows and 128 + 128 or 128 weight columns, K / 32
// bytes each) are staged in LDS once; per-step byte loads of scales through the vector memory path cost more than
// the weight stream. A super-step covers kSub 64-value chunks: the tile's activation codes for it are staged in
// LDS (double-buffered, one barrier per super-step) and the weights stream straight into registers one super-step
// ahead, kSub consecutive 32-byte chunks of a column issued back to back.
#include <type_traits>

#include "common.hpp"

using namespace qmm;

namespace {

#ifndef QMM_MX_DEPTH
#define QMM_MX_DEPTH 1
#endif
#ifndef QMM_MX_WAVES
#define QMM_MX_WAVES 3            // minimum waves per SIMD the register allocation must allow (3 workgroups per CU)
#endif
constexpr int kDepth = QMM_MX_DEPTH;
#ifndef QMM_MX_SUB
#define QMM_MX_SUB 2
#endif
constexpr int kSub = QMM_MX_SUB;                      // 64-value chunks per super-step (one barrier each)
constexpr int BM = 64, KC = 64, APITCH = kSub * KC + 16;   // activation bytes per LDS row (16-byte aligned rows)

enum Kind { kGU = 1, kDN = 2 };
typedef __attribute__((ext_vector_type(4))) u32 v4u;   // a native vector: the register rings stay in VGPRs

struct MArgs {
  int N, K;
  const u8 *x8, *xs;            // activation codes [rows, K], scales [rows, K/32]
  int x_rows;
  const u8 *wn, *wsc;           // gate (or down) nibbles / scales of expert 0
  const u8 *wn2, *wsc2;         // up nibbles / scales (gu, not fused) or NULL
  int64_t nib_ebytes, sc_ebytes;   // bytes of one expert's nibble / scale plane
  int64_t up_nib_off, up_sc_off;   // fused gu: offset of the up rows inside an expert
  const int32_t *tile_info, *rowmap;
  int KU, E, act;
  float *y;
  int n_blocks, max_tiles;
};

__device__ __forceinline__ float act_fn(int act, float g, float u) {
  if (act == QMM_ACT_SWIGLU_OAI) {
    const float xg = fminf(g, 7.0f);
    const float yu = fminf(fmaxf(u, -7.0f), 7.0f);
    return xg / (1.0f + expf(-1.702f * xg)) * (yu + 1.0f);
  }
  return g / (1.0f + expf(-g)) * u;
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
constexpr int kBatch = 8;
template <class T, class G>
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

template <int KIND, int DEPTH>
__global__ __launch_bounds__(256, QMM_MX_WAVES) void mxfp4_grouped_kernel(MArgs a) {
  constexpr int BN = 128;                   // output columns per workgroup
  constexpr int NJ = KIND == kGU ? 2 : 1;    // 32-column weight blocks per wave (gu: gate and up)
  __shared__ __align__(16) u8 As[2][BM][APITCH];
  __shared__ int src_row[BM];
  // Every E8M0 scale the workgroup needs, staged once: the tile's 64 activation rows and the block's weight columns
  // (gu: 128 gate then 128 up columns; dn: 128 columns), K / 32 bytes each. Per-step byte loads of scales through
  // the vector memory path (32 rows per instruction) would otherwise cost more than the weight stream itself.
  extern __shared__ __align__(16) u8 dyn_lds[];
  u8 *Asc = dyn_lds, *Wsc = dyn_lds + BM * (a.K / 32);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int xcd = (int)(blockIdx.x & 7), xi = (int)(blockIdx.x >> 3);
  const int tile = xcd + 8 * (xi / a.n_blocks);
  if (tile >= a.max_tiles) return;
  const int N = a.N, K = a.K, C = K / KC;
  const int n0 = (xi % a.n_blocks) * BN, m0 = tile * BM;
  int expert = a.tile_info[2 * tile];
  if (expert < 0) return;
  expert = expert >= a.E ? a.E - 1 : expert;

  int my_src = -1;
  if (tid < BM) {
    int src;
    if constexpr (KIND == kGU) {
      const int rm = a.rowmap[m0 + tid];
      src = rm >= 0 ? rm / a.KU : -1;
      src = src < a.x_rows ? src : -1;
    } else {
      src = a.rowmap[m0 + tid] >= 0 ? m0 + tid : -1;
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
  auto clampc = [&](int c) __attribute__((always_inline)) { return c < C ? c : C - 1; };
  const int SK = K / 32;   // scale bytes per row

  // ---- weights: this lane's two columns (gu: one column of the gate and of the up matrix) and K half
  const int h = lane >> 5, lc = lane & 31;
  const u8 *nbj[NJ], *sbj[NJ];
  const int col = n0 + 32 * wave + lc;       // the lane's output column
  if constexpr (KIND == kGU) {
    const u8 *gn = a.wn + (int64_t)expert * a.nib_ebytes, *gs = a.wsc + (int64_t)expert * a.sc_ebytes;
    nbj[0] = gn; sbj[0] = gs;
    if (a.wn2) { nbj[1] = a.wn2 + (int64_t)expert * a.nib_ebytes; sbj[1] = a.wsc2 + (int64_t)expert * a.sc_ebytes; }
    else { nbj[1] = gn + a.up_nib_off; sbj[1] = gs + a.up_sc_off; }
  } else {
    nbj[0] = a.wn + (int64_t)expert * a.nib_ebytes;
    sbj[0] = a.wsc + (int64_t)expert * a.sc_ebytes;
  }
  const u8 *wcn[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) wcn[j] = nbj[j] + (int64_t)(col < N ? col : N - 1) * (K / 2) + 16 * h;
  int wrow[NJ];   // the lane's weight columns as rows of Wsc (gu: the gate block, then the up block)
#pragma unroll
  for (int j = 0; j < NJ; ++j) wrow[j] = 128 * j + 32 * wave + lc;

  f32x16 acc[2][NJ];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Rings DEPTH super-steps deep. A super-step reads kSub consecutive 32-byte chunks of each weight column -- a
  // whole 128-byte line for kSub = 4 -- with back-to-back loads, so the L1 merges them into one request per line.
  v4u aring[DEPTH][kSub], bring[DEPTH][kSub][NJ];
  auto load_a = [&](int slot, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSub; ++i)
      aring[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)(aoff + (u32)(clampc(kSub * st + i) * KC)), 0, 0);
  };
  auto load_b = [&](int slot, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < kSub; ++i)
        bring[slot][i][j] = *reinterpret_cast<const v4u *>(wcn[j] + (int64_t)clampc(kSub * st + i) * 32);
  };
  auto stage = [&](int slot, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kSub; ++i) *reinterpret_cast<v4u *>(&As[buf][arow_i][KC * i + 16 * apart]) = aring[slot][i];
  };
  // The first activation chunk, then the weights, so the stream is running while the scales are staged; staging
  // the first chunk waits only for its own load (loads complete in issue order), and precedes the loads that
  // reuse its ring slot.
  load_a(0, 0);
  for_slots([&](auto uc) { constexpr int u = decltype(uc)::value; load_b(u, u); },
            std::make_integer_sequence<int, DEPTH>{});
  stage(0, 0);
  for_slots([&](auto uc) { constexpr int u = decltype(uc)::value; load_a((u + 1) % DEPTH, u + 1); },
            std::make_integer_sequence<int, DEPTH>{});
  // the scale rows: activation rows (a gathered row each), then the weight column blocks (contiguous in memory)
  batched_copy(reinterpret_cast<u16 *>(Asc), (int64_t)BM * (SK / 2), tid, [&](int64_t i) {
    const int r = (int)(i / (SK / 2)), q = (int)(i % (SK / 2));
    const int sr = src_row[r] >= 0 ? src_row[r] : 0;
    return reinterpret_cast<const u16 *>(a.xs + (int64_t)sr * SK)[q];
  });
  {
    const int cols = N - n0 < BN ? N - n0 : BN;   // columns past N are never stored
#pragma unroll
    for (int m = 0; m < NJ; ++m) copy_to_lds(Wsc + m * BN * SK, sbj[m] + (int64_t)n0 * SK, (int64_t)cols * SK, tid);
  }
  __syncthreads();

  // The super-step count is rounded up to a multiple of DEPTH. A padding chunk (c >= C) runs with both E8M0 scales
  // 0: its products are at most 448 * 6 * 2^-254, far below the smallest f32 subnormal, so they add exactly zero.
  // The loop body thus has no data-dependent branch; each super-step is instantiated with its ring slot as a
  // constant (integral_constant), so the rings stay in registers.
  auto step = [&](auto uc, int s0) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    constexpr int nx = (u + 1) % DEPTH;
    const int st = s0 + u;
    const int buf = st & 1;
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const bool live = kSub * st + i < C;
      const int sc_off = 2 * clampc(kSub * st + i) + h;   // the lane's E8M0 byte of this chunk in a scale row
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
        const v4u bv = bring[u][i][j];
        bf[j] = i32x8{(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w, 0, 0, 0, 0};
        sb[j] = live ? Wsc[wrow[j] * SK + sc_off] : 0;
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
    load_b(u, st + DEPTH);
    stage(nx, buf ^ 1);
    load_a(nx, st + 1 + DEPTH);
    __syncthreads();
  };
  const int S = (C + kSub - 1) / kSub;
  const int SP = (S + DEPTH - 1) / DEPTH * DEPTH;
  for (int s0 = 0; s0 < SP; s0 += DEPTH)
    for_steps(step, s0, std::make_integer_sequence<int, DEPTH>{});

  if (col >= N) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lr = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
      float v = 0.f;
      if (src_row[lr] >= 0) {
        if constexpr (KIND == kGU) v = act_fn(a.act, acc[i][0][r], acc[i][1][r]);
        else v = acc[i][0][r];
      }
      a.y[(int64_t)(m0 + lr) * N + col] = v;
    }
}

template <int KIND>
int launch(const MArgs &a, hipStream_t s) {
  const dim3 grid((unsigned)(8 * a.n_blocks * ((a.max_tiles + 7) / 8)));
  const size_t dyn = (size_t)(BM + (KIND == kGU ? 256 : 128)) * (a.K / 32);
  if (dyn > 32768) {   // beyond the default dynamic LDS limit (K > 3276): raise it once
    static bool raised = false;
    if (!raised) {
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(&mxfp4_grouped_kernel<KIND, kDepth>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn) != hipSuccess)
        return QMM_ERR_LAUNCH;
      raised = true;
    }
  }
  mxfp4_grouped_kernel<KIND, kDepth><<<grid, 256, dyn, s>>>(a);
  return launch_status();
}

}  // namespace

// The MXFP4 (split planes) path of qmm_moe_grouped.
int qmm_grouped_mxfp4(int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E, int KU,
                      const int32_t *tile_info, const int32_t *rowmap, const void *x, const void *x_scales,
                      int64_t x_rows, const void *w, const void *ws, const void *w2, const void *ws2, float *y,
                      hipStream_t s) {
  if (k % 64 || k > 12288) return QMM_ERR_SHAPE;   // the workgroup stages (64 + 256) x K / 32 scale bytes in LDS
  if (x_rows * k >= (1ll << 31)) return QMM_ERR_SHAPE;   // activation rows are addressed by a 32-bit buffer offset
  if (!x_scales || !ws) return QMM_ERR_NULL;
  if (!aligned(x_scales, 2)) return QMM_ERR_ALIGN;
  if (!aligned(x, 16) || !aligned(w, 16) || (w2 && !aligned(w2, 16))) return QMM_ERR_ALIGN;
  MArgs a{};
  a.N = (int)n; a.K = (int)k;
  a.x8 = static_cast<const u8 *>(x); a.xs = static_cast<const u8 *>(x_scales); a.x_rows = (int)x_rows;
  a.wn = static_cast<const u8 *>(w); a.wsc = static_cast<const u8 *>(ws);
  a.tile_info = tile_info; a.rowmap = rowmap; a.KU = KU; a.E = E; a.act = act; a.y = y;
  const int64_t nrow = k / 2, srow = k / 32;
  if (mode == 0) {
    if (!fused && (!w2 || !ws2)) return QMM_ERR_NULL;
    a.nib_ebytes = nrow * n * (fused ? 2 : 1);
    a.sc_ebytes = srow * n * (fused ? 2 : 1);
    a.up_nib_off = fused ? nrow * n : 0;
    a.up_sc_off = fused ? srow * n : 0;
    a.wn2 = fused ? nullptr : static_cast<const u8 *>(w2);
    a.wsc2 = fused ? nullptr : static_cast<const u8 *>(ws2);
    a.n_blocks = (int)((n + 127) / 128);
    a.max_tiles = (int)max_tiles;
    return launch<kGU>(a, s);
  }
  a.nib_ebytes = nrow * n;
  a.sc_ebytes = srow * n;
  a.n_blocks = (int)((n + 127) / 128);
  a.max_tiles = (int)max_tiles;
  return launch<kDN>(a, s);
}
