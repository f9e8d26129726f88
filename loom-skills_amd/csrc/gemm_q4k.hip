// GGUF-block matmuls on the f16 MFMA (Q4_K, Q6_K, Q4_0): the prefill GEMM g_gemm_{fmt}_{store|acc|swiglu}
// (S/gen_gemm.py:535-703) and the MoE grouped expert GEMMs g_moe_ggu_{fmt}[_fused]_k{H} / g_moe_gdn_{fmt}_k{FE}
// (S/gen_moe.py:1126-1228; the Q4_0 expert staging of S/moe_q4_0.py:11-61).
//
//   dense   Y[r, c]   = (acc ? Y[r, c] : 0) + inv[r] sum_k X16[r, k] W[c, k]
//   gu      act[r, c] = act_fn(inv[t] sum_k X16[t, k] Wg[e][c, k] + bg[e, c], inv[t] sum_k X16[t, k] Wu[e][c, k]
//                       + bu[e, c]),  t = rowmap[r] / KU  (rows gathered from the token rows)
//   dn      ys[r, c]  = inv[r] sum_k A16[r, k] Wd[e][c, k] + bd[e, c]            (rows already sorted)
//
// for every row r of every 64-row tile whose expert e = tile_info[tile, 0] >= 0; rows with rowmap[r] < 0 are not
// written. The optional expert biases (gpt-oss ffn_{gate,up,down}_exps.bias) are added after the row
// inverse, before the activation (_gemm_bias_act, S/gen_moe.py:958-1007). X16 / A16 are the row-scaled f16 operands the reference's g_row_scale_f16[_tiles] produces
// (S/gen_llm.py:1843-1915, S/gen_moe.py:503-527) and inv = their scales[row, 1]. W is dequantized to f16 in
// registers the way the reference stages it: Q4_K w = fma_f16(f16(q), f16(d sc), f16(-dmin m)) (S/gen_gemm.py:499-530),
// Q6_K w = fma_f16(f16(q), f16(d sc), f16(-32 d sc)) (S/gen_gemm.py:369-444), Q4_0 w = f16(q - 8) * d with one f16
// rounding (S/moe_q4_0.py:11-38: exactly f16(d (q - 8)) for every finite f16 d). fp32 accumulation throughout.
//
// Tiling (gfx950, wave64). A workgroup has four waves and one 64-row tile. Dense and dn: the tile is 64 x 128 and
// wave (nh, kh) computes the 64 x 64 quadrant nh over K-half kh; gu: the tile is 64 x 64 and wave (mat, kh)
// computes it for matrix mat (gate, up) over K-half kh. Each wave holds 2 x 2 v_mfma_f32_32x32x16_f16
// accumulators. The K-halves are summed through LDS at the end in a fixed order (and, for gu, the up result is
// handed to the gate wave for the activation). A step is one 64-value page of a super-block: the activation rows
// of both K-halves (2 x 64 x 64 f16) are staged in LDS, double-buffered, one barrier per step; each wave streams
// its own 64 weight columns straight into registers and dequantizes them there, so weights never touch LDS. Loads
// run DEPTH steps ahead of the math through register rings; the loads are unconditional (clamped addresses), so no
// branch splits the load stream and the compiler keeps them in flight.
//
// MFMA operand order. Lane l of a 32x32x16 step holds 8 K values of row/column l % 32, octet l / 32. Q4_K / Q6_K:
// lane half h takes code bytes 16h .. 16h+15 of a page, i.e. values 16h .. 16h+15 of both of the page's sub-blocks
// (gl = 0, 1); K16 step s2 of a sub-block uses the lane's values 8 s2 .. 8 s2 + 7, step position 32 gl + 16 h + 8 s2.
// Q4_0: a 64-value step is two blocks and lane half h takes block h's 16 code bytes, whose low nibbles (gl = 0) are
// the block's values 0..15 and high nibbles (gl = 1) values 16..31: step position 32 h + 16 gl + 8 s2. The A fragment
// is read from LDS at the same K.
//
// Tile order is XCD-aware: consecutive tile ids land on one XCD (dense: the M tiles of one N tile, which share
// weight columns; grouped: the column blocks of one expert tile, which share its activation rows).
#include <type_traits>

#include "common.hpp"
#include "deq_f16.hpp"

using namespace qmm;

namespace {

constexpr int BM = 64, KSTEP = 64;
#ifndef QMM_GEMM_DEPTH
#define QMM_GEMM_DEPTH 4
#endif
constexpr int kDepth = QMM_GEMM_DEPTH;   // steps of loads in flight per wave (even)
static_assert(kDepth % 2 == 0, "the LDS double buffer follows the step parity");
constexpr int APITCH = KSTEP + 8;   // f16 per LDS row: 144 bytes, rows 16-byte aligned, reads 2-way at most

// kDense: Y (+)= X W^T; kSwiglu: Y = silu(X Wg^T inv) (X Wu^T inv) over dense rows (the GEMM's swiglu mode);
// kGU / kDN: the grouped gate/up and down GEMMs over bucketed expert tiles
enum Kind { kDense = 0, kGU = 1, kDN = 2, kSwiglu = 3 };
// weight formats: GGUF Q4_K (144-byte super-blocks), Q6_K (210), Q4_0 (18-byte blocks of 32)
enum WFmt { kWQ4K = 0, kWQ6K = 1, kWQ40 = 2 };

struct Args {
  int M, N, K;                 // dense: rows; grouped: rows of the sorted output (max_tiles * 64)
  const _Float16 *x16;         // activation rows (dense / dn: [M, K]; gu: token rows [x_rows, K])
  const float *scales;         // [rows of x16, 2] or NULL
  int x_rows;                  // rows of x16 (gu)
  const u8 *w, *w2;            // dense: W; grouped: expert tensors (gu: gate, up; fused: w only)
  int64_t ebytes;              // bytes of one expert's matrix (grouped)
  int64_t ebytes2;             // gu, two tensors: bytes of one expert's up matrix (its own format's rows)
  int64_t up_off;              // gu: byte offset of the up matrix from the gate matrix of an expert (fused)
  const int32_t *tile_info, *rowmap;
  const float *bias, *bias2;   // grouped: per-expert output biases [E, N] (gu: gate, up; dn: bias only) or NULL
  int KU, E, act;
  void *y;
  int tiles_m, n_blocks, tiles_total;
};

// Scale tables: a workgroup decodes the (d sc, -dmin m) f16 pair of every sub-block of its 128 weight columns once
// into LDS (4 bytes per sub-block, 16 (K + 64) bytes) when that fits (K <= kStagedMaxK); each step then reads its two
// pairs per column with one 8-byte LDS read instead of loading and decoding the super-block header again.
constexpr int kStagedMaxK = 6144;

// WF2: the up matrix's format when it differs from the gate's (kGU / kSwiglu of a QMM_GATE_UP pair): the up waves
// load and dequantize in their own format, with their own row stride, the gate waves in WF.
// TL: Q4_K weights in the tiled layout QMM_Q4_KT (K % 512 == 0, N % 16 == 0): the lane reads the same code bytes and
// headers at their tiled addresses (column c's 16-row block at (c / 16) 16 RB; super-block sb of its row r = c % 16
// is half sb % 2 of unit sb / 2 of 4608 bytes: header at 16 (2 r + sb % 2), page p's bytes 16 h .. + 15 in plane
// 2 (p % 2) + h at 512 + 1024 (2 (p % 2) + h) + 16 (4 r + 2 (sb % 2) + p / 2)), so the results are the GGUF call's.
template <int KIND, bool ACC, bool BF16OUT, int DEPTH, bool STAGED, int WF, int KS, int WF2 = WF, bool TL = false>
__global__ __launch_bounds__(128 * KS, 1) void q4k_mfma_kernel(Args a) {
  constexpr int NT = 128 * KS;   // threads: 2 column halves (or matrices) x KS K-parts
  constexpr bool MIXED = WF2 != WF;
  static_assert(!(WF != kWQ4K && STAGED), "Q6_K / Q4_0 scales are read with the codes");
  constexpr bool kTwoW = KIND == kGU || KIND == kSwiglu;        // two weight matrices (gate, up): wave pairs
  static_assert(!MIXED || (kTwoW && !STAGED), "a second format is the up matrix's of gate/up, scales read with codes");
  static_assert(!TL || (WF == kWQ4K && !MIXED), "the tiled layout holds Q4_K");
  constexpr bool kDenseRows = KIND == kDense || KIND == kSwiglu;  // rows m0 .. m0 + 63 of x, tiles row-major
  constexpr int BN = kTwoW ? 64 : 128;
  extern __shared__ __align__(16) u32 scl[];   // STAGED: [128 columns][K / 32 + 2] (dsc | nmn << 16)
  __shared__ __align__(16) _Float16 As[2][KS][BM][APITCH];   // [buffer][K-part][row][k]
  __shared__ int src_row[BM];
  __shared__ float rinv[BM];   // the row's inverse activation scale (1 without scales)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sel = wave & 1, kh = wave >> 1;   // sel: N-half (dense, dn) or matrix (gu: 0 gate, 1 up); kh: K-part
  const bool upw = MIXED && sel == 1;         // a wave of the up matrix in its own format
  const int M = a.M, N = a.N, K = a.K;

  int m0, n0, expert = 0;
  if constexpr (kDenseRows) {
    // XCD-aware order: workgroup b runs on XCD b % 8, which gets a contiguous range of tiles
    const int per = (int)(gridDim.x / 8);
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= a.tiles_total) return;
    m0 = (t % a.tiles_m) * BM;
    n0 = (t / a.tiles_m) * BN;
  } else {
    // expert tiles dealt to the XCDs round-robin: the bucket writes the live tiles first, so a contiguous range per
    // XCD would leave the XCDs holding the trailing unused tiles idle; a tile's column blocks share one XCD's L2
    const int xcd = (int)(blockIdx.x & 7), xi = (int)(blockIdx.x >> 3);
    const int tile = xcd + 8 * (xi / a.n_blocks);
    if (tile >= a.tiles_m) return;
    n0 = (xi % a.n_blocks) * BN;
    m0 = tile * BM;
    expert = a.tile_info[2 * tile];
    if (expert < 0) return;
    expert = expert >= a.E ? a.E - 1 : expert;
  }
  // activation row of each tile row (-1: a dead row, written as zero)
  int my_src = -1;
  if (tid < BM) {
    int src;
    if constexpr (kDenseRows) src = m0 + tid < M ? m0 + tid : -1;
    else if constexpr (KIND == kGU) {
      const int rm = a.rowmap[m0 + tid];
      src = rm >= 0 ? rm / a.KU : -1;
      src = src < a.x_rows ? src : -1;
    } else {
      src = a.rowmap[m0 + tid] >= 0 ? m0 + tid : -1;
    }
    src_row[tid] = src;
    rinv[tid] = (a.scales && src >= 0) ? a.scales[2 * src + 1] : 1.f;
    my_src = src;
  }
  if constexpr (kDenseRows) {
    // skip-padding: a tile whose rows all have scale 0 (padding rows) does no work and writes nothing
    if (a.scales) {
      const bool live = tid < BM && my_src >= 0 && a.scales[2 * my_src] != 0.f;
      if (__syncthreads_or(live) == 0) return;
    }
  }
  // whether rows 32..63 hold a live row: if not, the upper 32-row MFMA blocks are skipped (their outputs are the
  // zeros of dead rows) -- expert tiles of prefill batches are often less than half full
  const bool upper = __syncthreads_or(tid >= 32 && my_src >= 0) != 0;

  auto rowb = [&](int f) { return f == kWQ40 ? (int64_t)K / 32 * 18 : (int64_t)K / 256 * (f == kWQ6K ? 210 : 144); };
  const int64_t RB = upw ? rowb(WF2) : rowb(WF);   // bytes per weight row of the wave's matrix
  const int S = K / KSTEP, S0 = S / KS;

  // ---- A staging map: chunk c = i * NT + tid of 16 bytes; K-part, row, 16-byte column. Loads are unconditional
  // (dead rows read activation row 0 and their outputs are zeroed; steps past S0 reload step S0 - 1 and get zero
  // weights in the math).
  // The loads go through a buffer resource over the activation rows: a dead row's offset lies past its end
  // (0x80000000), where the hardware returns zeros without touching memory, so a tile of a few live rows fetches
  // only those.
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(a.x16), (short)0, (int)((int64_t)a.x_rows * K * 2), 0x00020000);
  u32 aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = i * NT + tid, ckh = c >> 9, row = (c >> 3) & 63, col = c & 7;
    const int src = src_row[row];
    aoff[i] = src >= 0 ? (u32)(((int64_t)src * K + (int64_t)ckh * S0 * KSTEP + col * 8) * 2) : 0x80000000u;
  }
  auto a_load = [&](int i, int s) -> uint4 {
    typedef __attribute__((ext_vector_type(4))) u32 u32x4;
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)(aoff[i] + (u32)((s < S0 ? s : S0 - 1) * KSTEP * 2)), 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  auto a_dst = [&](int i, int buf) -> uint4 * {
    const int c = i * NT + tid, ckh = c >> 9, row = (c >> 3) & 63, col = c & 7;
    return reinterpret_cast<uint4 *>(&As[buf][ckh][row][col * 8]);
  };

  // ---- B: this lane's two weight columns and code half
  const int h = lane >> 5, lc = lane & 31;
  const u8 *wbase;
  if constexpr (KIND == kDense) wbase = a.w;
  else if constexpr (KIND == kSwiglu) wbase = sel ? a.w2 : a.w;
  else if constexpr (KIND == kGU) {
    const u8 *g = a.w + (int64_t)expert * a.ebytes;
    wbase = sel ? (a.w2 ? a.w2 + (int64_t)expert * a.ebytes2 : g + a.up_off) : g;
  } else {
    wbase = a.w + (int64_t)expert * a.ebytes;
  }
  const u8 *wcol[2];   // GGUF: the column's row; tiled: its 16-row block
  int tco[2], tho[2];  // tiled: the column's code and header offsets in a unit
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int c = n0 + (kTwoW ? 0 : sel * 64) + 32 * j + lc;
    c = c < N ? c : N - 1;
    wcol[j] = TL ? wbase + (int64_t)(c >> 4) * 16 * RB : wbase + (int64_t)c * RB;
    tco[j] = 512 + 1024 * h + 64 * (c & 15);
    tho[j] = 32 * (c & 15);
  }
  auto b_code = [&](int j, int s) -> uint4 {
    const int gs = kh * S0 + (s < S0 ? s : S0 - 1);
    if constexpr (TL) {
      const int sb = gs >> 2, p = gs & 3;
      return ld16(wcol[j] + tco[j] + (int64_t)(sb >> 1) * 4608 + 2048 * (p & 1) + 32 * (sb & 1) + 16 * (p >> 1));
    }
    return ld16(wcol[j] + (int64_t)(gs >> 2) * 144 + 16 + 32 * (gs & 3) + 16 * h);
  };
  // Q6_K page gs & 3 = (half, jh): groups j = 2 jh (ql bytes 64 half + l) and 2 jh + 1 (64 half + 32 + l), both with
  // qh bytes 32 half + l; lane half h takes l = 16 h .. 16 h + 15, the scales sc[8 half + 4 jh + h] and [.. + 2 + h]
  auto b_q6 = [&](int j, int s, uint4 &qa, uint4 &qb, uint4 &qh, u32 &sc, u32 &dd) {
    const int gs = kh * S0 + (s < S0 ? s : S0 - 1);
    const u8 *blk = wcol[j] + (int64_t)(gs >> 2) * 210;
    const int half = (gs >> 1) & 1, jh = gs & 1;
    qa = ld16u(blk + 64 * half + 16 * h);
    qb = ld16u(blk + 64 * half + 32 + 16 * h);
    qh = ld16u(blk + 128 + 32 * half + 16 * h);
    sc = ld4u(blk + 192 + 8 * half + 4 * jh);
    dd = *reinterpret_cast<const u16 *>(blk + 208);
  };
  // Q4_0 step gs: blocks 2 gs and 2 gs + 1; lane half h takes block 2 gs + h (16 code bytes after its f16 d)
  auto b_q40 = [&](int j, int s, uint4 &q, u32 &dd) {
    const int gs = kh * S0 + (s < S0 ? s : S0 - 1);
    const u8 *blk = wcol[j] + (int64_t)(2 * gs + h) * 18;
    q = ld16u(blk + 2);
    dd = *reinterpret_cast<const u16 *>(blk);
  };
  auto b_head = [&](int j, int s) -> uint4 {
    const int sb = (kh * S0 + (s < S0 ? s : S0 - 1)) >> 2;
    if constexpr (TL) return ld16(wcol[j] + tho[j] + (int64_t)(sb >> 1) * 4608 + 16 * (sb & 1));
    return ld16(wcol[j] + (int64_t)sb * 144);
  };
  // sub-blocks per column, and the staged table's row pitch in dwords: two more than K / 32 (a multiple of 8), so
  // the 32 columns a wave reads at once start two banks apart instead of all in one bank
  const int SB = K / 32, SBP = SB + 2;
  if constexpr (STAGED) {
    // local column cl = sel * 64 + 32 j + lc: dense / dn columns n0 + cl, gu: gate n0 + cl (cl < 64), up n0 + cl - 64
    // every header of the workgroup's columns, kHdrBatch loads in flight per thread before any is decoded
    constexpr int kHdrBatch = 4;
    const int nh = 128 * (K / 256);
    for (int b0 = 0; b0 < nh; b0 += kHdrBatch * NT) {
      uint4 hd[kHdrBatch];
#pragma unroll
      for (int q = 0; q < kHdrBatch; ++q) {
        int i = b0 + tid + NT * q;
        i = i < nh ? i : nh - 1;
        const int cl = i / (K / 256), b = i % (K / 256);
        const int msel = cl >> 6;
        const u8 *mb;
        if constexpr (KIND == kDense) mb = a.w;
        else if constexpr (KIND == kSwiglu) mb = msel ? a.w2 : a.w;
        else if constexpr (KIND == kGU) {
          const u8 *g = a.w + (int64_t)expert * a.ebytes;
          mb = msel ? (a.w2 ? a.w2 + (int64_t)expert * a.ebytes2 : g + a.up_off) : g;
        } else {
          mb = a.w + (int64_t)expert * a.ebytes;
        }
        int c = n0 + (kTwoW ? cl - 64 * msel : cl);
        c = c < N ? c : N - 1;
        hd[q] = TL ? ld16(mb + (int64_t)(c >> 4) * 16 * RB + 32 * (c & 15) + (int64_t)(b >> 1) * 4608 + 16 * (b & 1))
                   : ld16(mb + (int64_t)c * RB + (int64_t)b * 144);
      }
#pragma unroll
      for (int q = 0; q < kHdrBatch; ++q) {
        const int i = b0 + tid + NT * q;
        if (i >= nh) continue;
        const int cl = i / (K / 256), b = i % (K / 256);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          h2 dsc, nmn;
          sub_scale(hd[q], g, dsc, nmn);
          scl[cl * SBP + 8 * b + g] = (u32)__builtin_bit_cast(u16, dsc[0]) | ((u32)__builtin_bit_cast(u16, nmn[0]) << 16);
        }
      }
    }
  }

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Register rings, DEPTH steps deep: A chunks of steps s+1 .. s+DEPTH, B code/header of steps s .. s+DEPTH-1.
  // Step t lives in slot t % DEPTH; the step loop is unrolled DEPTH times so every slot index is static.
  uint4 aring[DEPTH][4], cring[DEPTH][2], hring[DEPTH][2];
  uint4 q6b[DEPTH][2], q6h[DEPTH][2];   // Q6_K: ql of group B and qh (cring holds ql of group A)
  u32 q6s[DEPTH][2], q6d[DEPTH][2];      // Q6_K scales and d; Q4_0: d in q6d (cring holds the codes)
  auto load_a = [&](int slot, int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) aring[slot][i] = a_load(i, st);
  };
  auto load_b_f = [&](auto fc, int slot, int st) __attribute__((always_inline)) {
    constexpr int F = decltype(fc)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (F == kWQ6K) {
        b_q6(j, st, cring[slot][j], q6b[slot][j], q6h[slot][j], q6s[slot][j], q6d[slot][j]);
      } else if constexpr (F == kWQ40) {
        b_q40(j, st, cring[slot][j], q6d[slot][j]);
      } else {
        cring[slot][j] = b_code(j, st);
        if constexpr (!STAGED) hring[slot][j] = b_head(j, st);
      }
    }
  };
  auto load_b = [&](int slot, int st) __attribute__((always_inline)) {
    if constexpr (!MIXED) load_b_f(std::integral_constant<int, WF>{}, slot, st);
    else if (upw) load_b_f(std::integral_constant<int, WF2>{}, slot, st);
    else load_b_f(std::integral_constant<int, WF>{}, slot, st);
  };
  // The prologue issues its loads in the loop's own order (a step issues the weights of step s + DEPTH, then the
  // activations of step s + 1 + DEPTH). Vector loads complete in issue order for s_waitcnt, and the compiler places
  // one wait per wait point valid on both paths into the loop header, so a prologue with another order (all
  // activations first, say) would make the loop's waits stricter than the loop needs and drain the ring.
  static_assert(DEPTH >= 2 && DEPTH % 2 == 0, "activation slots 0 and 1 hold steps 0 and 1 at once");
  load_b(0, 0);
  load_a(0, 0);
  load_a(1, 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) *a_dst(i, 0) = aring[0][i];
#pragma unroll
  for (int u = 1; u < DEPTH; ++u) {
    load_b(u, u);
    load_a((u + 1) % DEPTH, u + 1);
  }
  __syncthreads();

  // The step count is rounded up to a multiple of DEPTH; steps past S0 get zero weights (no contribution), so the
  // loop body has no data-dependent branch and every wave runs the same barriers. Every K-part has S0 steps
  // (K is a multiple of 256, so K / 64 is a multiple of 4).
  const int SP = (S0 + DEPTH - 1) / DEPTH * DEPTH;
  for (int s0 = 0; s0 < SP; s0 += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int s = s0 + u;
      const int buf = u & 1;   // DEPTH is even, so s & 1 == u & 1
      const int gstep = kh * S0 + (s < S0 ? s : S0 - 1);
      const int page = gstep & 3;
      typedef __attribute__((ext_vector_type(2))) u32 u32x2;
      u32x2 sp[2];
      if constexpr (STAGED) {
#pragma unroll
        for (int j = 0; j < 2; ++j) sp[j] = *reinterpret_cast<const u32x2 *>(&scl[(sel * 64 + 32 * j + lc) * SBP + 2 * gstep]);
      }
      auto math = [&](auto fc) __attribute__((always_inline)) {
        constexpr int F = decltype(fc)::value;
  #pragma unroll
        for (int gl = 0; gl < 2; ++gl) {
          h2 dsc[2], nmn[2];
  #pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (F == kWQ40) {
              const _Float16 d16 = __builtin_bit_cast(_Float16, (u16)q6d[u][j]);
              dsc[j] = h2{d16, d16};
              nmn[j] = h2{0, 0};
            } else if constexpr (F == kWQ6K) {
              // f16 (d sc, -32 d sc) of the lane's 16-value run: d sc is exact in f32 (S/gen_gemm.py:435-444)
              const float sv = f16_to_f32(q6d[u][j]) * (float)(signed char)((q6s[u][j] >> (8 * (2 * gl + h))) & 0xFFu);
              const _Float16 a16 = (_Float16)sv, b16 = (_Float16)(-32.f * sv);
              dsc[j] = h2{a16, a16};
              nmn[j] = h2{b16, b16};
            } else if constexpr (STAGED) {
              const u32 v = gl ? sp[j].y : sp[j].x;
              dsc[j] = as_h2((v & 0xFFFFu) * 0x10001u);
              nmn[j] = as_h2((v >> 16) * 0x10001u);
            } else {
              sub_scale(hring[u][j], 2 * page + gl, dsc[j], nmn[j]);
            }
            if (s >= S0) dsc[j] = nmn[j] = h2{0, 0};   // a padding step: zero weights
          }
  #pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            f16x8 bf[2], af[2];
  #pragma unroll
            for (int j = 0; j < 2; ++j) {
              if constexpr (F == kWQ6K) {
                // codes ((ql >> 4 jh) & 15) | (((qh >> (4 jh + 2 gl)) & 3) << 4), four to a dword
                const uint4 &ql = gl ? q6b[u][j] : cring[u][j];
                const u32 l0 = s2 ? ql.z : ql.x, l1 = s2 ? ql.w : ql.y;
                const u32 h0 = s2 ? q6h[u][j].z : q6h[u][j].x, h1 = s2 ? q6h[u][j].w : q6h[u][j].y;
                const u32 ls = 4u * (u32)(page & 1), hs = ls + 2u * (u32)gl;
                const u32 c0 = ((l0 >> ls) & 0x0F0F0F0Fu) | (((h0 >> hs) & 0x03030303u) << 4);
                const u32 c1 = ((l1 >> ls) & 0x0F0F0F0Fu) | (((h1 >> hs) & 0x03030303u) << 4);
                bf[j] = deq8_codes(c0, c1, dsc[j], nmn[j]);
              } else if constexpr (F == kWQ40) {
                const u32 q0 = s2 ? cring[u][j].z : cring[u][j].x, q1 = s2 ? cring[u][j].w : cring[u][j].y;
                bf[j] = gl ? deq8_q40<true>(q0, q1, dsc[j]) : deq8_q40<false>(q0, q1, dsc[j]);
              } else {
                const u32 q0 = s2 ? cring[u][j].z : cring[u][j].x, q1 = s2 ? cring[u][j].w : cring[u][j].y;
                bf[j] = gl ? deq8_e4m3<true>(q0, q1, dsc[j], nmn[j]) : deq8_e4m3<false>(q0, q1, dsc[j], nmn[j]);
              }
            }
            const int ak = F == kWQ40 ? 32 * h + 16 * gl + 8 * s2 : 32 * gl + 16 * h + 8 * s2;   // the lane's K position
            af[0] = *reinterpret_cast<const f16x8 *>(&As[buf][kh][lc][ak]);
  #pragma unroll
            for (int j = 0; j < 2; ++j) acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[0], bf[j], acc[0][j], 0, 0, 0);
            if (upper) {
              af[1] = *reinterpret_cast<const f16x8 *>(&As[buf][kh][32 + lc][ak]);
  #pragma unroll
              for (int j = 0; j < 2; ++j)
                acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[1], bf[j], acc[1][j], 0, 0, 0);
            }
          }
        }
      };
      if constexpr (!MIXED) math(std::integral_constant<int, WF>{});
      else if (upw) math(std::integral_constant<int, WF2>{});
      else math(std::integral_constant<int, WF>{});
      load_b(u, s + DEPTH);
      const int nx = (u + 1) % DEPTH;
#pragma unroll
      for (int i = 0; i < 4; ++i) *a_dst(i, buf ^ 1) = aring[nx][i];
      load_a(nx, s + 1 + DEPTH);
      __syncthreads();
    }
  }

  // ---- sum the K-parts through LDS in a fixed tree: with four parts, 2 and 3 hand theirs to 0 and 1, then 1 to 0
  float *red = reinterpret_cast<float *>(&As[0][0][0][0]);   // [slot][sel][64 values][64 lanes]
  static_assert(sizeof(As) >= (KS / 2) * 2 * 64 * 64 * 4, "K-part reduction staging");
  auto red_at = [&](int sl, int i, int j, int r) -> float & {
    return red[(sl * 64 + (i * 2 + j) * 16 + r) * 64 + lane];
  };
  auto hand = [&](int from, int to) __attribute__((always_inline)) {   // parts [from, 2 from) add into [to, ..)
    if (kh >= from && kh < 2 * from) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red_at(2 * (kh - from) + sel, i, j, r) = acc[i][j][r];
    }
    __syncthreads();
    if (kh < to) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += red_at(2 * kh + sel, i, j, r);
    }
    __syncthreads();
  };
  if constexpr (KS == 4) hand(2, 2);
  hand(1, 1);

  if constexpr (kTwoW) {
    // the up wave (K-half 0) hands its result to the gate wave; every wave takes part in the barriers
    __syncthreads();
    if (kh == 0 && sel == 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) red_at(0, i, j, r) = acc[i][j][r];
    }
    __syncthreads();
    if (sel == 1) return;
  }
  if (kh != 0) return;

  // ---- epilogue
  float *yf = static_cast<float *>(a.y);
  u16 *yb = static_cast<u16 *>(a.y);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        const int row = m0 + lr;
        const int col = n0 + (kTwoW ? 0 : sel * 64) + 32 * j + lc;
        if (col >= N || (kDenseRows && row >= M)) continue;
        const int src = src_row[lr];
        const int64_t o = (int64_t)row * N + col;
        if constexpr (kDenseRows) {
          float v;
          if constexpr (KIND == kSwiglu) v = act_fn(QMM_ACT_SILU, acc[i][j][r] * rinv[lr], red_at(0, i, j, r) * rinv[lr]);
          else v = acc[i][j][r] * rinv[lr];
          if constexpr (BF16OUT) {
            if constexpr (ACC) v += bf16_to_f32(yb[o]);
            yb[o] = (u16)f32_to_bf16_rne(v);
          } else {
            if constexpr (ACC) v += yf[o];
            yf[o] = v;
          }
        } else {
          if (src < 0) continue;   // a row without an assignment is not written
          const float inv = rinv[lr];
          const int64_t bo = (int64_t)expert * N + col;
          const float b = a.bias ? a.bias[bo] : 0.f;
          float v;
          if constexpr (KIND == kGU) {
            const float b2 = a.bias2 ? a.bias2[bo] : 0.f;
            v = act_fn(a.act, acc[i][j][r] * inv + b, red_at(0, i, j, r) * inv + b2);
          } else {
            v = acc[i][j][r] * inv + b;
          }
          yf[o] = v;
        }
      }
}

// Dense Q4_K rows (the prefill GEMM) run eight waves a workgroup, K in four parts: a 64 x 128 tile's workgroup then
// has two waves a SIMD, so one wave's dequantization overlaps the other's MFMAs (the grid of a 512-row GEMM is one
// workgroup a CU). The grouped GEMMs keep two K-parts (their expert tiles are many and their K short), and so does
// Q6_K.
template <int KIND, bool ACC, bool BF16OUT, int WF = kWQ4K, bool TL = false>
int launch(const Args &a, hipStream_t s) {
  constexpr bool kDenseRows = KIND == kDense || KIND == kSwiglu;
  constexpr int KS = kDenseRows && WF != kWQ6K ? 4 : 2;   // Q6_K's wider rings would spill at two waves a SIMD
  // staged scale tables beside the K-parts' activation buffers: 16 (K + 64) bytes, within 160 KB of LDS
  constexpr int kMaxK = KS == 4 ? 5120 : kStagedMaxK;
  const dim3 grid((unsigned)(kDenseRows ? 8 * ((a.tiles_total + 7) / 8) : 8 * a.n_blocks * ((a.tiles_m + 7) / 8)));
  if constexpr (WF != kWQ4K) {
    q4k_mfma_kernel<KIND, ACC, BF16OUT, kDepth, false, WF, KS><<<grid, 128 * KS, 0, s>>>(a);
    return launch_status();
  }
  if (a.K <= kMaxK) {
    const size_t dyn = (size_t)128 * (a.K / 32 + 2) * 4;
    if (dyn > 32768) {   // beyond the default dynamic LDS limit: raised to the largest table this kernel stages
      static std::atomic<unsigned> raised{0};
      if (int st = raise_dyn_lds(
              reinterpret_cast<const void *>(&q4k_mfma_kernel<KIND, ACC, BF16OUT, kDepth, true, kWQ4K, KS, kWQ4K, TL>),
              (int)((size_t)128 * (kMaxK / 32 + 2) * 4), raised))
        return st;
    }
    q4k_mfma_kernel<KIND, ACC, BF16OUT, kDepth, true, kWQ4K, KS, kWQ4K, TL><<<grid, 128 * KS, dyn, s>>>(a);
  } else {
    q4k_mfma_kernel<KIND, ACC, BF16OUT, kDepth, false, kWQ4K, KS, kWQ4K, TL><<<grid, 128 * KS, 0, s>>>(a);
  }
  return launch_status();
}

// the instantiation of (KIND, ACC, BF16OUT) for the weight format
template <int KIND, bool ACC, bool BF16OUT>
int launch_fmt(int fmt, const Args &a, hipStream_t s) {
  if (fmt == QMM_Q6_K) return launch<KIND, ACC, BF16OUT, kWQ6K>(a, s);
  if (fmt == QMM_Q4_0) return launch<KIND, ACC, BF16OUT, kWQ40>(a, s);
  if (fmt == QMM_Q4_KT) return launch<KIND, ACC, BF16OUT, kWQ4K, true>(a, s);
  return launch<KIND, ACC, BF16OUT, kWQ4K>(a, s);
}

// A gate/up pair in two formats (kSwiglu dense rows, kGU expert tiles): gate format WG, up format WU. Two K-parts
// (one wave a SIMD): the register rings of both formats would spill at two waves a SIMD.
template <int KIND, bool BF16OUT, int WG, int WU>
int launch_pair(const Args &a, hipStream_t s) {
  constexpr bool kDenseRows = KIND == kSwiglu;
  constexpr int KS = 2;
  const dim3 grid((unsigned)(kDenseRows ? 8 * ((a.tiles_total + 7) / 8) : 8 * a.n_blocks * ((a.tiles_m + 7) / 8)));
  q4k_mfma_kernel<KIND, false, BF16OUT, kDepth, false, WG, KS, WU><<<grid, 128 * KS, 0, s>>>(a);
  return launch_status();
}
int wfmt_of(int fmt) { return fmt == QMM_Q6_K ? kWQ6K : fmt == QMM_Q4_0 ? kWQ40 : kWQ4K; }
template <int KIND, bool BF16OUT, int WG>
int launch_pair_up(int wu, const Args &a, hipStream_t s) {
  if (wu == kWQ6K) return launch_pair<KIND, BF16OUT, WG, kWQ6K>(a, s);
  if (wu == kWQ40) return launch_pair<KIND, BF16OUT, WG, kWQ40>(a, s);
  return launch_pair<KIND, BF16OUT, WG, kWQ4K>(a, s);
}
template <int KIND, bool BF16OUT>
int launch_mixed(int fg, int fu, const Args &a, hipStream_t s) {
  const int wg = wfmt_of(fg), wu = wfmt_of(fu);
  if (wg == kWQ6K) return launch_pair_up<KIND, BF16OUT, kWQ6K>(wu, a, s);
  if (wg == kWQ40) return launch_pair_up<KIND, BF16OUT, kWQ40>(wu, a, s);
  return launch_pair_up<KIND, BF16OUT, kWQ4K>(wu, a, s);
}
bool gguf_gemm_fmt(int f) { return f == QMM_Q4_K || f == QMM_Q6_K || f == QMM_Q4_0; }

// bytes per row of K values, and the weight alignment the loads need (Q4_K: 16; Q6_K: 4, super-blocks realigned from
// even addresses; Q4_0: 2, 16-byte code runs read from even addresses)
int64_t fmt_row_bytes(int fmt, int64_t k) {
  return fmt == QMM_Q4_0 ? k / 32 * 18 : k / 256 * (fmt == QMM_Q6_K ? 210 : 144);
}
int fmt_align(int fmt) { return fmt == QMM_Q4_K || fmt == QMM_Q4_KT ? 16 : fmt == QMM_Q6_K ? 4 : 2; }

}  // namespace

// the dense Q4_K GEMM (gemm_dense.hip): store / acc modes, GGUF or tiled weights
int qmm_gemm_q4k_dense(int acc, int tiled, int64_t rows, int64_t k, int64_t n, const void *x, const float *scales,
                       const void *w, void *y, int y_bf16, hipStream_t s);

extern "C" int qmm_gemm(int fmt, int mode, int64_t rows, int64_t k, int64_t n, const void *x, int x_dtype,
                        const float *scales, const void *w, const void *w2, void *y, int y_dtype,
                        qmm_stream_t stream) {
  if (!fmt_code_ok(fmt)) return QMM_ERR_FORMAT;
  const int fu = fmt_up(fmt);   // QMM_GATE_UP(gate, up): the up matrix of the swiglu mode in its own format
  const bool mixed = fmt_mixed(fmt);
  fmt = fmt_gate(fmt);
  if (mixed && (mode != QMM_GEMM_SWIGLU || !gguf_gemm_fmt(fmt) || !gguf_gemm_fmt(fu))) return QMM_ERR_FORMAT;
  const bool tiled = fmt == QMM_Q4_KT;   // the decode GEMV's tiled Q4_K: one weight copy for decode and prefill
  if (!gguf_gemm_fmt(fmt) && !tiled) return QMM_ERR_FORMAT;   // MXFP4: qmm_gemm_mxfp4
  if (mode != QMM_GEMM_STORE && mode != QMM_GEMM_ACC && mode != QMM_GEMM_SWIGLU) return QMM_ERR_RANGE;
  if (!x || !w || !y || (mode == QMM_GEMM_SWIGLU && !w2)) return QMM_ERR_NULL;
  if (x_dtype != QMM_F16) return QMM_ERR_DTYPE;   // bf16 / f32 rows go through qmm_row_scale_f16 first
  if (y_dtype != QMM_F32 && y_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (rows <= 0 || n <= 0 || k <= 0 || k % 256) return QMM_ERR_SHAPE;
  if (rows > (1 << 24) || n > (1 << 24) || k > (1 << 20)) return QMM_ERR_SHAPE;
  if (tiled && (n % 16 || k % 512)) return QMM_ERR_SHAPE;   // whole 16-row blocks of whole 512-value units
  const int wal = fmt_align(fmt);
  if (!aligned(x, 16) || !aligned(w, wal) || !aligned(y, 4) || (w2 && !aligned(w2, fmt_align(fu))))
    return QMM_ERR_ALIGN;
  if (rows * k * 2 >= (1ll << 31)) return QMM_ERR_SHAPE;   // activation rows are addressed by a 32-bit buffer offset
  if (n * fmt_row_bytes(fmt, k) >= (1ll << 31) || n * fmt_row_bytes(fu, k) >= (1ll << 31))
    return QMM_ERR_SHAPE;   // so are the weight rows (buffer size, offsets)
  Args a{};
  a.M = (int)rows; a.N = (int)n; a.K = (int)k;
  a.x16 = static_cast<const _Float16 *>(x); a.scales = scales; a.x_rows = (int)rows;
  a.w = static_cast<const u8 *>(w); a.w2 = static_cast<const u8 *>(w2); a.y = y;
  a.tiles_m = (int)((rows + BM - 1) / BM);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool acc = mode == QMM_GEMM_ACC, bf = y_dtype == QMM_BF16;
  if (mode == QMM_GEMM_SWIGLU) {   // 64 output columns a workgroup: its wave pairs take the gate and the up matrix
    a.tiles_total = a.tiles_m * (int)((n + 63) / 64);
    if (mixed) return bf ? launch_mixed<kSwiglu, true>(fmt, fu, a, s) : launch_mixed<kSwiglu, false>(fmt, fu, a, s);
    return bf ? launch_fmt<kSwiglu, false, true>(fmt, a, s) : launch_fmt<kSwiglu, false, false>(fmt, a, s);
  }
  if (fmt == QMM_Q4_K || tiled) return qmm_gemm_q4k_dense(acc, tiled, rows, k, n, x, scales, w, y, bf, s);
  a.tiles_total = a.tiles_m * (int)((n + 127) / 128);
  if (acc && bf) return launch_fmt<kDense, true, true>(fmt, a, s);
  if (acc) return launch_fmt<kDense, true, false>(fmt, a, s);
  if (bf) return launch_fmt<kDense, false, true>(fmt, a, s);
  return launch_fmt<kDense, false, false>(fmt, a, s);
}

int qmm_grouped_q4k_narrow(int tiled, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E,
                           int KU, const int32_t *tile_info, const int32_t *rowmap, const void *x,
                           const float *x_scales, int64_t x_rows, const void *w, const void *w2, const float *bias,
                           const float *bias2, float *y, hipStream_t s);
bool qmm_grouped_narrow_fits(int64_t k, int64_t n);
#ifndef QMM_NARROW_ROWS
#define QMM_NARROW_ROWS 8
#endif
constexpr int64_t kNarrowRowsPerExpert = QMM_NARROW_ROWS;   // mean assignments an expert up to which it applies

// The Q4_K / Q6_K / Q4_0 path of qmm_moe_grouped (grouped.hip checks the arguments shared with the MXFP4 path).
int qmm_grouped_q4k(int fmt, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E, int KU,
                    const int32_t *tile_info, const int32_t *rowmap, const void *x, const float *x_scales,
                    int64_t x_rows, const void *w, const void *w2, const float *bias, const float *bias2, float *y,
                    hipStream_t s) {
  if (k % 256) return QMM_ERR_SHAPE;
  if (x_rows * k * 2 >= (1ll << 31)) return QMM_ERR_SHAPE;   // activation rows are addressed by a 32-bit buffer offset
  if (fmt_mixed(fmt)) {
    // QMM_GATE_UP(gate, up), gate/up of two tensors in GGUF blocks: the 64-row tile kernel, the up waves in the up
    // format (g_moe_ggu_{fg}_{fu}, S/gen_moe.py:1126-1141)
    const int fg = fmt_gate(fmt), fu = fmt_up(fmt);
    if (mode != 0 || fused || !gguf_gemm_fmt(fg) || !gguf_gemm_fmt(fu)) return QMM_ERR_FORMAT;
    if (!aligned(x, 16) || !aligned(w, fmt_align(fg)) || !aligned(w2, fmt_align(fu))) return QMM_ERR_ALIGN;
    Args a{};
    a.M = (int)(max_tiles * BM); a.N = (int)n; a.K = (int)k;
    a.x16 = static_cast<const _Float16 *>(x); a.scales = x_scales; a.x_rows = (int)x_rows;
    a.tile_info = tile_info; a.rowmap = rowmap; a.KU = KU; a.E = E; a.act = act; a.y = y;
    a.bias = bias; a.bias2 = bias2;
    a.w = static_cast<const u8 *>(w); a.w2 = static_cast<const u8 *>(w2);
    a.ebytes = fmt_row_bytes(fg, k) * n;
    a.ebytes2 = fmt_row_bytes(fu, k) * n;
    a.up_off = 0;
    a.n_blocks = (int)((n + 63) / 64);
    a.tiles_m = (int)max_tiles;
    a.tiles_total = (int)max_tiles * a.n_blocks;
    return launch_mixed<kGU, false>(fg, fu, a, s);
  }
  const int wal = fmt_align(fmt);
  if (!aligned(x, 16) || !aligned(w, wal) || (w2 && !aligned(w2, wal))) return QMM_ERR_ALIGN;
  // The tiled layout: the narrow kernel wherever it fits (at every batch size, so a token's output does not depend
  // on the batch), else (K beyond the narrow kernel's LDS rows) the 64-row tile kernel, which reads it in whole units
  // (K % 512 == 0, n % 16 == 0). GGUF Q4_K with few rows an expert (max_tiles = assignments / 64 + E, so
  // 64 (max_tiles - E) bounds the assignments): the narrow kernel too, which streams each expert's weights once
  // against 16-row groups held in LDS.
  const bool narrow = qmm_grouped_narrow_fits(k, n);
  if (fmt == QMM_Q4_KT && (narrow || k % 512 || n % 16)) {
    if (!narrow) return QMM_ERR_SHAPE;
    if (!aligned(y, 16)) return QMM_ERR_ALIGN;
    return qmm_grouped_q4k_narrow(1, mode, fused, act, max_tiles, k, n, E, KU, tile_info, rowmap, x, x_scales, x_rows,
                                  w, w2, bias, bias2, y, s);
  }
  if (fmt == QMM_Q4_K && narrow && aligned(y, 16) && 64 * (max_tiles - E) <= kNarrowRowsPerExpert * E)
    return qmm_grouped_q4k_narrow(0, mode, fused, act, max_tiles, k, n, E, KU, tile_info, rowmap, x, x_scales, x_rows,
                                  w, w2, bias, bias2, y, s);
  const int64_t RB = fmt_row_bytes(fmt, k);
  Args a{};
  a.M = (int)(max_tiles * BM); a.N = (int)n; a.K = (int)k;
  a.x16 = static_cast<const _Float16 *>(x); a.scales = x_scales; a.x_rows = (int)x_rows;
  a.tile_info = tile_info; a.rowmap = rowmap; a.KU = KU; a.E = E; a.act = act; a.y = y;
  a.bias = bias; a.bias2 = mode == 0 ? bias2 : nullptr;
  a.w = static_cast<const u8 *>(w);
  if (mode == 0) {
    if (!fused && !w2) return QMM_ERR_NULL;
    a.ebytes = RB * n * (fused ? 2 : 1);
    a.ebytes2 = RB * n;
    a.up_off = fused ? RB * n : 0;
    a.w2 = fused ? nullptr : static_cast<const u8 *>(w2);
    a.n_blocks = (int)((n + 63) / 64);
    a.tiles_m = (int)max_tiles;
    a.tiles_total = (int)max_tiles * a.n_blocks;
    return launch_fmt<kGU, false, false>(fmt, a, s);
  }
  a.ebytes = RB * n;
  a.n_blocks = (int)((n + 127) / 128);
  a.tiles_m = (int)max_tiles;
  a.tiles_total = (int)max_tiles * a.n_blocks;
  return launch_fmt<kDN, false, false>(fmt, a, s);
}
