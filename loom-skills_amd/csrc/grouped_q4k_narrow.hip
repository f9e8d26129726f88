// Grouped expert GEMMs over expert tiles that hold few rows: g_moe_ggu_q4_k[_fused]_k{H} / g_moe_gdn_q4_k_k{FE}
// (S/gen_moe.py:1126-1228) in the regime where a prefill batch gives each expert a handful of rows (Qwen3-30B-A3B,
// 64 tokens, top-8 of 128 experts: about four rows an expert). The arithmetic is the 64-row-tile kernel's
// (gemm_q4k.hip): row-scaled f16 activations, Q4_K weights staged to f16 as fma_f16(f16(q), f16(d sc), f16(-dmin m))
// (S/gen_gemm.py:499-530), fp32 accumulation, the row inverse, the expert biases and the activation in the
// epilogue (S/gen_moe.py:958-1007).
//
// There the weights are the bound: every expert's gate, up and down matrices are read once per layer, and the rows
// that multiply them are few. So the design is a weight stream with the activations held still:
//   - a workgroup takes one group of 16 rows of one expert tile (the N of v_mfma_f32_16x16x32_f16) and NW waves of
//     weight rows. The group's activation rows (all of K, f16) are staged into LDS once, in 16-byte chunks ordered
//     (k / 8, row) so the 16 lanes that read one K octet read 256 contiguous bytes; then the waves stream their
//     weights with no barrier at all.
//   - a wave owns two groups of 16 weight rows (gate/up: the same 16 columns of both matrices, so the activation
//     is applied in registers; down: 32 consecutive columns) and walks K in steps of 128 values, DEPTH steps of
//     loads in flight. Lane (c, q) = (lane % 16, lane / 16) loads 16 code bytes of weight row c per step: page
//     2 (step & 1) + q / 2 of the super-block, bytes 16 (q & 1) .. +15, i.e. values 16 (q & 1) .. +15 of the
//     page's two sub-blocks (low nibbles: sub-block 2 page, high: 2 page + 1), and the super-block's 16-byte
//     header (same cache lines). Its (d sc, -dmin m) pairs are decoded per step with two f16 multiplies.
//   - each (nibble, half) of those 16 bytes is one 16x16x32 MFMA: the weights are the A operand (16 weight rows x
//     the lane quarter's 8 K values), the activation rows the B operand read from LDS at the same K.
//   - the output fragment holds 4 consecutive output columns of one row per lane: one 16-byte store, only for rows
//     that hold an assignment (dead rows and unused tiles are not written).
// Row groups of a tile past its row count (tile_info[tile, 1], the bucket fills tiles from the top) exit at once;
// with few rows an expert the grid lists every tile's first row group before any second one, otherwise a tile's row
// groups are neighbours (they read the same weights, from L2 for all but the first).
//
// Weight layouts. GGUF rows as they are (above): one load instruction then reads 64 bytes of each of 16 rows, 1152
// bytes apart. The tiled layout QMM_Q4_KT (qmm_tile_q4k) stores each 16-row block as units of 512 values, 4608
// bytes: 32 headers, then four 1 KB planes, plane p holding at 16 (4 r + 2 sb + h) the code bytes 16 (4 h + p) .. of
// super-block sb of row r (a half unit of 2304 bytes ends the block when K % 512 == 256). There lane (c, q) of a
// step s_u of a unit reads plane s_u at 16 (4 c + q): super-block q / 2, half q % 2, page 2 (q % 2) + s_u / 2, bytes
// 16 (s_u % 2) .. of it, so the wave reads one contiguous kilobyte a step; its header (super-block q / 2 of row c)
// comes once a unit, and its four sub-block scale pairs (sub-blocks 4 (q % 2) .. + 3) are decoded once a unit. In
// the half unit lane (c, q) reads plane 2 s_u + q / 2 at 16 (2 c + q % 2): page 2 (q % 2) + s_u, bytes 16 (q / 2).
// The activation rows are read at exactly the K positions each lane's weights hold, so the MFMA sums the same
// products in another order.
#include "common.hpp"
#include "deq_f16.hpp"

#include <type_traits>

using namespace qmm;

namespace {

constexpr int kGroupRows = 16;   // activation rows per workgroup: the N of the 16x16x32 MFMA
constexpr int kTileRows = 64;    // rows of a bucketed expert tile
constexpr int kStepK = 128;      // K values a step: half a Q4_K super-block
constexpr int64_t kNarrowMaxK = 4096;   // largest K whose activation panel (16 rows x K f16) fits a workgroup's LDS
enum NKind { kNGU = 0, kNDN = 1 };

typedef __attribute__((ext_vector_type(4))) u32 u32x4;

struct NArgs {
  int N, K;                    // output columns (gu: FE, dn: H) and the reduction length
  const _Float16 *x16;         // gu: token rows [x_rows, K]; dn: sorted rows [max_rows, K]
  const float *scales;         // [rows of x16, 2] (inverse in [row, 1]) or NULL
  int x_rows;
  const u8 *w, *w2;            // gu: gate (or fused gate_up) and up tensors; dn: down
  int64_t ebytes, up_off;      // bytes of one expert's tensor; gu fused: offset of the up rows
  const int32_t *tile_info, *rowmap;
  const float *bias, *bias2;   // [E, N] or NULL
  int KU, E, act;
  u32 ku_magic;                // ceil(2^32 / KU) for KU > 1: token = umulhi(assignment, ku_magic)
  float *y;                    // [max_tiles * 64, N]
  int tiles, col_blocks;       // tiles of the table; workgroups across N per row group
  int rg_outer;                // grid order: row groups outermost (few rows an expert) or beside their tile
};

// (d sc_g, -dmin m_g) f16 pairs, each broadcast to both halves, of the two sub-blocks 2 pg and 2 pg + 1 a lane
// needs in a step: PAR = step & 1 (sub-blocks 0..3 or 4..7), sel = the perm selector of the lane's byte pair.
template <int PAR>
__device__ __forceinline__ void step_scales(const uint4 &hd, u32 sel0, u32 sel1, h2 (&dsc)[2], h2 (&nmn)[2]) {
  u32 scw, mnw;
  if constexpr (PAR == 0) {   // sub-blocks 0..3: 6-bit fields in bytes of S[0..3] / S[4..7]
    scw = hd.y & 0x3F3F3F3Fu;
    mnw = hd.z & 0x3F3F3F3Fu;
  } else {                    // 4..7: low 4 bits in S[8..11], high 2 bits in the top of S[0..3] / S[4..7]
    scw = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
    mnw = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  }
  const h2 dm = as_h2(hd.x ^ 0x80000000u);     // (d, -dmin)
  const h2 m1024 = as_h2(0xE400E400u);
  const u32 p[2] = {__builtin_amdgcn_perm(mnw, scw, sel0) | 0x64006400u,
                    __builtin_amdgcn_perm(mnw, scw, sel1) | 0x64006400u};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    // (1024 + sc, 1024 + m) - 1024 is exact; one rounding multiply = f16 of the exact f32 product d sc
    const u32 v = as_u32((as_h2(p[i]) + m1024) * dm);
    dsc[i] = as_h2(__builtin_amdgcn_perm(v, v, 0x01000100u));
    nmn[i] = as_h2(__builtin_amdgcn_perm(v, v, 0x03020302u));
  }
}

// The four MFMAs of one group-step: lane (c, q)'s 16 code bytes cq hold (low nibbles, sub-block A) and (high nibbles,
// sub-block B) of 16 consecutive values; (nibble, half) is one 8-value K octet, read from the LDS panel at chunk
// k8 + 4 nibble + half.
__device__ __forceinline__ void group_step(const uint4 (&cq)[2], const h2 (&dsc)[2][2], const h2 (&nmn)[2][2],
                                           const uint4 *xs, int k8, int lc, f32x4 (&acc)[2]) {
#pragma unroll
  for (int nib = 0; nib < 2; ++nib)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f16x8 bx = __builtin_bit_cast(f16x8, xs[(k8 + 4 * nib + half) * kGroupRows + lc]);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const u32 w0 = half ? cq[g].z : cq[g].x, w1 = half ? cq[g].w : cq[g].y;
        const f16x8 aw = nib ? deq8_e4m3<true>(w0, w1, dsc[g][1], nmn[g][1])
                             : deq8_e4m3<false>(w0, w1, dsc[g][0], nmn[g][0]);
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aw, bx, acc[g], 0, 0, 0);
      }
    }
}

// (d sc, -dmin m) of the four sub-blocks 4 h .. 4 h + 3 of a super-block header (h = 0: sub-blocks 0..3, 1: 4..7;
// per lane), each broadcast to both halves: the tiled layout's once-a-unit decode.
__device__ __forceinline__ void unit_scales(const uint4 &hd, u32 hmask, h2 (&dsc)[4], h2 (&nmn)[4]) {
  // both field sets, merged by the lane's mask (all ones for h = 1): a bit select, not a branch
  const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u), sc_lo = hd.y & 0x3F3F3F3Fu;
  const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u), mn_lo = hd.z & 0x3F3F3F3Fu;
  const u32 scw = (sc_hi & hmask) | (sc_lo & ~hmask), mnw = (mn_hi & hmask) | (mn_lo & ~hmask);
  const h2 dm = as_h2(hd.x ^ 0x80000000u);     // (d, -dmin)
  const h2 m1024 = as_h2(0xE400E400u);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32 sel = (u32)i | (0x0Cu << 8) | ((4u + i) << 16) | (0x0Cu << 24);
    const u32 v = as_u32((as_h2(__builtin_amdgcn_perm(mnw, scw, sel) | 0x64006400u) + m1024) * dm);
    dsc[i] = as_h2(__builtin_amdgcn_perm(v, v, 0x01000100u));
    nmn[i] = as_h2(__builtin_amdgcn_perm(v, v, 0x03020302u));
  }
}

// s_waitcnt immediate that waits until at most n vector memory loads are outstanding (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int KIND, int NW, int DEPTH, bool TILED>
__global__ __launch_bounds__(64 * NW) void q4k_narrow_kernel(NArgs a) {
  static_assert(DEPTH % 2 == 0, "a step's parity is static inside the unrolled step loop");
  static_assert(!TILED || DEPTH == 4, "the tiled layout streams one unit (four steps) a loop iteration");
  extern __shared__ __align__(16) uint4 xs[];   // [K / 8][16 rows]
  __shared__ int src_row[kGroupRows];
  __shared__ float rinv[kGroupRows];
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N, K = a.K;

  int cb, tile, rg;
  {
    const int b = (int)blockIdx.x;
    if (a.rg_outer) {   // [row group][tile][column block]
      cb = b % a.col_blocks;
      tile = (b / a.col_blocks) % a.tiles;
      rg = b / a.col_blocks / a.tiles;
    } else {            // [tile][row group][column block]
      cb = b % a.col_blocks;
      rg = (b / a.col_blocks) & 3;
      tile = b / a.col_blocks / 4;
    }
  }
  const int expert0 = a.tile_info[2 * tile], tile_rows = a.tile_info[2 * tile + 1];
  if ((expert0 < 0) | (kGroupRows * rg >= tile_rows)) return;   // uniform over the workgroup; one load for both
  const int expert = expert0 >= a.E ? a.E - 1 : expert0;
  const int r0 = tile * kTileRows + kGroupRows * rg;

  // ---- this lane's weight rows (GGUF: row c0 + lc of each group; tiled: the group's 16-row block), issued first so
  // the stream starts while the activations are staged
  const int lc = lane & 15, q = lane >> 4;
  const int c0 = (cb * NW + wave) * (KIND == kNGU ? 16 : 32);   // first output column of the wave (a multiple of 16)
  const int64_t RB = (int64_t)K / 256 * 144;
  const u8 *wrow[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    int c = c0 + (KIND == kNGU ? 0 : 16 * g) + (TILED ? 0 : lc);
    c = c < N ? c : (TILED ? N - 16 : N - 1);
    const u8 *base;
    if constexpr (KIND == kNGU) {
      const u8 *gate = a.w + (int64_t)expert * a.ebytes;
      base = g == 0 ? gate : (a.w2 ? a.w2 + (int64_t)expert * a.ebytes : gate + a.up_off);
    } else {
      base = a.w + (int64_t)expert * a.ebytes;
    }
    wrow[g] = base + (int64_t)c * RB;
  }
  const int S = K / kStepK;
  // GGUF: byte of the lane's 16 codes within the step's two pages
  const int qoff = 32 * (q >> 1) + 16 * (q & 1);
  auto ld_step = [&](int s, uint4 (&cq)[2], uint4 (&hd)[2]) __attribute__((always_inline)) {
    const int st = s < S ? s : S - 1;
    const int64_t sb = (int64_t)(st >> 1) * 144;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      cq[g] = ld16(wrow[g] + sb + 16 + 64 * (st & 1) + qoff);
      hd[g] = ld16(wrow[g] + sb);
    }
  };
  // tiled: per-lane byte offsets of the code piece (full unit: + 1024 s_u; half unit: + 1024 s_u) and the header
  const int F = K / 512;
  const bool half_unit = (K / 256) & 1;
  const int cf = 512 + 16 * (4 * lc + q), chh = 256 + 512 * (q >> 1) + 16 * (2 * lc + (q & 1));
  const int hf = 16 * (2 * lc + (q >> 1)), hh = 16 * lc;
  uint4 cring[DEPTH][2], hring[DEPTH][2], hnext[2];
  auto prefetch = [&]() __attribute__((always_inline)) {
    if constexpr (TILED) {   // unit 0 (or the half unit when K == 256): header, then codes, as the loop issues them
#pragma unroll
      for (int g = 0; g < 2; ++g) hnext[g] = ld16(wrow[g] + (F > 0 ? hf : hh));
#pragma unroll
      for (int su = 0; su < 4; ++su) {
        const int lo = F > 0 ? cf : chh;
#pragma unroll
        for (int g = 0; g < 2; ++g) cring[su][g] = ld16(wrow[g] + lo + 1024 * (F > 0 || su < 2 ? su : 0));
      }
    } else {
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) ld_step(u, cring[u], hring[u]);
    }
  };

  // ---- the weight prefetch first (it needs only the expert), then the row group's rows and inverse scales as
  // scalar loads (uniform addresses: they do not enter the vector load counter, so reading them does not wait for
  // the weights), then the activation rows into LDS (rows without an assignment: zeros, not read). gu: row i of the
  // group is assignment rowmap[r0 + i], of token rowmap[r0 + i] / KU; dn: the sorted row r0 + i itself when
  // 16 rg + i < tile_rows (the bucket fills a tile's rows from the top); the row map decides which rows are stored.
  prefetch();
  __builtin_amdgcn_sched_barrier(0);
  auto dn_row = [&](int i) { return kGroupRows * rg + i < tile_rows && r0 + i < a.x_rows ? r0 + i : -1; };
  const int own = tid & 15;   // the row this thread stages
  int rmv[kGroupRows], srv[kGroupRows];
  float invv[kGroupRows];
#pragma unroll
  for (int i = 0; i < kGroupRows; ++i) rmv[i] = a.rowmap[r0 + i];   // all issued before any is used
#pragma unroll
  for (int i = 0; i < kGroupRows; ++i) {
    if constexpr (KIND == kNGU) {
      const int tok = a.KU == 1 ? rmv[i] : (int)__umulhi((u32)rmv[i], a.ku_magic);
      srv[i] = (rmv[i] >= 0) & (tok < a.x_rows) ? tok : -1;
    } else {
      srv[i] = dn_row(i);
    }
  }
  if (a.scales) {
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) invv[i] = a.scales[2 * (srv[i] >= 0 ? srv[i] : 0) + 1];
  } else {
#pragma unroll
    for (int i = 0; i < kGroupRows; ++i) invv[i] = 1.f;
  }
  int rm_own = rmv[0], srow = srv[0];
  float inv_own = invv[0];
#pragma unroll
  for (int i = 1; i < kGroupRows; ++i) {
    rm_own = own == i ? rmv[i] : rm_own;
    srow = own == i ? srv[i] : srow;
    inv_own = own == i ? invv[i] : inv_own;
  }
  {
    // 16-byte chunks of the panel, row fastest: thread t stages chunks t, t + NT, ... (16 K / 8 / NT of them).
    // The loads go through a buffer resource over the activation rows; a row past them (or, for gu, without an
    // assignment) gets an offset past their end, where the hardware returns zeros without a memory access, so the
    // loop has no branch.
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16 *>(a.x16), (short)0, (int)((int64_t)a.x_rows * K * 2), 0x00020000);
    const u32 rbase = srow >= 0 ? (u32)srow * (u32)K * 2u : 0x80000000u;
    const int per = K / 8 * kGroupRows / NT;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // straight into LDS (buffer_load ... lds: no registers, no store instructions); the wave's 64 lanes fill 64
    // consecutive chunks, so the LDS destination is one wave-uniform address a load
#pragma unroll 8
    for (int i = 0; i < per; ++i) {
      const int c = i * NT + tid;   // chunk c: row c % 16 (= tid % 16), k8 c / 16
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (__attribute__((address_space(3))) void *)&xs[i * NT + 64 * wave_u], 16,
          (int)(srow >= 0 ? rbase + 16u * (u32)(c >> 4) : rbase), 0, 0, 0);
    }
  }
  if (tid < kGroupRows) {   // the rows the epilogue stores, with their inverse scales
    src_row[tid] = rm_own >= 0 ? srow : -1;
    rinv[tid] = srow >= 0 ? inv_own : 1.f;
  }
  // the weight prefetch and the staging loads (the first unit needs both)
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  if constexpr (TILED) {
    // ---- one unit (four steps) an iteration; the next unit's header and codes are issued as this unit's are used.
    // NEXT (compile time): 0 the next full unit, 1 the half unit (two steps), 2 nothing: the loop body has no
    // run-time choice, so the compiler's load waits stay a unit deep.
    const u32 hq = 0u - (u32)(q & 1);   // the lane's sub-block half as a mask
    const int kbf = 32 * (q >> 1) + 16 * (q & 1), kbh = 16 * (q & 1) + 2 * (q >> 1);
    auto unit = [&](int u, auto next) __attribute__((always_inline)) {
      constexpr int NEXT = decltype(next)::value;
      h2 usc[2][4], umn[2][4];
#pragma unroll
      for (int g = 0; g < 2; ++g) unit_scales(hnext[g], hq, usc[g], umn[g]);
      if constexpr (NEXT < 2) {   // the next unit's header first: needed before any of its codes
        const int ho = NEXT == 0 ? 4608 * (u + 1) + hf : 4608 * F + hh;
#pragma unroll
        for (int g = 0; g < 2; ++g) hnext[g] = ld16(wrow[g] + ho);
      }
#pragma unroll
      for (int su = 0; su < 4; ++su) {
        h2 dsc[2][2], nmn[2][2];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int nib = 0; nib < 2; ++nib) {
            dsc[g][nib] = usc[g][2 * (su >> 1) + nib];
            nmn[g][nib] = umn[g][2 * (su >> 1) + nib];
          }
        group_step(cring[su], dsc, nmn, xs, 64 * u + kbf + 8 * (su >> 1) + 2 * (su & 1), lc, acc);
        if constexpr (NEXT == 0) {
#pragma unroll
          for (int g = 0; g < 2; ++g) cring[su][g] = ld16(wrow[g] + 4608 * (u + 1) + cf + 1024 * su);
        } else if constexpr (NEXT == 1) {
          if (su < 2) {
#pragma unroll
            for (int g = 0; g < 2; ++g) cring[su][g] = ld16(wrow[g] + 4608 * F + chh + 1024 * su);
          }
        }
        // keep the loads where they are issued: the scheduler would otherwise sink them towards their use to save
        // registers, and the stream would lose its prefetch distance
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (F > 0) {
      for (int u = 0; u + 1 < F; ++u) unit(u, std::integral_constant<int, 0>{});
      if (half_unit) unit(F - 1, std::integral_constant<int, 1>{});
      else unit(F - 1, std::integral_constant<int, 2>{});
    }
    if (half_unit) {   // the half unit: two steps, sub-block pairs 2 s_u + nib of the lane's four
      h2 usc[2][4], umn[2][4];
#pragma unroll
      for (int g = 0; g < 2; ++g) unit_scales(hnext[g], hq, usc[g], umn[g]);
#pragma unroll
      for (int su = 0; su < 2; ++su) {
        h2 dsc[2][2], nmn[2][2];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int nib = 0; nib < 2; ++nib) {
            dsc[g][nib] = usc[g][2 * su + nib];
            nmn[g][nib] = umn[g][2 * su + nib];
          }
        group_step(cring[su], dsc, nmn, xs, 64 * F + kbh + 8 * su, lc, acc);
      }
    }
  } else {
    // ---- GGUF: per step 2 groups x (2 nibbles x 2 halves) MFMAs
    const u32 b0 = 2 * (q >> 1);   // byte of sub-block 2 pg (page pg = 2 (step & 1) + q / 2) in the field dwords
    const u32 sel0 = b0 | (0x0Cu << 8) | ((4 + b0) << 16) | (0x0Cu << 24);
    const u32 sel1 = sel0 + 0x00010001u;
    const int xoff = 8 * (q >> 1) + 2 * (q & 1);   // K octet of the lane's first value within a step, in chunks
    // S is a multiple of DEPTH (the launch picks DEPTH so): no padding step, no branch in the loop body, so the
    // compiler's load waits stay DEPTH - 1 steps deep
    for (int s0 = 0; s0 < S; s0 += DEPTH) {
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) {
        const int s = s0 + u;
        h2 dsc[2][2], nmn[2][2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          if (u & 1) step_scales<1>(hring[u][g], sel0, sel1, dsc[g], nmn[g]);
          else step_scales<0>(hring[u][g], sel0, sel1, dsc[g], nmn[g]);
        }
        group_step(cring[u], dsc, nmn, xs, 16 * s + xoff, lc, acc);
        ld_step(s + DEPTH, cring[u], hring[u]);
        __builtin_amdgcn_sched_barrier(0);   // the loads stay DEPTH steps ahead (no sinking towards their use)
      }
    }
  }

  // ---- epilogue: lane (lc, q) holds output columns 4 q .. 4 q + 3 of its group for row r0 + lc
  const int src = src_row[lc];
  const float inv = rinv[lc];
  float *yrow = a.y + (int64_t)(r0 + lc) * N;
  if constexpr (KIND == kNGU) {
    if (src < 0) return;
    const int f = c0 + 4 * q;
    if (f >= N) return;
    f32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float bg = a.bias ? a.bias[(int64_t)expert * N + f + i] : 0.f;
      const float bu = a.bias2 ? a.bias2[(int64_t)expert * N + f + i] : 0.f;
      o[i] = act_fn(a.act, acc[0][i] * inv + bg, acc[1][i] * inv + bu);
    }
    *reinterpret_cast<f32x4 *>(yrow + f) = o;
  } else {
    if (src >= 0) {
      // both groups' outputs (and their bias loads) before any store, so no store waits for another
      f32x4 o[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int f = c0 + 16 * g + 4 * q, fb = f < N ? f : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[g][i] = acc[g][i] * inv + (a.bias ? a.bias[(int64_t)expert * N + fb + i] : 0.f);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int f = c0 + 16 * g + 4 * q;
        if (f >= N) continue;
        *reinterpret_cast<f32x4 *>(yrow + f) = o[g];
      }
    }
  }
}

template <int KIND, int NW, int DEPTH, bool TILED>
int launch_narrow(const NArgs &a, hipStream_t s) {
  const size_t lds = (size_t)a.K / 8 * kGroupRows * 16;
  if (lds > 32768) {
    static std::atomic<unsigned> raised{0};
    if (int st = raise_dyn_lds(reinterpret_cast<const void *>(&q4k_narrow_kernel<KIND, NW, DEPTH, TILED>),
                               (int)(kNarrowMaxK / 8 * kGroupRows * 16), raised))
      return st;
  }
  const unsigned grid = (unsigned)(4 * a.tiles * a.col_blocks);
  q4k_narrow_kernel<KIND, NW, DEPTH, TILED><<<grid, 64 * NW, lds, s>>>(a);
  return launch_status();
}

// GGUF: DEPTH divides the step count S = K / 128 (even, since K % 256 == 0); tiled: one unit an iteration
template <int KIND, int NW>
int launch_depth(const NArgs &a, bool tiled, hipStream_t s) {
  if (tiled) return launch_narrow<KIND, NW, 4, true>(a, s);
  const int S = a.K / kStepK;
  if (S % 4 == 0) return launch_narrow<KIND, NW, 4, false>(a, s);
  if (S % 6 == 0) return launch_narrow<KIND, NW, 6, false>(a, s);
  return launch_narrow<KIND, NW, 2, false>(a, s);
}

}  // namespace

#ifndef QMM_NARROW_WAVES_GU
#define QMM_NARROW_WAVES_GU 8
#endif
#ifndef QMM_NARROW_WAVES_DN
#define QMM_NARROW_WAVES_DN 4
#endif


// The narrow path of qmm_moe_grouped for Q4_K weights (gemm_q4k.hip's qmm_grouped_q4k decides when it applies).
int qmm_grouped_q4k_narrow(int tiled, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E,
                           int KU, const int32_t *tile_info, const int32_t *rowmap, const void *x,
                           const float *x_scales, int64_t x_rows, const void *w, const void *w2, const float *bias,
                           const float *bias2, float *y, hipStream_t s) {
  NArgs a{};
  a.rg_outer = 64 * (max_tiles - E) <= 8 * E;   // assignments (<= 64 (max_tiles - E)) up to 8 an expert
  a.N = (int)n; a.K = (int)k;
  a.x16 = static_cast<const _Float16 *>(x); a.scales = x_scales; a.x_rows = (int)x_rows;
  a.tile_info = tile_info; a.rowmap = rowmap; a.KU = KU; a.E = E; a.act = act; a.y = y;
  a.ku_magic = KU > 1 ? (u32)((0x100000000ull + (unsigned long long)KU - 1) / (unsigned long long)KU) : 0u;   // exact below 2^24
  a.bias = bias; a.bias2 = mode == 0 ? bias2 : nullptr;
  a.w = static_cast<const u8 *>(w);
  a.tiles = (int)max_tiles;
  const int64_t RB = k / 256 * 144;
  if (mode == 0) {
    a.ebytes = RB * n * (fused ? 2 : 1);
    a.up_off = fused ? RB * n : 0;
    a.w2 = fused ? nullptr : static_cast<const u8 *>(w2);
    a.col_blocks = (int)((n + 16 * QMM_NARROW_WAVES_GU - 1) / (16 * QMM_NARROW_WAVES_GU));
    return launch_depth<kNGU, QMM_NARROW_WAVES_GU>(a, tiled != 0, s);
  }
  a.ebytes = RB * n;
  a.col_blocks = (int)((n + 32 * QMM_NARROW_WAVES_DN - 1) / (32 * QMM_NARROW_WAVES_DN));
  return launch_depth<kNDN, QMM_NARROW_WAVES_DN>(a, tiled != 0, s);
}

bool qmm_grouped_narrow_fits(int64_t k, int64_t n) { return k % 256 == 0 && k <= kNarrowMaxK && n % 16 == 0; }
