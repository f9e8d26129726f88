// The dense Q4_K prefill GEMM g_gemm_q4_k_{store|acc} (S/gen_gemm.py:535-703) for GGUF Q4_K weights:
//
//   Y[r, c] = (acc ? Y[r, c] : 0) + inv[r] sum_k X16[r, k] W16[c, k]
//
// X16 is the row-scaled f16 operand of g_row_scale_f16 (S/gen_llm.py:1843-1915) and inv = scales[r, 1]; W16 is the
// weight staged to f16 the way the reference stages it, fma_f16(f16(q), f16(d sc), f16(-dmin m)) with one rounding
// (S/gen_gemm.py:499-530); fp32 accumulation.
//
// Design (gfx950: wave64, v_mfma_f32_32x32x16_f16, 160 KB LDS, 256 CUs in 8 XCDs). A workgroup computes a 64 x 128
// output tile over all of K; its four waves split K by super-blocks, and each wave computes the whole tile over its
// share (2 x 4 accumulators of 32 x 32), so every weight is dequantized once per workgroup and each dequantized
// fragment feeds two MFMAs, while each activation fragment feeds four. Nothing in the main loop synchronizes the
// workgroup:
//   - activations: a wave stages its own 64 rows x 64 values a step (a code page) through its own LDS area, double
//     buffered: coalesced 16-byte loads (eight lanes a 128-byte row piece) two steps ahead in registers, written to
//     LDS rows of 144 bytes (a row pitch of 16 mod 128 keeps the fragment reads free of bank conflicts);
//   - weights: a lane loads, for each of its four columns, the 16-byte code pieces of all four pages of a
//     super-block at once (with the header, whole 144-byte blocks are read together, so no cache line is fetched
//     twice), one super-block ahead, and dequantizes them in registers: a code byte 0000qqqq read as OCP E4M3 is
//     q 2^-9 exactly, so v_cvt_scalef32_pk_f16_fp8 with scale 512 gives the f16 codes (two a instruction), then one
//     v_pk_fma_f16 with (f16(d sc), f16(-dmin m)) -- the reference's single rounding;
//   - scales: the wave decodes the (f16(d sc), f16(-dmin m)) pairs of the next super-block's 128 columns into a
//     two-slot LDS table (two columns a lane, exact: (1024 + sc) - 1024 times d, one rounding), read as one 8-byte
//     LDS read per column a step;
//   - the four K-parts meet at the end through LDS in a fixed order ((p0 + p2) + (p1 + p3) for every output, so the
//     result does not depend on which wave stores it).
// MFMA operand order as in the other f16 MFMA kernels here: lane (lc, h) = (lane % 32, lane / 32) takes code bytes
// 16 h .. 16 h + 15 of a page; K16 step (gl, s2) of the page holds its values 16 h + 8 s2 .. + 7 of sub-block
// 2 page + gl, i.e. K positions 64 page + 32 gl + 16 h + 8 s2 .. + 7, where the activation fragment is read too.
// Tiles are dealt XCD-aware: the eight M tiles of an N tile run on one XCD and share its weight columns in L2.
//
// Weights in the tiled layout QMM_Q4_KT (qmm_tile_q4k, the decode GEMV's; K % 512 == 0, N % 16 == 0): the lane reads
// the same 16 code bytes and header, at their tiled addresses. Column c's block of 16 rows starts at (c / 16) 16 RB
// (RB = K / 256 * 144 bytes a row); super-block sb of its row r = c % 16 is half sb % 2 of unit sb / 2 (4608 bytes):
// header at 16 (2 r + sb % 2), and code bytes 16 (4 h' + q) .. + 15 in plane q at 512 + 1024 q + 16 (4 r + 2 (sb % 2)
// + h'). Page p's bytes 16 h .. + 15 are chunk 2 p + h: plane 2 (p % 2) + h, h' = p / 2. So the per-column part of an
// address is (c / 16) 16 RB + 512 + 1024 h + 64 r (codes) or + 32 r (header), and the rest, (sb / 2) 4608 +
// 2048 (p % 2) + 32 (sb % 2) + 16 (p / 2) (codes) or (sb / 2) 4608 + 16 (sb % 2) (header), is the same for every lane.
#include "common.hpp"
#include "deq_f16.hpp"

#include <type_traits>

using namespace qmm;

namespace {

constexpr int kBM = 64, kBN = 128, kWaves = 4;
constexpr int kApitch = 144;                  // bytes of a staged activation row (64 f16 + 16 bytes)
constexpr int kAbuf = kBM * kApitch;          // bytes of one staged step of a wave
constexpr int kSlot = 4 * kBN * 2;            // dwords of one scale slot: [page][column][sub-block of the page]

struct DArgs {
  int M, N, K;
  const _Float16 *x16;      // [M, K]
  const float *scales;      // [M, 2] or NULL
  const u8 *w;              // GGUF Q4_K [N, K / 256 * 144]
  void *y;                  // [M, N] f32 or bf16
  int tiles_m, tiles_total;
};

typedef __attribute__((ext_vector_type(4))) u32 u32x4;

// the eight (f16(d sc_g), f16(-dmin m_g)) pairs of a super-block header, g = 0..7, as (dsc | nmn << 16)
__device__ __forceinline__ void header_pairs(const uint4 &hd, u32 (&out)[8]) {
  const u32 sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
  const u32 sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
  const u32 mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
  const h2 dm = as_h2(hd.x ^ 0x80000000u);   // (d, -dmin)
  const h2 m1024 = as_h2(0xE400E400u);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const u32 scw = g < 4 ? sc_lo : sc_hi, mnw = g < 4 ? mn_lo : mn_hi;
    const int b = g & 3;
    // (1024 + sc, 1024 + m) as an f16 pair: bytes (sc, 0x64, m, 0x64); less 1024 is exact; one rounding multiply
    const u32 sel = (u32)(b | 0x0C00u | ((4 + b) << 16) | 0x0C000000u);
    const u32 p = __builtin_amdgcn_perm(mnw, scw, sel) | 0x64006400u;
    out[g] = as_u32((as_h2(p) + m1024) * dm);
  }
}

template <bool ACC, bool BF16OUT, bool TL>
__global__ __launch_bounds__(kWaves * 64, 1) void q4k_dense_kernel(DArgs a) {
  __shared__ __align__(16) u8 abuf[kWaves][2][kAbuf];   // also the K-part reduction area at the end
  __shared__ __align__(16) u32 stab[kWaves][2][kSlot];
  __shared__ int src_row[kBM];
  __shared__ float rinv[kBM];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: the K split and loops are scalar
  const int lc = lane & 31, h = lane >> 5;
  const int M = a.M, N = a.N, K = a.K;

  // XCD-aware order: workgroup b runs on XCD b % 8, which takes a contiguous range of tiles (an N tile's M tiles)
  const int per = (int)(gridDim.x / 8);
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= a.tiles_total) return;
  const int m0 = (t % a.tiles_m) * kBM, n0 = (t / a.tiles_m) * kBN;

  int my_src = -1;
  if (tid < kBM) {
    const int src = m0 + tid < M ? m0 + tid : -1;
    src_row[tid] = src;
    rinv[tid] = (a.scales && src >= 0) ? a.scales[2 * src + 1] : 1.f;
    my_src = src;
  }
  // skip-padding (GEMM_SKIP_PADDING): a tile whose rows all have scale 0 does no work and writes nothing
  if (a.scales) {
    const bool live = tid < kBM && my_src >= 0 && a.scales[2 * my_src] != 0.f;
    if (__syncthreads_or(live) == 0) return;
  }
  __syncthreads();   // src_row and rinv are read by every wave

  // ---- the wave's super-blocks
  const int nsb = K / 256;
  const int sb_lo = wave * nsb / kWaves, sb_hi = (wave + 1) * nsb / kWaves;
  const int nw = sb_hi - sb_lo;            // may be 0 for K < 1024 (the wave then adds zeros)
  const int npair = (nw + 1) / 2;          // super-blocks run in pairs; an odd count ends with a zero-weight one
  const int sbl = nw > 0 ? sb_hi - 1 : 0;  // the last real super-block: padding steps reload it
  const u32 RB = (u32)nsb * 144u;

  // Every load goes through a buffer resource, its per-lane part in a vector offset and the step's part in the
  // scalar offset. Activation rows past M get a vector offset past the buffer's end: the hardware returns zeros.
  // Activation staging map: load i of a step reads row 8 i + lane / 8, bytes 16 (lane % 8) .. of the step's 128.
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(a.x16), (short)0, (int)((int64_t)M * K * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<u8 *>(a.w), (short)0, (int)((int64_t)N * RB), 0x00020000);
  u32 aoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int src = src_row[8 * i + (lane >> 3)];
    aoff[i] = src >= 0 ? (u32)src * (u32)K * 2u + (u32)(lane & 7) * 16u : 0x80000000u;
  }
  // weight columns of the lane (four 32-column blocks: code bytes 16 h .. of each page) and of its two decoded
  // headers (columns lane, lane + 64)
  u32 wv[4], whv[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int c = n0 + 32 * j + lc;
    c = c < N ? c : N - 1;
    wv[j] = TL ? (u32)(c >> 4) * 16u * RB + 512u + 1024u * (u32)h + 64u * (u32)(c & 15)
               : (u32)c * RB + 16u + 16u * (u32)h;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int c = n0 + 64 * j + lane;
    c = c < N ? c : N - 1;
    whv[j] = TL ? (u32)(c >> 4) * 16u * RB + 32u * (u32)(c & 15) : (u32)c * RB;
  }
  // the lane-independent parts of a super-block's code page and header addresses
  auto code_at = [&](int sb, int p) { return TL ? (sb >> 1) * 4608 + 2048 * (p & 1) + 32 * (sb & 1) + 16 * (p >> 1)
                                                : sb * 144 + 32 * p; };
  auto head_at = [&](int sb) { return TL ? (sb >> 1) * 4608 + 16 * (sb & 1) : sb * 144; };
  auto a_load = [&](u32x4 (&r)[8], int step) __attribute__((always_inline)) {   // step of the wave's range
    int s = sb_lo * 4 + step;
    s = s < 4 * (sbl + 1) ? s : 4 * sbl + 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)aoff[i], s * 128, 0);
  };
  auto a_store = [&](const u32x4 (&r)[8], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<u32x4 *>(&abuf[wave][buf][(8 * i + (lane >> 3)) * kApitch + (lane & 7) * 16]) = r[i];
  };
  // weights of super-block sbi (a padding one reloads the last real one), in halves: half hf = column blocks 2 hf,
  // 2 hf + 1 (all four pages of each column at once, so a column's whole block is read together) and the header of
  // columns 64 hf + lane
  auto b_load = [&](u32x4 (&r)[4][4], u32x4 (&hd)[2], int sbi, int hf) __attribute__((always_inline)) {
    const int sb = sbi < sb_hi ? sbi : sbl;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int p = 0; p < 4; ++p)
        r[2 * hf + jj][p] = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)wv[2 * hf + jj], code_at(sb, p), 0);
    hd[hf] = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)whv[hf], head_at(sb), 0);
  };
  typedef __attribute__((ext_vector_type(2))) u32 u32x2;
  // the scale pairs of header half hf (columns 64 hf + lane) into scale slot `slot`, page pages of it
  auto decode_pages = [&](const u32x4 &hq, int hf, int slot, bool pad, int p0, int p1) __attribute__((always_inline)) {
    u32 pr[8];
    header_pairs(uint4{hq.x, hq.y, hq.z, hq.w}, pr);
    const int col = 64 * hf + lane;
#pragma unroll
    for (int pg = 0; pg < 4; ++pg)
      if (pg >= p0 && pg < p1)
        *reinterpret_cast<u32x2 *>(&stab[wave][slot][(pg * kBN + col) * 2]) =
            pad ? u32x2{0u, 0u} : u32x2{pr[2 * pg], pr[2 * pg + 1]};
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  u32x4 bq[2][4][4], hd[2];
  u32x4 ar[2][8];
  // prologue, in the loop's issue order: weights of the first super-block, activations of steps 0 and 1
  b_load(bq[0], hd, sb_lo, 0);
  b_load(bq[0], hd, sb_lo, 1);
  a_load(ar[0], 0);
  a_load(ar[1], 1);
  decode_pages(hd[0], 0, 0, nw == 0, 0, 4);
  decode_pages(hd[1], 1, 0, nw == 0, 0, 4);
  a_store(ar[0], 0);

  // ---- the pipelined K16 steps. A substep (super-block slot b, page pg, u = 2 gl + s2) issues its eight MFMAs on
  // fragments prepared by the substep before, and between them dequantizes the next substep's weights and reads its
  // activation fragments: the matrix pipe runs while the vector pipe works a substep ahead, across page and
  // super-block boundaries. Scheduling barriers keep the vector and matrix instructions in this order (memory and
  // scalar instructions may move).
  u32 bcur[4][4], bnxt[4][4];     // B fragments (f16x8 as four dwords) of the current / next substep
  f16x8 acur[2], anxt[2];         // A fragments
  u32x2 spc[4], spn[4];           // scale pairs (sub-blocks 2 pg, 2 pg + 1) of the current / next page
  h2 dn[4], nn[4];                // (d sc, -dmin m) of the next substep's sub-block, broadcast
  auto bcast = [&](const u32x2 (&sp)[4], int gl) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32 v = gl ? sp[j].y : sp[j].x;
      dn[j] = as_h2(__builtin_amdgcn_perm(v, v, 0x01000100u));
      nn[j] = as_h2(__builtin_amdgcn_perm(v, v, 0x03020302u));
    }
  };
  auto read_sp = [&](u32x2 (&sp)[4], int slot, int pg) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sp[j] = *reinterpret_cast<const u32x2 *>(&stab[wave][slot][(pg * kBN + 32 * j + lc) * 2]);
  };
  auto read_a = [&](f16x8 (&af)[2], int buf, int u) __attribute__((always_inline)) {
    const int ak = 2 * (32 * (u >> 1) + 16 * h + 8 * (u & 1));   // byte offset of the lane's K octet in a staged row
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const f16x8 *>(&abuf[wave][buf][(32 * i + lc) * kApitch + ak]);
  };
  // half `part` (code dword s2 * 2 + part of the page piece) of column block j's next fragment
  auto deq_part = [&](int nb, int npg, int nu, int j, int part) __attribute__((always_inline)) {
    const u32x4 &q = bq[nb][j][npg];
    const int s2 = nu & 1;
    const u32 w = s2 ? (part ? q.w : q.z) : (part ? q.y : q.x);
    const u32 n = (nu >> 1) ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu;
    const h2 c0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n, 512.0f, false);
    const h2 c1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n, 512.0f, true);
    bnxt[j][2 * part] = as_u32(__builtin_elementwise_fma(c0, dn[j], nn[j]));
    bnxt[j][2 * part + 1] = as_u32(__builtin_elementwise_fma(c1, dn[j], nn[j]));
  };
  constexpr int kPin = 0x0004 | 0x0010 | 0x0080;   // scalar, VMEM and DS instructions may cross the barriers
  // first substep's operands
  read_sp(spc, 0, 0);
  bcast(spc, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) { deq_part(0, 0, 0, j, 0); deq_part(0, 0, 0, j, 1); }
  read_a(acur, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int w = 0; w < 4; ++w) bcur[j][w] = bnxt[j][w];

  auto substep = [&](auto bc, auto pgc, auto uc, int st, int sb0) __attribute__((always_inline)) {
    constexpr int b = decltype(bc)::value, pg = decltype(pgc)::value, u = decltype(uc)::value;
    constexpr int buf = pg & 1;   // steps of a super-block pair: st % 2 == page % 2
    constexpr int nb = u < 3 ? b : (pg < 3 ? b : b ^ 1);
    constexpr int npg = u < 3 ? pg : (pg < 3 ? pg + 1 : 0);
    constexpr int nu = u < 3 ? u + 1 : 0;
    constexpr int nbuf = npg & 1;
    if constexpr (u == 0) {
      // staging: the activations of step st + 1 into the other buffer, those of step st + 2 into registers; the
      // next super-block's weights in halves at pages 0 and 2
      a_store(ar[buf ^ 1], buf ^ 1);
      a_load(ar[buf], st + 2);
      if constexpr (pg == 0 || pg == 2) b_load(bq[b ^ 1], hd, sb0 + b + 1, pg >> 1);
      if constexpr (pg < 3) read_sp(spn, b, pg + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (pg == 3 && u == 2) read_sp(spn, b ^ 1, 0);   // decoded in substeps 0 and 1 of this page
    read_a(anxt, nbuf, nu);
    if constexpr (nu == 0) bcast(spn, 0);
    else if constexpr (nu == 2) bcast(spc, 1);
    __builtin_amdgcn_sched_barrier(kPin);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[0], __builtin_bit_cast(f16x8, u32x4{bcur[j][0], bcur[j][1], bcur[j][2], bcur[j][3]}), acc[0][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(kPin);
      deq_part(nb, npg, nu, j, 0);
      __builtin_amdgcn_sched_barrier(kPin);
      acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[1], __builtin_bit_cast(f16x8, u32x4{bcur[j][0], bcur[j][1], bcur[j][2], bcur[j][3]}), acc[1][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(kPin);
      deq_part(nb, npg, nu, j, 1);
      __builtin_amdgcn_sched_barrier(kPin);
    }
    if constexpr (pg == 3 && u < 2) {
      decode_pages(hd[u], u, b ^ 1, sb0 + b + 1 >= sb_hi, 0, 4);
      __builtin_amdgcn_sched_barrier(kPin);
    }
    if constexpr (nu == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) spc[j] = spn[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w) bcur[j][w] = bnxt[j][w];
    acur[0] = anxt[0];
    acur[1] = anxt[1];
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  auto page = [&](auto bc, auto pgc, int st, int sb0) __attribute__((always_inline)) {
    substep(bc, pgc, I0{}, st, sb0);
    substep(bc, pgc, I1{}, st, sb0);
    substep(bc, pgc, I2{}, st, sb0);
    substep(bc, pgc, I3{}, st, sb0);
  };
  for (int pi = 0; pi < npair; ++pi) {
    const int sb0 = sb_lo + 2 * pi, st = 8 * pi;
    page(I0{}, I0{}, st, sb0);
    page(I0{}, I1{}, st + 1, sb0);
    page(I0{}, I2{}, st + 2, sb0);
    page(I0{}, I3{}, st + 3, sb0);
    page(I1{}, I0{}, st + 4, sb0);
    page(I1{}, I1{}, st + 5, sb0);
    page(I1{}, I2{}, st + 6, sb0);
    page(I1{}, I3{}, st + 7, sb0);
  }

  // ---- the K-parts meet through LDS as row-major f32 tiles (64 x 128, rows of kRp floats): waves 2, 3 store theirs
  // in slots 0, 1; waves 0, 1 add slot 0, 1 into their own and store the sums back; then every wave finishes 16 rows
  // as slot 0 + slot 1 = (p0 + p2) + (p1 + p3), times the row inverse, with 16-byte stores (sixteen lanes a row).
  constexpr int kRp = kBN + 4;
  __syncthreads();   // every wave is done with its staging area
  float *red = reinterpret_cast<float *>(&abuf[0][0][0]);
  static_assert(sizeof(abuf) >= 2 * kBM * kRp * 4, "reduction staging");
  auto red_at = [&](int sl, int i, int j, int r) -> float & {
    return red[(sl * kBM + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3)) * kRp + 32 * j + lc];
  };
  if (wave >= 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) red_at(wave - 2, i, j, r) = acc[i][j][r];
  }
  __syncthreads();
  if (wave < 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float &v = red_at(wave, i, j, r);
          v = acc[i][j][r] + v;
        }
  }
  __syncthreads();
  const bool vec = (N % 8) == 0;   // 16-byte aligned output chunks of 8 values
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int lr = 16 * pass + (tid >> 4), lcol = (tid & 15) * 8;
    const int row = m0 + lr, col = n0 + lcol;
    if (row >= M || col >= N) continue;
    const f32x4 *s0 = reinterpret_cast<const f32x4 *>(&red[lr * kRp + lcol]);
    const f32x4 *s1 = reinterpret_cast<const f32x4 *>(&red[(kBM + lr) * kRp + lcol]);
    const float inv = rinv[lr];
    float v[8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x4 x0 = s0[q], x1 = s1[q];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * q + e] = (x0[e] + x1[e]) * inv;
    }
    const int64_t o = (int64_t)row * N + col;
    if (vec && col + 8 <= N) {
      if constexpr (BF16OUT) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf2;
        u16 *yb = static_cast<u16 *>(a.y) + o;
        if constexpr (ACC) {
          const u32x4 old = *reinterpret_cast<const u32x4 *>(yb);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[2 * e] += bf16_to_f32(old[e] & 0xFFFFu);
            v[2 * e + 1] += bf16_to_f32(old[e] >> 16);
          }
        }
        u32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = __builtin_bit_cast(u32, bf2{(__bf16)v[2 * e], (__bf16)v[2 * e + 1]});
        *reinterpret_cast<u32x4 *>(yb) = out;
      } else {
        f32x4 *yf = reinterpret_cast<f32x4 *>(static_cast<float *>(a.y) + o);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          f32x4 out = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          if constexpr (ACC) out += yf[q];
          yf[q] = out;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (col + e >= N) break;
        if constexpr (BF16OUT) {
          u16 *yb = static_cast<u16 *>(a.y) + o + e;
          float w = v[e];
          if constexpr (ACC) w += bf16_to_f32(*yb);
          *yb = __builtin_bit_cast(u16, (__bf16)w);
        } else {
          float *yf = static_cast<float *>(a.y) + o + e;
          *yf = ACC ? *yf + v[e] : v[e];
        }
      }
    }
  }
}

template <bool ACC, bool BF16OUT>
int launch_dense(const DArgs &a, bool tiled, hipStream_t s) {
  const dim3 grid((unsigned)(8 * ((a.tiles_total + 7) / 8)));
  if (tiled) q4k_dense_kernel<ACC, BF16OUT, true><<<grid, kWaves * 64, 0, s>>>(a);
  else q4k_dense_kernel<ACC, BF16OUT, false><<<grid, kWaves * 64, 0, s>>>(a);
  return launch_status();
}

}  // namespace

// The Q4_K store / acc path of qmm_gemm (gemm_q4k.hip validates the arguments): GGUF Q4_K weights or (tiled) the
// QMM_Q4_KT layout, f16 rows.
int qmm_gemm_q4k_dense(int acc, int tiled, int64_t rows, int64_t k, int64_t n, const void *x, const float *scales,
                       const void *w, void *y, int y_bf16, hipStream_t s) {
  DArgs a{};
  a.M = (int)rows; a.N = (int)n; a.K = (int)k;
  a.x16 = static_cast<const _Float16 *>(x); a.scales = scales;
  a.w = static_cast<const u8 *>(w); a.y = y;
  a.tiles_m = (int)((rows + kBM - 1) / kBM);
  a.tiles_total = a.tiles_m * (int)((n + kBN - 1) / kBN);
  if (acc && y_bf16) return launch_dense<true, true>(a, tiled, s);
  if (acc) return launch_dense<true, false>(a, tiled, s);
  if (y_bf16) return launch_dense<false, true>(a, tiled, s);
  return launch_dense<false, false>(a, tiled, s);
}
