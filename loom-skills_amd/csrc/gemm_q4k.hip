// Q4_K prefill GEMM on the f16 MFMA: the g_gemm_q4_k_{store|acc}[_m128|_m256] family (S/gen_gemm.py:535-703).
//
//   Y[r, c] = (acc ? Y[r, c] : 0) + inv[r] * sum_k X16[r, k] W[c, k]         fp32 accumulation
//
// X16 is the row-scaled f16 operand the reference's g_row_scale_f16 produces (S/gen_llm.py:1843-1915) with
// inv[r] = scales[r, 1]; W is Q4_K, dequantized to f16 in registers the way the reference stages it
// (S/gen_gemm.py:499-530): w = fma_f16(f16(q), f16(d sc), f16(-dmin m)).
//
// Tiling (gfx950, wave64). A workgroup owns a 64 x 128 output tile and has four waves: wave (nh, kh) computes the
// 64 x 64 quadrant nh of the tile over K-half kh with 2 x 2 v_mfma_f32_32x32x16_f16 tiles, so 256 workgroups
// fill the 256 CUs with one wave per SIMD at the Qwen3-8B o_proj shape (512 x 4096 x 4096). The two K-halves are
// summed through LDS at the end, in a fixed order. A step is one 64-value page of a super-block: the X16 rows of
// both K-halves (2 x 64 x 64 f16) are staged in LDS, double-buffered, one barrier per step; each wave streams its
// own 64 weight columns straight into registers (one 16-byte code chunk per column per step, the 16-byte header
// once per super-block) and dequantizes them there, so B never touches LDS.
//
// MFMA operand order. Lane l of a 32x32x16 step holds 8 K values of row/column l % 32, octet l / 32. Lane half h
// takes code bytes 16h .. 16h+15 of a page, i.e. values 16h .. 16h+15 of both of the page's sub-blocks; K16 step
// s2 of a sub-block uses the lane's values 8 s2 .. 8 s2 + 7. The A fragment is read from LDS at the same K.
//
// Tile order is XCD-aware: consecutive tile ids (the M tiles of one N tile) land on one XCD, so the weight columns
// a tile streams are read from HBM once per XCD and served from its L2 to the other M tiles.
#include "common.hpp"

using namespace qmm;

namespace {

constexpr int BM = 64, BN = 128, KSTEP = 64;
#ifndef QMM_GEMM_DEPTH
#define QMM_GEMM_DEPTH 4
#endif
constexpr int kDepth = QMM_GEMM_DEPTH;   // steps of loads in flight per wave (even)
static_assert(kDepth % 2 == 0, "the LDS double buffer follows the step parity");
constexpr int APITCH = KSTEP + 8;   // f16 per LDS row: 144 bytes, rows 16-byte aligned, reads 2-way at most
typedef __attribute__((ext_vector_type(2))) _Float16 h2;

__device__ __forceinline__ h2 as_h2(u32 v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ u32 as_u32(h2 v) { return __builtin_bit_cast(u32, v); }

// 8 f16 weights of one column in K order from two code dwords (values 0..3 and 4..7 of the run) of one nibble
// plane: bytes become (1024 + q) f16 pairs with one v_perm each, the 1024 is removed exactly, then one rounding
// fma with the sub-block's f16 scale and negated minimum.
template <bool HI>
__device__ __forceinline__ f16x8 deq8(u32 q0, u32 q1, h2 dsc, h2 nmn) {
  const u32 n0 = HI ? (q0 >> 4) & 0x0F0F0F0Fu : q0 & 0x0F0F0F0Fu;
  const u32 n1 = HI ? (q1 >> 4) & 0x0F0F0F0Fu : q1 & 0x0F0F0F0Fu;
  const u32 k64 = 0x64646464u;
  const h2 m1024 = as_h2(0xE400E400u);
  const u32 t[4] = {__builtin_amdgcn_perm(k64, n0, 0x04010400u), __builtin_amdgcn_perm(k64, n0, 0x04030402u),
                    __builtin_amdgcn_perm(k64, n1, 0x04010400u), __builtin_amdgcn_perm(k64, n1, 0x04030402u)};
  u32 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = as_u32(__builtin_elementwise_fma(as_h2(t[i]) + m1024, dsc, nmn));
  typedef __attribute__((ext_vector_type(4))) u32 u32x4;
  return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

// f16 (d sc, -dmin m) of sub-block g from a super-block header, broadcast to both halves
__device__ __forceinline__ void sub_scale(const uint4 &hd, int g, h2 &dsc, h2 &nmn) {
  u32 sc, mn;
  q4k_scale_min(hd.y, hd.z, hd.w, g, sc, mn);
  const _Float16 a = (_Float16)(f16_to_f32(hd.x) * (float)sc);
  const _Float16 b = (_Float16)(-(f16_to_f32(hd.x >> 16) * (float)mn));
  dsc = h2{a, a};
  nmn = h2{b, b};
}

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

template <bool ACC, bool BF16OUT, int DEPTH>
__global__ __launch_bounds__(256, 1) void gemm_q4k_kernel(int M, int N, int K, const _Float16 *__restrict__ x16,
                                                          const float *__restrict__ scales,
                                                          const u8 *__restrict__ w, void *__restrict__ yv,
                                                          int tiles_m, int tiles_total) {
  __shared__ __align__(16) _Float16 As[2][2][BM][APITCH];   // [buffer][K-half][row][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nh = wave & 1, kh = wave >> 1;
  const int per = (int)(gridDim.x / 8);
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= tiles_total) return;
  const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
  const int64_t RB = (int64_t)K / 256 * 144;
  const int S = K / KSTEP, S0 = (S + 1) / 2, S1 = S - S0;
  const int my_steps = kh ? S1 : S0;

  // ---- A staging map: chunk c = i * 256 + tid of 16 bytes; K-half, row, 16-byte column. Loads are unconditional
  // with clamped addresses, so no branch or select splits the load stream: rows past M load row M - 1 (their
  // outputs are never stored) and steps past S0 load step S0 - 1 (their weights are zeroed in the compute).
  auto a_load = [&](int i, int s) -> uint4 {
    const int c = i * 256 + tid, ckh = c >> 9, row = (c >> 3) & 63, col = c & 7;
    const int r = m0 + row < M ? m0 + row : M - 1, gs = ckh * S0 + (s < S0 ? s : S0 - 1);
    return *reinterpret_cast<const uint4 *>(x16 + (int64_t)r * K + (int64_t)gs * KSTEP + col * 8);
  };
  auto a_dst = [&](int i, int buf) -> uint4 * {
    const int c = i * 256 + tid, ckh = c >> 9, row = (c >> 3) & 63, col = c & 7;
    return reinterpret_cast<uint4 *>(&As[buf][ckh][row][col * 8]);
  };

  // ---- B: this lane's two weight columns and code half
  const int h = lane >> 5, lc = lane & 31;
  const u8 *wcol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int c = n0 + nh * 64 + 32 * j + lc;
    c = c < N ? c : N - 1;
    wcol[j] = w + (int64_t)c * RB;
  }
  auto b_code = [&](int j, int s) -> uint4 {
    const int gs = kh * S0 + (s < S0 ? s : S0 - 1);
    return ld16(wcol[j] + (int64_t)(gs >> 2) * 144 + 16 + 32 * (gs & 3) + 16 * h);
  };
  auto b_head = [&](int j, int s) -> uint4 {
    return ld16(wcol[j] + (int64_t)((kh * S0 + (s < S0 ? s : S0 - 1)) >> 2) * 144);
  };

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
  auto load_a = [&](int slot, int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) aring[slot][i] = a_load(i, st);
  };
  auto load_b = [&](int slot, int st) {
#pragma unroll
    for (int j = 0; j < 2; ++j) { cring[slot][j] = b_code(j, st); hring[slot][j] = b_head(j, st); }
  };
  // prologue: A of step 0 into LDS buffer 0, A of steps 1..DEPTH and B of steps 0..DEPTH-1 in flight
  load_a(0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) *a_dst(i, 0) = aring[0][i];
#pragma unroll
  for (int u = 1; u <= DEPTH; ++u) load_a(u % DEPTH, u);
#pragma unroll
  for (int u = 0; u < DEPTH; ++u) load_b(u, u);
  __syncthreads();

  // The step count is rounded up to a multiple of DEPTH; steps past S0 get zero weights (no contribution), so
  // the loop body has no data-dependent branch and every wave runs the same barriers. Both K-halves have S0 steps
  // (K is a multiple of 256, so K / 64 is even).
  const int SP = (S0 + DEPTH - 1) / DEPTH * DEPTH;
  for (int s0 = 0; s0 < SP; s0 += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int s = s0 + u;
      const int buf = u & 1;   // DEPTH is even, so s & 1 == u & 1
      const int page = (kh * S0 + (s < S0 ? s : S0 - 1)) & 3;
#pragma unroll
      for (int gl = 0; gl < 2; ++gl) {
        h2 dsc[2], nmn[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          sub_scale(hring[u][j], 2 * page + gl, dsc[j], nmn[j]);
          if (s >= S0) dsc[j] = nmn[j] = h2{0, 0};   // a padding step: zero weights
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          f16x8 bf[2], af[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const u32 q0 = s2 ? cring[u][j].z : cring[u][j].x, q1 = s2 ? cring[u][j].w : cring[u][j].y;
            bf[j] = gl ? deq8<true>(q0, q1, dsc[j], nmn[j]) : deq8<false>(q0, q1, dsc[j], nmn[j]);
          }
#pragma unroll
          for (int i = 0; i < 2; ++i)
            af[i] = *reinterpret_cast<const f16x8 *>(&As[buf][kh][32 * i + lc][32 * gl + 16 * h + 8 * s2]);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
      }
      load_b(u, s + DEPTH);
      const int nx = (u + 1) % DEPTH;
#pragma unroll
      for (int i = 0; i < 4; ++i) *a_dst(i, buf ^ 1) = aring[nx][i];
      load_a(nx, s + 1 + DEPTH);
      __syncthreads();
    }
  }

  // ---- sum the K-halves through LDS (K-half 1 hands its partial to K-half 0), then the epilogue
  float *red = reinterpret_cast<float *>(&As[0][0][0][0]);   // [nh][64 values][64 lanes]
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(nh * 64 + (i * 2 + j) * 16 + r) * 64 + lane] = acc[i][j][r];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        const int col = n0 + nh * 64 + 32 * j + lc;
        if (row < M && col < N) {
          float v = acc[i][j][r] + red[(nh * 64 + (i * 2 + j) * 16 + r) * 64 + lane];
          if (scales) v *= scales[2 * row + 1];
          const int64_t o = (int64_t)row * N + col;
          if constexpr (BF16OUT) {
            u16 *y = static_cast<u16 *>(yv);
            if constexpr (ACC) v += bf16_to_f32(y[o]);
            y[o] = (u16)f32_to_bf16_rne(v);
          } else {
            float *y = static_cast<float *>(yv);
            if constexpr (ACC) v += y[o];
            y[o] = v;
          }
        }
      }
}

}  // namespace

extern "C" int qmm_gemm(int fmt, int mode, int64_t rows, int64_t k, int64_t n, const void *x, int x_dtype,
                        const float *scales, const void *w, const void *w2, void *y, int y_dtype,
                        qmm_stream_t stream) {
  (void)w2;
  if (fmt != QMM_Q4_K) return QMM_ERR_FORMAT;
  if (mode != QMM_GEMM_STORE && mode != QMM_GEMM_ACC) return QMM_ERR_RANGE;
  if (!x || !w || !y) return QMM_ERR_NULL;
  if (x_dtype != QMM_F16) return QMM_ERR_DTYPE;   // bf16 / f32 rows go through qmm_row_scale_f16 first
  if (y_dtype != QMM_F32 && y_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (rows <= 0 || n <= 0 || k <= 0 || k % 256) return QMM_ERR_SHAPE;
  if (rows > (1 << 24) || n > (1 << 24) || k > (1 << 20)) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tiles_m = (int)((rows + BM - 1) / BM), tiles_n = (int)((n + BN - 1) / BN);
  const int total = tiles_m * tiles_n, per = (total + 7) / 8;
  const dim3 grid((unsigned)(8 * per));
  const _Float16 *xp = static_cast<const _Float16 *>(x);
  const u8 *wp = static_cast<const u8 *>(w);
  const bool acc = mode == QMM_GEMM_ACC, bf = y_dtype == QMM_BF16;
  if (acc && bf) gemm_q4k_kernel<true, true, kDepth><<<grid, 256, 0, s>>>((int)rows, (int)n, (int)k, xp, scales, wp, y, tiles_m, total);
  else if (acc) gemm_q4k_kernel<true, false, kDepth><<<grid, 256, 0, s>>>((int)rows, (int)n, (int)k, xp, scales, wp, y, tiles_m, total);
  else if (bf) gemm_q4k_kernel<false, true, kDepth><<<grid, 256, 0, s>>>((int)rows, (int)n, (int)k, xp, scales, wp, y, tiles_m, total);
  else gemm_q4k_kernel<false, false, kDepth><<<grid, 256, 0, s>>>((int)rows, (int)n, (int)k, xp, scales, wp, y, tiles_m, total);
  return launch_status();
}
