// Q4_K decode GEMV with bf16 activations, K = 4096 or 8192: the fast path of qmm_mv for g_mv_q4_k_k{K}[_t{TG}]
// (S/gen_llm.py:1159-1378).
//
// Launch shape. One workgroup of 8 waves per block of 16 (K = 4096) or 8 (K = 8192) consecutive weight rows (the
// defaults below; both are compile-time knobs), each wave streaming its rows with all loads in flight. A lane owns
// half a super-block of one row: its 16-byte header and the 64 code bytes of pages 2h, 2h+1 (sub-blocks 4h..4h+3),
// five 128-bit loads. For K = 4096 a row is 32 lanes (a wave covers two rows per slot), for K = 8192 it is 64.
// A wave owns kSlots slots; all its loads are issued before any math, the activations first.
//
// Activations. The workgroup stages each token once in LDS as f16 x' = x 2^-e, e a per-token power of two that
// puts the row maximum in [2^14, 2^15) (x' equals x for every bf16 value whose f16 image is normal), stored in
// groups of four as (x0, x2), (x1, x3), the order the code pairs come in, plus every 32-value sub-block's sum of x'.
//
// Codes. For a code dword Q, (Q & 0x000F000F) is the bit pattern of the f16 pair (q0 2^-24, q2 2^-24) -- exact
// subnormals -- and (Q & 0x00F000F0) that of the high nibbles times 16; the same masks on Q >> 8 give bytes 1 and 3.
// Five ALU ops unpack eight codes and v_dot2_f32_f16 multiplies them with the staged activations (exact products).
// Per sub-block g:  sum_l (d sc q_l - dmin m) x_l = 2^e [d sc 2^24 P_g - dmin m S_g]   (high nibbles: 2^20).
//
// Rows are summed with a transposed butterfly, the same tree for every token count, and a token's arithmetic does
// not depend on the other tokens of its group: results are identical whatever the number of tokens in the call.
#include "bfly.hpp"

using namespace qmm;

namespace {

typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

__device__ __forceinline__ float fdot2(u32 a, u32 b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

#ifndef QMM_Q4K_WAVES
#define QMM_Q4K_WAVES 8
#endif
#ifndef QMM_Q4K_SLOTS
#define QMM_Q4K_SLOTS 1
#endif
constexpr int kWaves = QMM_Q4K_WAVES;
constexpr int kThreads = kWaves * 64;
constexpr int kSlots = QMM_Q4K_SLOTS;

template <int TG, int KB>
__global__ __launch_bounds__(kThreads) void mv_q4k_kernel(int64_t n, int64_t tokens, int accumulate,
                                                          const u16 *__restrict__ x, const u8 *__restrict__ w,
                                                          float *__restrict__ y) {
  constexpr int K = KB * 4096;
  constexpr int L = 32 * KB;            // lanes per row
  constexpr int RPP = 64 / L;           // rows per wave and slot
  constexpr int WG_ROWS = kWaves * kSlots * RPP;
  constexpr int64_t RB = (int64_t)K / 256 * 144;
  constexpr int NCH = K / 8;            // 8-value chunks of a token row
  constexpr int CPT = (NCH + kThreads - 1) / kThreads;
  constexpr int ITEMS = K / 128;        // (block, half) items of a row = 8-value chunks per item / 16

  __shared__ __align__(16) u32 xs[TG][K / 2];        // f16 pairs, permuted in groups of four, lane-major chunks
  __shared__ __align__(16) float ssum[TG][K / 32];   // sub-block sums of x'
  __shared__ float red[kWaves];
  __shared__ int eexp[TG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.y * TG;
  const int64_t wrow0 = (int64_t)blockIdx.x * WG_ROWS + wave * kSlots * RPP;
  const int rp = lane / L;              // row of the slot this lane works on
  const int item = lane % L;            // (block, half) of that row
  const int b = item >> 1, h = item & 1;

  // ---- loads: activations first (an L2 read), then the weights (vector loads retire in issue order)
  uint4 xv[TG][CPT];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const int64_t tok = t0 + t < tokens ? t0 + t : tokens - 1;
    const uint4 *xr = reinterpret_cast<const uint4 *>(x + tok * K);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      xv[t][i] = c < NCH ? xr[c] : make_uint4(0, 0, 0, 0);
    }
  }
  uint4 wd[kSlots][5];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    int64_t row = wrow0 + s * RPP + rp;
    row = row < n ? row : n - 1;        // rows past n read row n-1 and are never stored
    const uint4 *bp = reinterpret_cast<const uint4 *>(w + row * RB + (int64_t)b * 144);
    wd[s][0] = bp[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) wd[s][1 + i] = bp[1 + 4 * h + i];
  }

  // ---- stage the activations
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const u32 d[4] = {xv[t][i].x, xv[t][i].y, xv[t][i].z, xv[t][i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) m = fmaxf(m, fmaxf(fabsf(bf16_to_f32(d[q] & 0xFFFFu)), fabsf(bf16_to_f32(d[q] >> 16))));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kWaves; ++i) m = fmaxf(m, red[i]);
    int e = 0;
    if (m > 0.f) {
      int ex;
      frexpf(m, &ex);
      e = min(max(ex - 1 - 14, -100), 100);
    }
    const float sc = ldexpf(1.0f, -e);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      if (c < NCH) {
        const u32 d[4] = {xv[t][i].x, xv[t][i].y, xv[t][i].z, xv[t][i].w};
        _Float16 hv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          hv[2 * q] = (_Float16)(bf16_to_f32(d[q] & 0xFFFFu) * sc);
          hv[2 * q + 1] = (_Float16)(bf16_to_f32(d[q] >> 16) * sc);
        }
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) s += (float)hv[q];
        u32 o[4];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          o[2 * g] = (u32)__builtin_bit_cast(u16, hv[4 * g]) | ((u32)__builtin_bit_cast(u16, hv[4 * g + 2]) << 16);
          o[2 * g + 1] = (u32)__builtin_bit_cast(u16, hv[4 * g + 1]) | ((u32)__builtin_bit_cast(u16, hv[4 * g + 3]) << 16);
        }
        // lane-major: the 16-byte chunk i (0..15) of item it = c / 16 sits at chunk index i * ITEMS + it, so the
        // 16 reads of a wave each cover consecutive chunks (no bank conflicts)
        reinterpret_cast<uint4 *>(xs[t])[(c % 16) * ITEMS + c / 16] = make_uint4(o[0], o[1], o[2], o[3]);
        // the 4 chunks of a 32-value sub-block are held by 4 consecutive threads of one wave
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((c & 3) == 0) ssum[t][c >> 2] = s;
      }
    }
    if (tid == 0) eexp[t] = t0 + t < tokens ? e : 0;
    __syncthreads();
  }

  // ---- the lane's activations: values [256 b + 128 h, +128) = sub-blocks 4h .. 4h+3
  u32 xa[TG][64];
  float sg[TG][4];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const uint4 *p = reinterpret_cast<const uint4 *>(xs[t]) + item;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint4 v = p[i * ITEMS];
      xa[t][4 * i] = v.x; xa[t][4 * i + 1] = v.y; xa[t][4 * i + 2] = v.z; xa[t][4 * i + 3] = v.w;
    }
    const float4 ss = *reinterpret_cast<const float4 *>(&ssum[t][8 * b + 4 * h]);
    sg[t][0] = ss.x; sg[t][1] = ss.y; sg[t][2] = ss.z; sg[t][3] = ss.w;
  }

  const u32 upper = 0u - (u32)h;       // bit select of the half's scale layout, no divergent branch
  float acc[kSlots * TG];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const uint4 hd = wd[s][0];
    // the four 6-bit scales and minima of the lane's half, one per byte (ggml get_scale_min_k4)
    const u32 s0 = hd.y, s1 = hd.z, s2 = hd.w;
    const u32 sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u), sc_lo = s0 & 0x3F3F3F3Fu;
    const u32 m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u), m_lo = s1 & 0x3F3F3F3Fu;
    const u32 scP = (sc_hi & upper) | (sc_lo & ~upper);
    const u32 mP = (m_hi & upper) | (m_lo & ~upper);
    const float d = f16_to_f32(hd.x), dmin = f16_to_f32(hd.x >> 16);
    const float c0 = (float)(scP & 0xFFu), c1 = (float)((scP >> 8) & 0xFFu);
    const float c2 = (float)((scP >> 16) & 0xFFu), c3 = (float)(scP >> 24);
    const float m0 = (float)(mP & 0xFFu), m1 = (float)((mP >> 8) & 0xFFu);
    const float m2 = (float)((mP >> 16) & 0xFFu), m3 = (float)(mP >> 24);
    const float d24 = d * 16777216.0f;   // codes are f16 subnormals (2^-24); high nibbles carry a further 16
    const u32 q[16] = {wd[s][1].x, wd[s][1].y, wd[s][1].z, wd[s][1].w, wd[s][2].x, wd[s][2].y, wd[s][2].z, wd[s][2].w,
                       wd[s][3].x, wd[s][3].y, wd[s][3].z, wd[s][3].w, wd[s][4].x, wd[s][4].y, wd[s][4].z, wd[s][4].w};
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      float p[4];
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) {       // page 2h + pg: low nibbles -> sub-block 4h + 2pg, high -> +1
        float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
        const u32 *xl = &xa[t][32 * pg], *xh = &xa[t][32 * pg + 16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const u32 Q = q[8 * pg + i], Q8 = Q >> 8;
          lo0 = fdot2(Q & 0x000F000Fu, xl[2 * i], lo0);
          lo1 = fdot2(Q8 & 0x000F000Fu, xl[2 * i + 1], lo1);
          hi0 = fdot2(Q & 0x00F000F0u, xh[2 * i], hi0);
          hi1 = fdot2(Q8 & 0x00F000F0u, xh[2 * i + 1], hi1);
        }
        p[2 * pg] = lo0 + lo1;
        p[2 * pg + 1] = hi0 + hi1;
      }
      const float lo = __builtin_fmaf(c2, p[2], c0 * p[0]);
      const float hi = __builtin_fmaf(c3, p[3], c1 * p[1]);
      const float pos = d24 * __builtin_fmaf(hi, 0.0625f, lo);
      const float neg = dmin * __builtin_fmaf(m3, sg[t][3], __builtin_fmaf(m2, sg[t][2], __builtin_fmaf(m1, sg[t][1], m0 * sg[t][0])));
      acc[s * TG + t] = pos - neg;
    }
  }

  constexpr int NV = kSlots * TG;
  int idx;
  const float tot = group_reduce<NV, L>(acc, lane, idx);
  constexpr int kHalve = log2i(NV);
  constexpr int low_mask = (L >> kHalve) - 1;
  if ((lane & low_mask) == 0) {
    const int s = idx / TG, t = idx % TG;
    const int64_t row = wrow0 + s * RPP + rp, tok = t0 + t;
    if (row < n && tok < tokens) {
      const float v = ldexpf(tot, eexp[t]);
      float *py = y + tok * n + row;
      *py = accumulate ? *py + v : v;
    }
  }
}

template <int TG, int KB>
int launch(int64_t n, int64_t tokens, int accumulate, const void *x, const void *w, float *y, hipStream_t s) {
  constexpr int WG_ROWS = kWaves * kSlots * (2 / KB);
  const dim3 grid((unsigned)((n + WG_ROWS - 1) / WG_ROWS), (unsigned)((tokens + TG - 1) / TG));
  mv_q4k_kernel<TG, KB><<<grid, kThreads, 0, s>>>(n, tokens, accumulate, static_cast<const u16 *>(x),
                                                  static_cast<const u8 *>(w), y);
  return launch_status();
}

}  // namespace

// Fast path of qmm_mv: Q4_K, bf16 activations, K = 4096 or 8192 (returns 1 when the shape is not covered).
int qmm_mv_q4k_fast(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w, float *y,
                    hipStream_t s) {
  if (tokens > 65535ll * 2) return 1;
  if (k == 4096) return tokens >= 2 ? launch<2, 1>(n, tokens, accumulate, x, w, y, s) : launch<1, 1>(n, tokens, accumulate, x, w, y, s);
  if (k == 8192) return tokens >= 2 ? launch<2, 2>(n, tokens, accumulate, x, w, y, s) : launch<1, 2>(n, tokens, accumulate, x, w, y, s);
  return 1;
}
