// The Q4_K decode matvec on Q8_1 activations over the tiled weight layout (qmm_tile_q4k), and that layout's
// repack and dequant kernels.
//
// Tiled layout: units of 16 rows x 512 values (two super-blocks a row), ordered (row block, slice), 4608 bytes
// each. A unit holds the 32 16-byte headers ([f16 d][f16 dmin][12 scale bytes]) of super-block sb of row r at
// 16 (2 r + sb), then four 1 KB code planes: plane q holds at 16 l, l = 4 r + 2 sb + h, code bytes
// 16 (4 h + q) .. 16 (4 h + q) + 15 of that super-block. Lane l of a wave is exactly the lane that multiplies
// half h of super-block sb of row r, so the wave's five loads per unit (a header, four code planes) are each one
// contiguous run of bytes, where the GGUF layout spreads every load instruction over 16 rows 2304 bytes apart
// (measured on MI355X for a 28.3 MB matrix: 6.14 us to read the GGUF pattern, 5.67 us the tiled one).
//
// Matvec (the g_mv_q4_k_k{K}_q8 family, S/gen_llm.py:1288-1301, iq_dot :1024-1071): a workgroup owns one row block
// (16 rows); its NW waves split K, wave w taking slices U w .. U w + U - 1 (K = 512 U NW). Each wave quantizes its
// own activation slices to Q8_1 in LDS (or copies planar Q8_1 codes), exactly as qmm_quant_q8 does, and each lane
// then adds, per 32-value group of its half super-block, (di d sc - xs dmin m) da with di the exact int32 dot of
// codes. The row's four lanes meet in a butterfly, the waves in LDS in a fixed order; for K = 4096 the arithmetic
// and its order are those of the GGUF-layout kernel, so both give the same bits.
//
// Q4_0 in the same units (QMM_Q4_0T, qmm_tile_q40): 512 values of a Q4_0 row are 16 blocks of 18 bytes, the bytes of
// two Q4_K super-blocks, so a unit keeps the Q4_K unit's shape. Header slot 16 (2 r + sb) holds the eight f16 d of
// blocks 8 sb .. 8 sb + 7 of the unit's row r; the 128 code bytes of those eight blocks are laid out as a Q4_K
// super-block's (page p = bytes 32 p .. 32 p + 31: low nibbles the 32 codes of block 2 p in value order, high nibbles
// those of block 2 p + 1) and cut into the same four planes. A lane then takes blocks 4 h .. 4 h + 3 of its span and
// adds, per block, (d da) (di - 8 xs): di the exact dot of the codes with the activation codes, xs their sum, i.e. the
// integer dot of codes q - 8 the reference's Q4_0 int8 matvec forms (@g_q4_0_icodes, S/gen_llm.py:536-552).
//
// Two-matrix variants stream a second matrix W2 of the same shape in the same waves, with the same per-lane arithmetic
// and reductions for each: swiglu y = silu(x W^T) (x W2^T) (g_mv_q4_k_k{K}_swiglu[_t{TG}]_q8, S/gen_llm.py:1159-1197)
// and pair y = x W^T, y2 = x W2^T (g_mv_q4_k_k{K}_pair[_t{TG}]_q8, S/gen_llm.py:1166-1176), each row of a pair
// equal bit for bit to the one-matrix kernel's.
#include <type_traits>

#include "bfly.hpp"

using namespace qmm;

namespace {

typedef __attribute__((ext_vector_type(4))) u32 v4u;
typedef __attribute__((ext_vector_type(2))) u32 v2u;

constexpr int kUnit = 4608, kMaxWaves = 8;
enum Mode { kPlain = 0, kSwiglu = 1, kPair = 2 };
enum TFmt { kTQ4K = 0, kTQ40 = 1 };   // the tiled layouts: Q4_K (qmm_tile_q4k), Q4_0 (qmm_tile_q40)

__device__ __forceinline__ int sdot4(u32 a, u32 b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 8 activations of the lane as f32: from 16 bytes of bf16 or 32 bytes of f32 at element offset e
__device__ __forceinline__ void load8(const void *x, bool bf, int64_t e, float (&v)[8]) {
  if (bf) {
    const v4u q = *reinterpret_cast<const v4u *>(static_cast<const u16 *>(x) + e);
    const u32 d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_to_f32(d[j] & 0xFFFFu); v[2 * j + 1] = bf16_to_f32(d[j] >> 16); }
  } else {
    const v4u a = *reinterpret_cast<const v4u *>(static_cast<const float *>(x) + e);
    const v4u b = *reinterpret_cast<const v4u *>(static_cast<const float *>(x) + e + 4);
    const u32 d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = u32_as_f32(d[j]);
  }
}

// Q8_1 of one 32-value group held by four consecutive lanes (8 values each): the lane's codes as two dwords, the
// group's f16-rounded d and code sum (llama.cpp quantize_q8_1; the arithmetic of qmm_quant_q8)
__device__ __forceinline__ void q8_group(const float (&v)[8], u32 &c0, u32 &c1, float &d16, float &sum) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
  const float d = amax / 127.f;
  int s = 0;
  u32 c[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = d > 0.f ? v[i] / d : 0.f;
    const int q = (int)copysignf(floorf(fabsf(t) + 0.5f), t);
    s += q;
    c[i >> 2] |= ((u32)q & 0xFFu) << (8 * (i & 3));
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  c0 = c[0];
  c1 = c[1];
  d16 = (float)(_Float16)d;
  sum = (float)s;
}

template <int TG, int U, bool STAGEQ, int MODE, int WF>
__global__ __launch_bounds__(kMaxWaves * 64) void mv_q4kt_q8_kernel(int64_t n, int64_t tokens, int64_t K,
                                                                   int accumulate, const void *__restrict__ x, int bf,
                                                                   const u8 *__restrict__ w, const u8 *__restrict__ w2,
                                                                   float *__restrict__ y, float *__restrict__ y2) {
  constexpr int SLICE = 512 * U, NG = SLICE / 32;   // values / Q8 groups of a wave
  constexpr int NM = MODE == kPlain ? 1 : 2;        // weight matrices streamed
  // the codes of a token's slice, four dwords of padding after every 32 (pidx): the four lane classes (super-block
  // half sb, h) read fragments 32 dwords apart, which would sit in the same LDS banks
  __shared__ __align__(16) u32 xc[kMaxWaves][TG][SLICE / 4 + SLICE / 32];
  auto pidx = [](int d) { return d + 4 * (d >> 5); };
  __shared__ __align__(16) float xm[kMaxWaves][TG][NG][2];
  __shared__ float red[kMaxWaves][NM][16][TG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NW = (int)(blockDim.x >> 6);
  const int64_t t0 = (int64_t)blockIdx.y * TG;
  const int64_t rb = blockIdx.x;                    // row block: rows 16 rb .. 16 rb + 15
  const int r = lane >> 2, sb = (lane >> 1) & 1, h = lane & 1;
  const int64_t k0 = (int64_t)wave * SLICE;         // the wave's first value

  // ---- the wave's activations first, then its weights: U units (a header and four code planes each) through
  //      NSLOT register slots, units 0 .. NSLOT - 1 now and unit u + NSLOT once unit u is consumed
  float xv[TG][U][8];
  v2u qv[TG][U];
  float2 mv[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const int64_t tok = t0 + t < tokens ? t0 + t : tokens - 1;
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int c = lane + 64 * j;                 // 8-value chunk of the wave's values
      if constexpr (STAGEQ) load8(x, bf, tok * K + k0 + 8 * c, xv[t][j]);
      else qv[t][j] = *reinterpret_cast<const v2u *>(static_cast<const u8 *>(x) + tok * K + k0 + 8 * c);
    }
    if constexpr (!STAGEQ) {
      const float2 *meta = reinterpret_cast<const float2 *>(static_cast<const u8 *>(x) + tokens * K);
      mv[t] = meta[tok * (K / 32) + k0 / 32 + (lane < NG ? lane : 0)];
    }
  }
  // register slots of the weight ring: two (units u and u + 1 in flight) for one matrix; one for two matrices, whose
  // unit already keeps ten 16-byte loads in flight (two slots would spill from U = 2 on)
  constexpr int NSLOT = (U == 1 || NM == 2) ? 1 : 2;
  v4u wd[NM][NSLOT][5];
  auto load_unit = [&](int slot, int u) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const v4u *up = reinterpret_cast<const v4u *>((m ? w2 : w) + (rb * (K / 512) + (int64_t)wave * U + u) * kUnit);
      wd[m][slot][0] = up[lane >> 1];
#pragma unroll
      for (int q = 0; q < 4; ++q) wd[m][slot][1 + q] = up[32 + 64 * q + lane];
    }
  };
#pragma unroll
  for (int u = 0; u < NSLOT; ++u) load_unit(u, u);

  // ---- the wave's slices: codes and group pairs into its own LDS area
#pragma unroll
  for (int t = 0; t < TG; ++t) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int c = lane + 64 * j;
      if constexpr (STAGEQ) {
        u32 c0, c1;
        float d16, sum;
        q8_group(xv[t][j], c0, c1, d16, sum);
        xc[wave][t][pidx(2 * c)] = c0;
        xc[wave][t][pidx(2 * c) + 1] = c1;
        if ((c & 3) == 0) { xm[wave][t][c >> 2][0] = d16; xm[wave][t][c >> 2][1] = sum; }
      } else {
        xc[wave][t][pidx(2 * c)] = qv[t][j].x;
        xc[wave][t][pidx(2 * c) + 1] = qv[t][j].y;
      }
    }
    if constexpr (!STAGEQ) {
      if (lane < NG) { xm[wave][t][lane][0] = mv[t].x; xm[wave][t][lane][1] = mv[t].y; }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // a token's activation fragment of the lane's 4 groups of unit u (16 u + 8 sb + 4 h + 0..3): codes (8 dwords a
  // group) and (d, code sum) pairs, from LDS
  auto frag = [&](int t, int u, u32 (&xa)[4][8], float (&md)[4], float (&ms)[4]) __attribute__((always_inline)) {
    const int g0 = 16 * u + 8 * sb + 4 * h;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v4u p0 = *reinterpret_cast<const v4u *>(&xc[wave][t][pidx(8 * (g0 + g))]);
      const v4u p1 = *reinterpret_cast<const v4u *>(&xc[wave][t][pidx(8 * (g0 + g)) + 4]);
      xa[g][0] = p0.x; xa[g][1] = p0.y; xa[g][2] = p0.z; xa[g][3] = p0.w;
      xa[g][4] = p1.x; xa[g][5] = p1.y; xa[g][6] = p1.z; xa[g][7] = p1.w;
      md[g] = xm[wave][t][g0 + g][0];
      ms[g] = xm[wave][t][g0 + g][1];
    }
  };
  // Up to two tokens every fragment a unit needs is read at once (for the first unit before the weights are
  // awaited); beyond two tokens one token's at a time inside the token loop, so the registers do not grow with the
  // token count.
  constexpr bool kHoist = TG <= 2;
  constexpr int TH = kHoist ? TG : 1;
  u32 xah[TH][4][8];
  float mdh[TH][4], msh[TH][4];
  float part[NM][TG];

  // the math of unit u held in slot `slot`: adds the lane's partial sums of its half super-block into part[]
  auto unit_math = [&](int u, auto slotc, bool first) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
    if constexpr (kHoist) {
#pragma unroll
      for (int t = 0; t < TG; ++t) frag(t, u, xah[t], mdh[t], msh[t]);
      if (first) {
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i2 = 0; i2 < 8; ++i2) asm volatile("" ::"v"(xah[t][g][i2]));
            asm volatile("" ::"v"(mdh[t][g]), "v"(msh[t][g]));
          }
      }
    }
    v4u hd[NM];
    u32 q[NM][16];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      hd[m] = wd[m][slot][0];
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) {
        q[m][4 * i2] = wd[m][slot][1 + i2].x; q[m][4 * i2 + 1] = wd[m][slot][1 + i2].y;
        q[m][4 * i2 + 2] = wd[m][slot][1 + i2].z; q[m][4 * i2 + 3] = wd[m][slot][1 + i2].w;
      }
    }
    if constexpr (U > 1) {
      if (u + NSLOT < U) load_unit(slot, u + NSLOT);
    }
    u32 lo[NM][16], hi[NM][16];   // the code nibbles as int8 lanes, shared by every token
    float sc[NM][4], mn[NM][4];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) { lo[m][i2] = q[m][i2] & 0x0F0F0F0Fu; hi[m][i2] = (q[m][i2] >> 4) & 0x0F0F0F0Fu; }
      if constexpr (WF == kTQ40) {   // the d of blocks 4 h .. 4 h + 3 of the span: dwords 2 h, 2 h + 1
        const u32 w0 = h ? hd[m].z : hd[m].x, w1 = h ? hd[m].w : hd[m].y;
        sc[m][0] = f16_to_f32(w0); sc[m][1] = f16_to_f32(w0 >> 16);
        sc[m][2] = f16_to_f32(w1); sc[m][3] = f16_to_f32(w1 >> 16);
#pragma unroll
        for (int g = 0; g < 4; ++g) mn[m][g] = 0.f;
      } else {
        const float d = f16_to_f32(hd[m].x), dmin = f16_to_f32(hd[m].x >> 16);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32 s_, m_;
          q4k_scale_min(hd[m].y, hd[m].z, hd[m].w, 4 * h + g, s_, m_);
          sc[m][g] = d * (float)s_;
          mn[m][g] = dmin * (float)m_;
        }
      }
    }
    auto token = [&](int t, const u32 (&xa)[4][8], const float (&md)[4], const float (&ms)[4])
        __attribute__((always_inline)) {
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        float p = 0.f;
#pragma unroll
        for (int pg = 0; pg < 2; ++pg) {   // code pages 2 h and 2 h + 1: low nibbles group 2 pg, high 2 pg + 1
          int ia = 0, ib = 0;
#pragma unroll
          for (int i2 = 0; i2 < 8; ++i2) {
            ia = sdot4(lo[m][8 * pg + i2], xa[2 * pg][i2], ia);
            ib = sdot4(hi[m][8 * pg + i2], xa[2 * pg + 1][i2], ib);
          }
          if constexpr (WF == kTQ40) {   // codes q - 8: the code sum is an exact integer
            ia -= 8 * (int)ms[2 * pg];
            ib -= 8 * (int)ms[2 * pg + 1];
            p += (sc[m][2 * pg] * md[2 * pg]) * (float)ia;
            p += (sc[m][2 * pg + 1] * md[2 * pg + 1]) * (float)ib;
          } else {
            p += ((float)ia * sc[m][2 * pg] - ms[2 * pg] * mn[m][2 * pg]) * md[2 * pg];
            p += ((float)ib * sc[m][2 * pg + 1] - ms[2 * pg + 1] * mn[m][2 * pg + 1]) * md[2 * pg + 1];
          }
        }
        part[m][t] = u == 0 ? p : part[m][t] + p;
      }
    };
    if constexpr (kHoist) {
#pragma unroll
      for (int t = 0; t < TG; ++t) token(t, xah[t], mdh[t], msh[t]);
    } else {
#pragma unroll
      for (int t = 0; t < TG; ++t) {
        u32 xa[4][8];
        float md[4], ms[4];
        frag(t, u, xa, md, ms);
        token(t, xa, md, ms);
      }
    }
  };
  if constexpr (U == 1) {
    unit_math(0, std::integral_constant<int, 0>{}, true);
  } else if constexpr (NSLOT == 1) {
#pragma unroll 1
    for (int u = 0; u < U; ++u) unit_math(u, std::integral_constant<int, 0>{}, u == 0);
  } else {
    // units in pairs (slots 0 and 1 as constants); the pair loop is not unrolled, so only one pair's fragments
    // are live at a time
#pragma unroll 1
    for (int u = 0; u < U; u += 2) {
      unit_math(u, std::integral_constant<int, 0>{}, u == 0);
      if (u + 1 < U) unit_math(u + 1, std::integral_constant<int, 1>{}, false);
    }
  }
  // the row's four lanes of this wave (its two super-blocks' halves) meet in a butterfly, then the waves in LDS
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      float p = part[m][t];
      p += xshfl<1>(p);
      p += xshfl<2>(p);
      part[m][t] = p;
    }
  if ((lane & 3) == 0) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < TG; ++t) red[wave][m][r][t] = part[m][t];
  }
  __syncthreads();
  if (tid < 16 * TG) {
    const int rr = tid / TG, t = tid % TG;
    float tot[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      tot[m] = 0.f;
      for (int wv = 0; wv < NW; ++wv) tot[m] += red[wv][m][rr][t];
    }
    const int64_t row = 16 * rb + rr, tok = t0 + t;
    if (tok < tokens) {
      float *py = y + tok * n + row;
      if constexpr (MODE == kSwiglu) {
        const float v = tot[0] / (1.0f + expf(-tot[0])) * tot[NM - 1];
        *py = accumulate ? *py + v : v;
      } else {
        *py = accumulate ? *py + tot[0] : tot[0];
      }
      if constexpr (MODE == kPair) {
        float *py2 = y2 + tok * n + row;
        *py2 = accumulate ? *py2 + tot[NM - 1] : tot[NM - 1];
      }
    }
  }
}

// the launch arguments of one call (the weights and outputs of the second matrix for swiglu / pair)
// ------------------------------------------------------------------------- Q4_0 tiled, f32 / bf16 activations
// The reference's default Q4_0 decode (its int8 path covers Q4_0 only with Q4_0_Q8=1, S/formats.py:20-30): the matvec
// g_mv_q4_0_k{K}[_t{TG}] on f32 activations (S/gen_llm.py:1187-1197 with @g_q4_0_values, S/quant_values.loom:386-408)
// over the tiled units (QMM_Q4_0T), with the int8 kernel's launch shape and lane map. Each wave stages its K slice of
// every token in LDS as f32 with the sum of each 32-value block (four lanes' chunks, summed in a fixed tree); a lane
// then contracts its four blocks (4 h .. 4 h + 3 of span sb of row r) with them, s = sum q x over the block's codes
// 0..15 as f32 (one fma chain in value order), and adds d (s - 8 sum x): sum d (q - 8) x up to f32 rounding. The row's
// four lanes meet in a butterfly, the waves in LDS in a fixed order, so a multi-token call equals one-token calls.
template <int TG, int U, bool BF>
__global__ __launch_bounds__(kMaxWaves * 64) void mv_q40t_f32_kernel(int64_t n, int64_t tokens, int64_t K,
                                                                     int accumulate, const void *__restrict__ x,
                                                                     const u8 *__restrict__ w, float *__restrict__ y) {
  constexpr int SLICE = 512 * U, NB = SLICE / 32;
  __shared__ __align__(16) float xs[kMaxWaves][TG][SLICE];
  __shared__ float xsum[kMaxWaves][TG][NB];
  __shared__ float red[kMaxWaves][16][TG];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NW = (int)(blockDim.x >> 6);
  const int64_t t0 = (int64_t)blockIdx.y * TG;
  const int64_t rb = blockIdx.x;
  const int r = lane >> 2, sb = (lane >> 1) & 1, h = lane & 1;
  const int64_t k0 = (int64_t)wave * SLICE;

  // ---- the wave's activations (chunk c = lane + 64 j: 8 values), then its U units (a header and four planes each)
  float xv[TG][U][8];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const int64_t tok = t0 + t < tokens ? t0 + t : tokens - 1;
#pragma unroll
    for (int j = 0; j < U; ++j) load8(x, BF, tok * K + k0 + 8 * (lane + 64 * j), xv[t][j]);
  }
  v4u wd[U][5];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const v4u *up = reinterpret_cast<const v4u *>(w + (rb * (K / 512) + (int64_t)wave * U + u) * kUnit);
    wd[u][0] = up[lane >> 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) wd[u][1 + q] = up[32 + 64 * q + lane];
  }
#pragma unroll
  for (int t = 0; t < TG; ++t)
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int c = lane + 64 * j;
      float4 *dst = reinterpret_cast<float4 *>(&xs[wave][t][8 * c]);
      dst[0] = make_float4(xv[t][j][0], xv[t][j][1], xv[t][j][2], xv[t][j][3]);
      dst[1] = make_float4(xv[t][j][4], xv[t][j][5], xv[t][j][6], xv[t][j][7]);
      float bs = xv[t][j][0];
#pragma unroll
      for (int i = 1; i < 8; ++i) bs += xv[t][j][i];
      bs += xshfl<1>(bs);
      bs += xshfl<2>(bs);
      if ((c & 3) == 0) xsum[wave][t][c >> 2] = bs;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- math: block 4 h + blk of the span is page 2 h + blk / 2 (low nibbles for even blk, high for odd), its codes
  //      16 half .. 16 half + 15 in plane 2 (blk / 2) + half
  float part[TG];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const v4u hd = wd[u][0];
    const u32 w0 = h ? hd.z : hd.x, w1 = h ? hd.w : hd.y;
    const float d[4] = {f16_to_f32(w0), f16_to_f32(w0 >> 16), f16_to_f32(w1), f16_to_f32(w1 >> 16)};
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      float p = 0.f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int base = 512 * u + 32 * (8 * sb + 4 * h + blk);   // the block's first value in the slice
        float sq = 0.f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const v4u pl = wd[u][1 + 2 * (blk >> 1) + half];
          const u32 dw[4] = {pl.x, pl.y, pl.z, pl.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32 cq = (blk & 1 ? dw[i] >> 4 : dw[i]) & 0x0F0F0F0Fu;
            const float4 xq = *reinterpret_cast<const float4 *>(&xs[wave][t][base + 16 * half + 4 * i]);
            sq = __builtin_fmaf((float)((cq >> 0) & 255u), xq.x, sq);
            sq = __builtin_fmaf((float)((cq >> 8) & 255u), xq.y, sq);
            sq = __builtin_fmaf((float)((cq >> 16) & 255u), xq.z, sq);
            sq = __builtin_fmaf((float)((cq >> 24) & 255u), xq.w, sq);
          }
        }
        p += d[blk] * (sq - 8.f * xsum[wave][t][16 * u + 8 * sb + 4 * h + blk]);
      }
      part[t] = u == 0 ? p : part[t] + p;
    }
  }
  // ---- the row's four lanes (h, then sb), then the waves in order
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    float v = part[t];
    v += xshfl<1>(v);
    v += xshfl<2>(v);
    if ((lane & 3) == 0) red[wave][r][t] = v;
  }
  __syncthreads();
  if (tid < 16 * TG) {
    const int rr = tid / TG, t = tid % TG;
    float tot = red[0][rr][t];
    for (int wv = 1; wv < NW; ++wv) tot += red[wv][rr][t];
    const int64_t row = 16 * rb + rr, tok = t0 + t;
    if (row < n && tok < tokens) {
      float *py = y + tok * n + row;
      *py = accumulate ? *py + tot : tot;
    }
  }
}

template <int TG, int U>
int launch_q40t_f32(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, bool bf, const void *w,
                    float *y, int nw, hipStream_t s) {
  const dim3 grid((unsigned)(n / 16), (unsigned)((tokens + TG - 1) / TG));
  if (bf)
    mv_q40t_f32_kernel<TG, U, true><<<grid, nw * 64, 0, s>>>(n, tokens, k, accumulate, x, static_cast<const u8 *>(w), y);
  else
    mv_q40t_f32_kernel<TG, U, false><<<grid, nw * 64, 0, s>>>(n, tokens, k, accumulate, x, static_cast<const u8 *>(w),
                                                              y);
  return launch_status();
}

struct TArgs {
  int64_t n, tokens, k;
  int accumulate;
  const void *x;
  int bf;
  const void *w, *w2;
  float *y, *y2;
  int nw;
  int wf;   // TFmt
};

template <int TG, int U, bool STAGEQ, int MODE>
int launch_tg(const TArgs &a, hipStream_t s) {
  const dim3 grid((unsigned)(a.n / 16), (unsigned)((a.tokens + TG - 1) / TG));
  if (a.wf == kTQ40) {
    mv_q4kt_q8_kernel<TG, U, STAGEQ, MODE, kTQ40><<<grid, a.nw * 64, 0, s>>>(
        a.n, a.tokens, a.k, a.accumulate, a.x, a.bf, static_cast<const u8 *>(a.w), static_cast<const u8 *>(a.w2), a.y,
        a.y2);
    return launch_status();
  }
  mv_q4kt_q8_kernel<TG, U, STAGEQ, MODE, kTQ4K><<<grid, a.nw * 64, 0, s>>>(
      a.n, a.tokens, a.k, a.accumulate, a.x, a.bf, static_cast<const u8 *>(a.w), static_cast<const u8 *>(a.w2), a.y,
      a.y2);
  return launch_status();
}

template <int U, bool STAGEQ, int MODE>
int launch_u(const TArgs &a, hipStream_t s) {
  // up to 8 tokens a workgroup share its weight loads (the activations of a token stage U x 8 registers a lane,
  // so the token group shrinks as the slices a wave grow: 8, 4, 2, 1 for U = 1..4, halved again when two matrices
  // stream); the group is the smallest power of two holding every token, a workgroup's spare slots repeating its
  // last token without storing it
  constexpr int TG1 = U == 1 ? 8 : U == 2 ? 4 : U == 3 ? 2 : 1;
  constexpr int TGMAX = MODE == kPlain ? TG1 : (TG1 > 1 ? TG1 / 2 : 1);
  constexpr int T8 = TGMAX >= 8 ? 8 : 1, T4 = TGMAX >= 4 ? 4 : 1, T2 = TGMAX >= 2 ? 2 : 1;
  const int64_t tokens = a.tokens;
  // the output stage takes one thread an output (16 rows x TG tokens): eight tokens need two waves (K >= 1024)
  if (tokens >= 5 && T8 == 8 && a.nw >= 2) return launch_tg<T8, U, STAGEQ, MODE>(a, s);
  if (tokens >= 3 && T4 == 4) return launch_tg<T4, U, STAGEQ, MODE>(a, s);
  if (tokens >= 2 && T2 == 2) return launch_tg<T2, U, STAGEQ, MODE>(a, s);
  return launch_tg<1, U, STAGEQ, MODE>(a, s);
}

// One thread per 16-byte piece of the tiled matrix. A row block is 16 rows x K / 256 super-blocks: F = K / 512 full
// units of 288 pieces (pieces 0..31 the headers of (row p / 2, super-block p % 2), the others the code planes), then,
// when K % 512 == 256, a half unit of 144 pieces (pieces 0..15 the headers of the rows' last super-blocks, then four
// planes of 32 pieces, piece 32 q + 2 r + h holding code bytes 16 (4 h + q) of row r).
__global__ void tile_q4k_kernel(const u8 *__restrict__ src, int64_t rows, int64_t K, u8 *__restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rbp = K / 256 * 144;   // pieces of a row block: 16 rows x K / 256 x 144 bytes / 16
  if (i >= rows / 16 * rbp) return;
  const int64_t rb = i / rbp;
  const int p = (int)(i % rbp), F = (int)(K / 512);
  const int sl = p / (kUnit / 16), pu = p % (kUnit / 16);
  int r, b, off;
  if (sl < F) {
    if (pu < 32) {
      r = pu >> 1; b = 2 * sl + (pu & 1); off = 0;
    } else {
      const int q = (pu - 32) >> 6, l = (pu - 32) & 63;
      r = l >> 2; b = 2 * sl + ((l >> 1) & 1);
      off = 16 + 16 * (4 * (l & 1) + q);
    }
  } else {
    const int ph = p - F * (kUnit / 16);
    if (ph < 16) {
      r = ph; off = 0;
    } else {
      const int q = (ph - 16) >> 5, l = (ph - 16) & 31;
      r = l >> 1;
      off = 16 + 16 * (4 * (l & 1) + q);
    }
    b = 2 * F;
  }
  const u8 *blk = src + (16 * rb + r) * (K / 256 * 144) + (int64_t)b * 144 + off;
  *reinterpret_cast<v4u *>(dst + 16 * i) = *reinterpret_cast<const v4u *>(blk);
}

// f32 values of a tiled Q4_K matrix, one thread per 32-value sub-block, the value helper's arithmetic
// (S/gen_llm.py:269-326): (f32(d) sc) q - f32(dmin) m.
__global__ void dequant_q4kt_kernel(const u8 *__restrict__ w, int64_t rows, int64_t K, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t G = K / 32;
  if (gi >= rows * G) return;
  const int64_t row = gi / G;
  const int g = (int)(gi % G), b = g >> 3, s = g & 7;
  const int i = (int)(row & 15), sb = b & 1, F = (int)(K / 512);
  const u8 *rbase = w + (row >> 4) * (K / 256 * 144 * 16);
  const bool tail = b >= 2 * F;   // the half unit of K % 512 == 256
  const u8 *unit = rbase + (int64_t)(tail ? F : b >> 1) * kUnit;
  const u32 *hd = reinterpret_cast<const u32 *>(unit + (tail ? 16 * i : 16 * (2 * i + sb)));
  u32 sc, mn;
  q4k_scale_min(hd[1], hd[2], hd[3], s, sc, mn);
  const float scale = f16_to_f32(hd[0]) * (float)sc;
  const float minimum = f16_to_f32(hd[0] >> 16) * (float)mn;
  const int shift = 4 * (s & 1);
  float *o = out + gi * 32;
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    const int c = 32 * (s >> 1) + l;   // code byte of the super-block
    const int q = (c >> 4) & 3, h = c >> 6;
    const u8 v = tail ? unit[256 + 512 * q + 16 * (2 * i + h) + (c & 15)]
                      : unit[512 + 1024 * q + 16 * (4 * i + 2 * sb + h) + (c & 15)];
    o[l] = __fsub_rn(__fmul_rn(scale, (float)((v >> shift) & 15u)), minimum);
  }
}


// Q4_0 -> QMM_Q4_0T, one thread per 16-byte piece of the tiled matrix: unit (row block, slice) pieces 0..31 the
// header slots (row p / 2, span p % 2: its eight d), then four planes of 64 pieces, piece 32 + 64 q + l (l = 4 r + 2 sb
// + h) holding bytes 16 (4 h + q) .. + 15 of row r's span sb: byte 32 P + i of a span is code i of block 2 P in its
// low nibble and code i of block 2 P + 1 in its high nibble (code i of a block: byte i & 15, low nibble for i < 16).
__global__ void tile_q40_kernel(const u8 *__restrict__ src, int64_t rows, int64_t K, u8 *__restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rbp = K / 512 * (kUnit / 16);   // pieces of a row block
  if (i >= rows / 16 * rbp) return;
  const int64_t rb = i / rbp;
  const int p = (int)(i % rbp), u = p / (kUnit / 16), pu = p % (kUnit / 16);
  const int64_t RB = K / 32 * 18;
  u32 o[4];
  if (pu < 32) {
    const int r = pu >> 1, sb = pu & 1;
    const u8 *row = src + (16 * rb + r) * RB + (int64_t)(16 * u + 8 * sb) * 18;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = (u32)row[36 * j] | ((u32)row[36 * j + 1] << 8) | ((u32)row[36 * j + 18] << 16) | ((u32)row[36 * j + 19] << 24);
  } else {
    const int q = (pu - 32) >> 6, l = (pu - 32) & 63, r = l >> 2, sb = (l >> 1) & 1, h = l & 1;
    const u8 *row = src + (16 * rb + r) * RB + (int64_t)(16 * u + 8 * sb) * 18;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = 0u;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int c = 16 * (4 * h + q) + b, P = c >> 5, ci = c & 31;   // span byte c: page P, code index ci
      const u8 *b0 = row + (2 * P) * 18 + 2, *b1 = row + (2 * P + 1) * 18 + 2;
      const u32 lo = ci < 16 ? b0[ci] & 15u : (u32)b0[ci - 16] >> 4;
      const u32 hi = ci < 16 ? b1[ci] & 15u : (u32)b1[ci - 16] >> 4;
      o[b >> 2] |= (lo | (hi << 4)) << (8 * (b & 3));
    }
  }
  *reinterpret_cast<v4u *>(dst + 16 * i) = v4u{o[0], o[1], o[2], o[3]};
}

// f32 values of a QMM_Q4_0T matrix, one thread per block: d (q - 8) as the value helper (S/quant_values.loom:386-408)
__global__ void dequant_q40t_kernel(const u8 *__restrict__ w, int64_t rows, int64_t K, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t G = K / 32;
  if (gi >= rows * G) return;
  const int64_t row = gi / G;
  const int b = (int)(gi % G), u = b >> 4, sb = (b >> 3) & 1, j = b & 7, r = (int)(row & 15);
  const u8 *unit = w + ((row >> 4) * (K / 512) + u) * kUnit;
  const u16 dbits = *reinterpret_cast<const u16 *>(unit + 16 * (2 * r + sb) + 2 * j);
  const float d = f16_to_f32(dbits);
  float *o = out + gi * 32;
#pragma unroll
  for (int v = 0; v < 32; ++v) {
    const int c = 32 * (j >> 1) + v, h = c >> 6, q = (c >> 4) & 3;
    const u8 byte = unit[512 + 1024 * q + 16 * (4 * r + 2 * sb + h) + (c & 15)];
    const int code = (j & 1) ? byte >> 4 : byte & 15;
    o[v] = __fmul_rn(d, (float)(code - 8));
  }
}

template <int MODE>
int launch_mode(TArgs &a, int x_dtype, hipStream_t s) {
  if (a.n % 16 || a.k % 512 || a.n / 16 > 2147483647ll || a.tokens > 65535) return QMM_ERR_SHAPE;   // grid.y <= 65535
  const int64_t slices = a.k / 512;
  int U = 1;
  while (U <= 4 && (slices % U || slices / U > kMaxWaves)) ++U;
  if (U > 4) return QMM_ERR_SHAPE;
  a.nw = (int)(slices / U);
  const bool stage = x_dtype != QMM_Q8;
  a.bf = x_dtype == QMM_BF16;
  switch (U) {
    case 1: return stage ? launch_u<1, true, MODE>(a, s) : launch_u<1, false, MODE>(a, s);
    case 2: return stage ? launch_u<2, true, MODE>(a, s) : launch_u<2, false, MODE>(a, s);
    case 3: return stage ? launch_u<3, true, MODE>(a, s) : launch_u<3, false, MODE>(a, s);
    default: return stage ? launch_u<4, true, MODE>(a, s) : launch_u<4, false, MODE>(a, s);
  }
}

}  // namespace

// The tiled-layout path of qmm_mv_q8 (fmt QMM_Q4_KT): rows % 16 == 0, K % 512 == 0, K = 512 U NW with U <= 4
// slices a wave and NW <= 8 waves. mode 0: y = x W^T; 1 (swiglu): y = silu(x W^T) (x W2^T); 2 (pair): y = x W^T and
// y2 = x W2^T.
int qmm_mv_q4kt_q8(int fmt, int mode, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                   int x_dtype, const void *w, const void *w2, float *y, float *y2, hipStream_t s) {
  TArgs a{n, tokens, k, accumulate, x, 0, w, w2, y, y2, 0, fmt == QMM_Q4_0T ? kTQ40 : kTQ4K};
  if (mode == kSwiglu) return launch_mode<kSwiglu>(a, x_dtype, s);
  if (mode == kPair) return launch_mode<kPair>(a, x_dtype, s);
  return launch_mode<kPlain>(a, x_dtype, s);
}


// The f32 / bf16-activation matvec of the tiled Q4_0 layout (the qmm_mv path of QMM_Q4_0T): rows % 16 == 0,
// K = 512 U NW with U <= 3 slices a wave (the staged slices fit a workgroup's LDS) and NW <= 8 waves; a workgroup a
// (row block, token).
int qmm_mv_q40t_f32(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype, const void *w,
                    float *y, hipStream_t s) {
  if (n % 16 || k % 512 || n / 16 > 2147483647ll || tokens > 65535) return QMM_ERR_SHAPE;
  const int64_t slices = k / 512;
  int U = 1;
  while (U <= 3 && (slices % U || slices / U > kMaxWaves)) ++U;
  if (U > 3) return QMM_ERR_SHAPE;
  const int nw = (int)(slices / U);
  const bool bf = x_dtype == QMM_BF16;
  if (U == 1) return launch_q40t_f32<1, 1>(k, n, tokens, accumulate, x, bf, w, y, nw, s);
  return U == 2 ? launch_q40t_f32<1, 2>(k, n, tokens, accumulate, x, bf, w, y, nw, s)
                : launch_q40t_f32<1, 3>(k, n, tokens, accumulate, x, bf, w, y, nw, s);
}

int qmm_dequant_q4kt(const void *w, int64_t rows, int64_t k, float *out, hipStream_t s) {
  if (rows % 16 || k % 256) return QMM_ERR_SHAPE;
  if (!aligned(w, 4)) return QMM_ERR_ALIGN;
  const int64_t groups = rows * (k / 32);
  dequant_q4kt_kernel<<<(unsigned)((groups + 255) / 256), 256, 0, s>>>(static_cast<const u8 *>(w), rows, k, out);
  return launch_status();
}

int qmm_dequant_q40t(const void *w, int64_t rows, int64_t k, float *out, hipStream_t s) {
  if (rows % 16 || k % 512) return QMM_ERR_SHAPE;
  if (!aligned(w, 4)) return QMM_ERR_ALIGN;
  const int64_t blocks = rows * (k / 32);
  dequant_q40t_kernel<<<(unsigned)((blocks + 255) / 256), 256, 0, s>>>(static_cast<const u8 *>(w), rows, k, out);
  return launch_status();
}

extern "C" int qmm_tile_q40(const void *w, int64_t rows, int64_t k, void *w_t, qmm_stream_t stream) {
  if (!w || !w_t) return QMM_ERR_NULL;
  if (rows <= 0 || rows % 16 || k <= 0 || k % 512 || k > (1 << 20)) return QMM_ERR_SHAPE;
  if (!aligned(w_t, 16)) return QMM_ERR_ALIGN;
  const int64_t pieces = rows / 16 * (k / 512) * (kUnit / 16);
  tile_q40_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const u8 *>(w), rows, k, static_cast<u8 *>(w_t));
  return launch_status();
}

extern "C" int qmm_tile_q4k(const void *w, int64_t rows, int64_t k, void *w_t, qmm_stream_t stream) {
  if (!w || !w_t) return QMM_ERR_NULL;
  if (rows <= 0 || rows % 16 || k <= 0 || k % 256 || k > (1 << 20)) return QMM_ERR_SHAPE;
  if (!aligned(w, 16) || !aligned(w_t, 16)) return QMM_ERR_ALIGN;
  const int64_t pieces = rows * (k / 256) * 9;   // 16-byte pieces: 144 bytes a super-block
  tile_q4k_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const u8 *>(w), rows, k, static_cast<u8 *>(w_t));
  return launch_status();
}
