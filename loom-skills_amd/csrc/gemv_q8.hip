// Decode matvecs on Q8_1 activations, the reference's default decode path (ACT_Q8 = 1, S/gen_llm.py:519):
//
//   qmm_quant_q8   x f32 / bf16 [rows, K] -> planar Q8_1               g_quant_q8, S/gen_llm.py:684-749
//   qmm_mv_q8      y[t, r] (+)= sum over 32-value groups g of the row   g_mv_{fmt}_k{K}[_t{TG}]_q8[_r{R}],
//                                                                        S/gen_llm.py:1288-1301
//
// Planar Q8_1 (the reference's layout): int8 codes [rows][K/32][32], then at byte rows * K the f32 pairs
// (f16-rounded d, sum of the group's codes) [rows][K/32][2]. Per group of 32 (llama.cpp quantize_q8_1, oracle
// make_kernel_tests.py:32-39): d = amax / 127, q = sign(x/d) floor(|x/d| + 1/2), q = 0 when d = 0.
//
// Weight side (iq_dot, S/gen_llm.py:1024-1071): a group's integer dot di = sum q_w q_x is exact (v_dot4_i32_i8
// over eight dwords). Q4_K keeps its unsigned 4-bit codes; with sc = d sc_g and mn = dmin m_g (f32) the group adds
// (di sc - xs mn) da, da the f16-rounded activation scale and xs the code sum. Q4_0 codes are q - 8: di is taken on
// the unsigned nibbles and 8 xs subtracted (the same integer), and the group adds (sc da) di with sc = d.
//
// Kernels. The quantizer gives each 32-value group to four consecutive lanes (8 values each). The generic matvec
// is the item walk of gemv.hip with Q8 activation fragments (any K % 256 for Q4_K, K % 64 for Q4_0). The Q4_K fast
// path (K = 4096, 8192) splits K between the eight waves of a workgroup (see mv_q4k_q8s_kernel); given f32 / bf16
// activations it quantizes them while staging, with the quantizer's own arithmetic, so both input forms give
// identical results. The generic matvec also streams two matrices of one input: swiglu y = silu(x W^T) (x W2^T)
// (g_mv_{fmt}_k{K}_swiglu[_t{TG}]_q8) and pair y = x W^T, y2 = x W2^T (g_mv_{fmt}_k{K}_pair[_t{TG}]_q8,
// S/gen_llm.py:1159-1197), each matrix's rows rounded as the one-matrix kernel rounds them.
//
//   qmm_moe_expert_mv_q8  the decode expert matvecs on Q8_1 activations, g_moe_{gu|dn}_{fmt}[_fused]_q8_k{K}_r{R}
//                         (S/gen_moe.py:535-727 with iq; the MOE_Q8 default of S/gen_llm.py:5290-5303)
#include "bfly.hpp"
#include "rowdot.hpp"

using namespace qmm;

namespace {

typedef __attribute__((ext_vector_type(4))) u32 v4u;
typedef __attribute__((ext_vector_type(2))) u32 v2u;

__device__ __forceinline__ int sdot4(u32 a, u32 b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 8 activations of the lane as f32: from 16 bytes of bf16 or 32 bytes of f32 at element offset e
__device__ __forceinline__ void load8_act(const void *x, bool bf, int64_t e, float (&v)[8]) {
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

// One 32-value group held by four consecutive lanes of a wave (8 values each, the group's first lane a multiple of
// 4): the lane's 8 codes as two dwords, and the group's f16-rounded d and code sum.
__device__ __forceinline__ void q8_group4(const float (&v)[8], u32 &c0, u32 &c1, float &d16, float &sum) {
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

// --------------------------------------------------------------------------------------------- quantizer
__global__ __launch_bounds__(256) void quant_q8_kernel(int64_t rows, int64_t k, const void *__restrict__ x, int bf,
                                                       u8 *__restrict__ xq) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // 8-value chunk
  const int64_t chunks = rows * (k / 8);
  const bool in = i < chunks;
  const int64_t ic = in ? i : chunks - 1;                       // the group's lanes stay together (chunks % 4 == 0)
  float v[8];
  load8_act(x, bf, ic * 8, v);
  u32 c0, c1;
  float d16, sum;
  q8_group4(v, c0, c1, d16, sum);
  if (!in) return;
  reinterpret_cast<v2u *>(xq)[ic] = v2u{c0, c1};
  if ((threadIdx.x & 3) == 0) {
    float *meta = reinterpret_cast<float *>(xq + rows * k);
    reinterpret_cast<float2 *>(meta)[ic / 4] = make_float2(d16, sum);
  }
}

// ------------------------------------------------------------------------------------ generic matvec
// Activation fragment of an item of 64 values = groups A and B: 8 code dwords each and their (d, code sum).
struct XQ {
  u32 a[8], b[8];
  float da, sa, db, sb;
};

__device__ __forceinline__ void xq_load(const u8 *codes, const float *meta, int64_t g, bool live, XQ &x) {
  const v4u *c = reinterpret_cast<const v4u *>(codes + 32 * g);
  const v4u m = live ? *reinterpret_cast<const v4u *>(meta + 2 * g) : v4u{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const v4u p = live ? c[i] : v4u{0u, 0u, 0u, 0u}, q = live ? c[2 + i] : v4u{0u, 0u, 0u, 0u};
    x.a[4 * i] = p.x; x.a[4 * i + 1] = p.y; x.a[4 * i + 2] = p.z; x.a[4 * i + 3] = p.w;
    x.b[4 * i] = q.x; x.b[4 * i + 1] = q.y; x.b[4 * i + 2] = q.z; x.b[4 * i + 3] = q.w;
  }
  x.da = u32_as_f32(m.x); x.sa = u32_as_f32(m.y); x.db = u32_as_f32(m.z); x.sb = u32_as_f32(m.w);
}

// Q4_K: item = 4 * block + page j; groups 8 block + 2 j (low nibbles) and + 1 (high nibbles)
struct Q4K8 {
  static constexpr bool kSplit = false;
  struct W { v4u h, q0, q1; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 256) * 4; }
  static __device__ __forceinline__ int64_t group(int item) { return (int64_t)(item >> 2) * 8 + 2 * (item & 3); }
  static __device__ __forceinline__ void load_w(const u8 *row, int item, bool live, W &w) {
    const u8 *b = row + (int64_t)(item >> 2) * 144;
    const int j = item & 3;
    const v4u z{0u, 0u, 0u, 0u};
    w.h = live ? *reinterpret_cast<const v4u *>(b) : z;
    w.q0 = live ? *reinterpret_cast<const v4u *>(b + 16 + 32 * j) : z;
    w.q1 = live ? *reinterpret_cast<const v4u *>(b + 32 + 32 * j) : z;
  }
  static __device__ __forceinline__ float dot(const W &w, const XQ &x, int item) {
    const int j = item & 3;
    u32 sc0, m0, sc1, m1;
    q4k_scale_min(w.h.y, w.h.z, w.h.w, 2 * j, sc0, m0);
    q4k_scale_min(w.h.y, w.h.z, w.h.w, 2 * j + 1, sc1, m1);
    const float d = f16_to_f32(w.h.x), dmin = f16_to_f32(w.h.x >> 16);
    const u32 q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    int ia = 0, ib = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ia = sdot4(q[i] & 0x0F0F0F0Fu, x.a[i], ia);
      ib = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, x.b[i], ib);
    }
    const float ga = ((float)ia * (d * (float)sc0) - x.sa * (dmin * (float)m0)) * x.da;
    const float gb = ((float)ib * (d * (float)sc1) - x.sb * (dmin * (float)m1)) * x.db;
    return ga + gb;
  }
};

// Q4_0: item = pair of blocks p (36 bytes at 36 p, 4-byte aligned when K % 64 == 0); groups 2 p and 2 p + 1
struct Q408 {
  static constexpr bool kSplit = false;
  struct W { u32 v[9]; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 64); }
  static __device__ __forceinline__ int64_t group(int item) { return 2 * (int64_t)item; }
  static __device__ __forceinline__ void load_w(const u8 *row, int item, bool live, W &w) {
    const u32 *p = reinterpret_cast<const u32 *>(row + (int64_t)item * 36);
#pragma unroll
    for (int i = 0; i < 9; ++i) w.v[i] = live ? p[i] : 0u;
  }
  static __device__ __forceinline__ float dot(const W &w, const XQ &x, int) {
    const float d[2] = {f16_to_f32(w.v[0]), f16_to_f32(w.v[4] >> 16)};
    const u32 q0[4] = {__builtin_amdgcn_alignbit(w.v[1], w.v[0], 16), __builtin_amdgcn_alignbit(w.v[2], w.v[1], 16),
                       __builtin_amdgcn_alignbit(w.v[3], w.v[2], 16), __builtin_amdgcn_alignbit(w.v[4], w.v[3], 16)};
    const u32 q1[4] = {w.v[5], w.v[6], w.v[7], w.v[8]};
    // a block's low nibbles are its values 0..15 (activation dwords 0..3), its high nibbles values 16..31
    int ia = 0, ib = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ia = sdot4(q0[i] & 0x0F0F0F0Fu, x.a[i], ia);
      ia = sdot4((q0[i] >> 4) & 0x0F0F0F0Fu, x.a[4 + i], ia);
      ib = sdot4(q1[i] & 0x0F0F0F0Fu, x.b[i], ib);
      ib = sdot4((q1[i] >> 4) & 0x0F0F0F0Fu, x.b[4 + i], ib);
    }
    ia -= 8 * (int)x.sa;   // codes q - 8: the code sum is an exact integer
    ib -= 8 * (int)x.sb;
    return (d[0] * x.da) * (float)ia + (d[1] * x.db) * (float)ib;
  }
};

// Q6_K: item = 4 b + 2 half + jh (rowdot.hpp q6k_load); groups 2 item (values 0..31) and 2 item + 1. The codes are
// taken unsigned and 32 times the activation code sum of each 16-value run removed, the same integer as the
// reference's signed codes q - 32 (iq_dot, S/gen_llm.py:1036-1044): per group (ilo s0 + ihi s1) da, s = d sc.
struct Q6K8 {
  static constexpr bool kSplit = false;
  using W = Q6W;
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 256) * 4; }
  static __device__ __forceinline__ int64_t group(int item) { return 2 * (int64_t)item; }
  static __device__ __forceinline__ void load_w(const u8 *row, int item, bool live, W &w) {
    q6k_load(row, item, live, w);
  }
  static __device__ __forceinline__ float dot(const W &w, const XQ &x, int item) {
    u32 ca[8], cb[8];
    q6k_codes(w, item & 1, ca, cb);
    float s[4];
    q6k_scales(w, s);
    int i16[4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      int ia = 0, za = 0, ib = 0, zb = 0;
#pragma unroll
      for (int i = 4 * q; i < 4 * q + 4; ++i) {
        ia = sdot4(ca[i], x.a[i], ia);
        za = sdot4(0x20202020u, x.a[i], za);
        ib = sdot4(cb[i], x.b[i], ib);
        zb = sdot4(0x20202020u, x.b[i], zb);
      }
      i16[q] = ia - za;
      i16[2 + q] = ib - zb;
    }
    const float ga = __builtin_fmaf((float)i16[1], s[1], (float)i16[0] * s[0]) * x.da;
    const float gb = __builtin_fmaf((float)i16[3], s[3], (float)i16[2] * s[2]) * x.db;
    return ga + gb;
  }
};

// MXFP4 split planes, the reference's opt-in int8 decode (MXFP4S_Q8, S/formats.py:26-28; @g_mxfp4s_icodes,
// S/gen_mxfp4s.py:1113-1160): a 32-value block's signed codes c = 2 x its E2M1 values (0 1 2 3 4 6 8 12 and their
// negatives; -0 is 0) and d = 2^(e - 128) from its E8M0 byte e (the codes carry the factor 2), so d c is the weight
// exactly. The group's integer dot di = sum c q is exact (eight v_dot4 steps) and adds (d da) di, as the reference's
// one-scale formats do (iq_dot, S/gen_llm.py:1047-1049). Item = blocks 2 p and 2 p + 1 of a row: 32 nibble bytes at
// 32 p of the nibble plane, two E8M0 bytes at 2 p of the scale plane.
__device__ __forceinline__ u32 e2m1x4_codes(u32 nb) {   // four E2M1 codes, one in each byte's low nibble
  const u32 sel = nb & 0x07070707u;
  const u32 pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);   // bytes 0 1 2 3 4 6 8 12
  const u32 neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);   // bytes 0 -1 -2 -3 -4 -6 -8 -12
  const u32 m = ((nb >> 3) & 0x01010101u) * 0xFFu;                        // 0xFF in the bytes with the sign bit
  return (neg & m) | (pos & ~m);
}

__device__ __forceinline__ float e8m0_half(u32 e) {   // 2^(e - 128), exact (a subnormal for e < 2)
  return u32_as_f32(e < 2 ? 0x00200000u << e : (e - 1) << 23);
}

// the exact integer dot of one block's 16 nibble bytes (byte j: values 2 j low, 2 j + 1 high) with 32 codes
__device__ __forceinline__ int e2m1_block_dot(v4u nib, const u32 (&xq)[8]) {
  const u32 b[4] = {nib.x, nib.y, nib.z, nib.w};
  int acc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32 lo = e2m1x4_codes(b[i] & 0x0F0F0F0Fu), hi = e2m1x4_codes((b[i] >> 4) & 0x0F0F0F0Fu);
    acc = sdot4(__builtin_amdgcn_perm(hi, lo, 0x05010400u), xq[2 * i], acc);       // values 8 i .. 8 i + 3
    acc = sdot4(__builtin_amdgcn_perm(hi, lo, 0x07030602u), xq[2 * i + 1], acc);   // values 8 i + 4 .. 8 i + 7
  }
  return acc;
}

struct MX4S8 {
  static constexpr bool kSplit = true;
  struct W { v4u a, b; u32 e; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 64); }
  static __device__ __forceinline__ int64_t group(int item) { return 2 * (int64_t)item; }
  static __device__ __forceinline__ void load_w(const u8 *row, const u8 *srow, int item, bool live, W &w) {
    const v4u z{0u, 0u, 0u, 0u};
    w.a = live ? *reinterpret_cast<const v4u *>(row + 32 * (int64_t)item) : z;
    w.b = live ? *reinterpret_cast<const v4u *>(row + 32 * (int64_t)item + 16) : z;
    w.e = live ? (u32) * reinterpret_cast<const u16 *>(srow + 2 * (int64_t)item) : 0u;
  }
  static __device__ __forceinline__ float dot(const W &w, const XQ &x, int) {
    const int ia = e2m1_block_dot(w.a, x.a), ib = e2m1_block_dot(w.b, x.b);
    return (e8m0_half(w.e & 255u) * x.da) * (float)ia + (e8m0_half(w.e >> 8) * x.db) * (float)ib;
  }
};

// a row's weights of item `item`; split planes also read the row's scale plane srow
template <class P>
__device__ __forceinline__ void load_row(const u8 *row, const u8 *srow, int item, bool live, typename P::W &w) {
  if constexpr (P::kSplit) P::load_w(row, srow, item, live, w);
  else P::load_w(row, item, live, w);
}

constexpr int kWaves = 4;
enum Mode { kPlain = 0, kSwiglu = 1, kPair = 2 };

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// RW rows per wave (4 for one matrix, 2 when two stream), TG tokens per workgroup sharing every weight load
// LPR lanes a row (the item count's power of two, at least 64 / RW), the butterfly restricted to the row's lanes:
// the row sums equal the full-wave butterfly's over one row a pass (the expert matvecs' lane map)
template <class P, int TG, int MODE, int RW, int LPR = 64>
__global__ __launch_bounds__(256) void mv_q8_kernel(int64_t n, int64_t tokens, int64_t k, int accumulate,
                                                    const u8 *__restrict__ codes, const float *__restrict__ meta,
                                                    const u8 *__restrict__ w, const u8 *__restrict__ w2, int64_t rb,
                                                    const u8 *__restrict__ ws, const u8 *__restrict__ ws2, int64_t sb,
                                                    float *__restrict__ y, float *__restrict__ y2) {
  constexpr int NM = MODE == kPlain ? 1 : 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TG;
  const int64_t row0 = ((int64_t)blockIdx.y * kWaves + wave) * RW;
  if (row0 >= n) return;
  const int nitems = P::items(k);
  const int64_t G = k / 32;
  constexpr int GR = 64 / LPR, RL = RW / GR;   // row groups a wave, rows a lane
  static_assert(RL >= 1 && RW % GR == 0, "LPR below 64 / RW");
  const int sub = lane % LPR, rg = lane / LPR;
  float acc[NM][RL][TG];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < RL; ++r)
#pragma unroll
      for (int t = 0; t < TG; ++t) acc[m][r][t] = 0.f;
  for (int it0 = 0; it0 < nitems; it0 += LPR) {
    const int item = it0 + sub;
    const bool live = item < nitems;
    XQ xs[TG];
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      const int64_t tok = t0 + t;
      xq_load(codes + tok * k, meta + 2 * tok * G, P::group(item), live && tok < tokens, xs[t]);
    }
    typename P::W wv[NM][RL];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int r = 0; r < RL; ++r) {
        const int64_t row = row0 + rg + GR * r;
        load_row<P>((m ? w2 : w) + row * rb, (m ? ws2 : ws) + row * sb, item, live && row < n, wv[m][r]);
      }
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int r = 0; r < RL; ++r)
#pragma unroll
        for (int t = 0; t < TG; ++t) acc[m][r][t] += P::dot(wv[m][r], xs[t], item);
  }
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < RL; ++r)
#pragma unroll
      for (int t = 0; t < TG; ++t)
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) acc[m][r][t] += __shfl_xor(acc[m][r][t], off, kWave);
  if (sub == 0) {
#pragma unroll
    for (int r = 0; r < RL; ++r)
#pragma unroll
      for (int t = 0; t < TG; ++t) {
        const int64_t row = row0 + rg + GR * r, tok = t0 + t;
        if (row < n && tok < tokens) {
          float *py = y + tok * n + row;
          const float v = MODE == kSwiglu ? silu_mul(acc[0][r][t], acc[NM - 1][r][t]) : acc[0][r][t];
          *py = accumulate ? *py + v : v;
          if constexpr (MODE == kPair) {
            float *py2 = y2 + tok * n + row;
            *py2 = accumulate ? *py2 + acc[NM - 1][r][t] : acc[NM - 1][r][t];
          }
        }
      }
  }
}

// The decode expert matvecs on Q8_1 activations: one assignment a per workgroup column (blockIdx.x); a wave owns
// 64 / LPR output rows, LPR lanes a row, lane (row rr, sub) taking items sub, sub + LPR, ... of its row; e =
// clamp(ids[a], 0, E - 1) (S/gen_moe.py:592-596). gu: act[a] = act_fn(Wg[e] xq[a / KU], Wu[e] xq[a / KU]) (+ the
// expert biases before the activation); dn: ys[a] = Wd[e] xq[a] (+ bias). xq is the planar Q8_1 buffer of x_rows
// rows (gu: the tokens; dn: the assignments). LPR is the item count rounded up to a power of two (16 to 64), so
// rows with fewer than 64 items (Q4_K K = 768: 12) fill the wave instead of leaving most lanes idle. A row's LPR
// lanes meet in the butterfly of wave_sum restricted to their group (xor LPR / 2 .. 1): with one item a lane up to
// LPR items, the lanes a full-wave butterfly would add past the group hold zeros, so every row's sum is the same
// for every LPR.
template <class P, bool GU, int LPR>
__global__ __launch_bounds__(256) void expert_mv_q8_kernel(int64_t n, int64_t assignments, int KU, int E, int64_t k,
                                                           const int32_t *__restrict__ ids, const u8 *__restrict__ codes,
                                                           const float *__restrict__ meta, const u8 *__restrict__ w,
                                                           const u8 *__restrict__ w2, int64_t rb, int64_t ebytes,
                                                           const u8 *__restrict__ ws, const u8 *__restrict__ ws2,
                                                           int64_t sb, int64_t sebytes, const float *__restrict__ bias,
                                                           const float *__restrict__ bias2, int act,
                                                           float *__restrict__ y) {
  constexpr int RPW = 64 / LPR, NM = GU ? 2 : 1;   // rows a wave, matrices streamed
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rr = lane / LPR;
  const int64_t a = blockIdx.x;
  const int64_t row0 = ((int64_t)blockIdx.y * kWaves + wave) * RPW;
  if (row0 >= n || a >= assignments) return;
  const int64_t row = row0 + rr;
  const bool rlive = row < n;
  int e = ids[a];
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);
  const int64_t xr = GU ? a / KU : a;
  const int64_t G = k / 32;
  const u8 *xc = codes + xr * k;
  const float *xm = meta + 2 * xr * G;
  const u8 *we[NM], *se[NM];
  we[0] = w + e * ebytes;
  se[0] = ws + e * sebytes;   // split planes: the expert's scale rows (unused otherwise)
  if constexpr (GU) {
    we[NM - 1] = w2 + e * ebytes;
    se[NM - 1] = ws2 + e * sebytes;
  }
  const int nitems = P::items(k);
  float acc[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) acc[m] = 0.f;
  for (int it0 = 0; it0 < nitems; it0 += LPR) {
    const int item = it0 + sub;
    const bool live = item < nitems;
    XQ xs;
    xq_load(xc, xm, P::group(item), live, xs);
    typename P::W wv[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) load_row<P>(we[m] + row * rb, se[m] + row * sb, item, live && rlive, wv[m]);
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] += P::dot(wv[m], xs, item);
  }
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off, kWave);
  if (sub == 0 && rlive) {
    float g = acc[0];
    if (bias) g += bias[e * n + row];
    float v = g;
    if constexpr (GU) {
      float u = acc[NM - 1];
      if (bias2) u += bias2[e * n + row];
      v = act_fn(act, g, u);
    }
    y[a * n + row] = v;
  }
}

// ---------------------------------------------------------------- Q4_K K-sliced path (K 4096 / 8192)
// Wave w of a workgroup owns the K-slice [512 KB w, 512 KB (w + 1)) of the workgroup's RW = 16 / KB rows; lane
// (r, it) takes half super-block it of row r inside the slice (five 128-bit loads). The wave quantizes its own
// slice of the activations into its own LDS area, so only a wavefront fence -- no workgroup barrier -- stands
// between the weight loads and the math, and it moves the lane's 128 activation codes into registers before it
// waits for its weights: once they land only ALU work is left. The slices' row sums meet in LDS at the end (one
// barrier, a fixed order).
constexpr int kSWaves = 8;
#ifndef QMM_Q8_SLOTS
#define QMM_Q8_SLOTS 1
#endif
constexpr int kSSlots = QMM_Q8_SLOTS;   // row groups per wave (they share the lane's activations)

template <int TG, int KB, bool STAGEQ>
__global__ __launch_bounds__(kSWaves * 64) void mv_q4k_q8s_kernel(int64_t n, int64_t tokens, int accumulate,
                                                                 const void *__restrict__ x, int bf,
                                                                 const u8 *__restrict__ w, float *__restrict__ y) {
  constexpr int K = KB * 4096, IPR = 4 * KB, RG = 64 / IPR, RW = RG * kSSlots, SLICE = 512 * KB, NG = SLICE / 32;
  constexpr int64_t RB = (int64_t)K / 256 * 144;
  __shared__ __align__(16) u32 xc[kSWaves][TG][SLICE / 4];
  __shared__ __align__(16) float xm[kSWaves][TG][NG][2];
  __shared__ float red[kSWaves][RW][TG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.y * TG;
  const int64_t row0 = (int64_t)blockIdx.x * RW;
  const int r = lane / IPR, it = lane % IPR;
  const int sl = it >> 1, h = it & 1;              // slice-local super-block and half
  const int64_t k0 = (int64_t)wave * SLICE;        // the slice's first value

  // ---- the slice's activations first, then the weights
  float xv[TG][KB][8];
  v2u qv[TG][KB];
  float2 mv[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const int64_t tok = t0 + t < tokens ? t0 + t : tokens - 1;
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int c = lane + 64 * j;               // 8-value chunk of the slice
      if constexpr (STAGEQ) load8_act(x, bf, tok * K + k0 + 8 * c, xv[t][j]);
      else qv[t][j] = *reinterpret_cast<const v2u *>(static_cast<const u8 *>(x) + tok * K + k0 + 8 * c);
    }
    if constexpr (!STAGEQ) {
      const float2 *meta = reinterpret_cast<const float2 *>(static_cast<const u8 *>(x) + tokens * K);
      mv[t] = meta[tok * (K / 32) + k0 / 32 + (lane < NG ? lane : 0)];
    }
  }
  v4u wd[kSSlots][5];
#pragma unroll
  for (int so = 0; so < kSSlots; ++so) {
    int64_t row = row0 + r + RG * so;
    row = row < n ? row : n - 1;        // rows past n read row n-1 and are never stored
    const v4u *bp = reinterpret_cast<const v4u *>(w + row * RB + (k0 / 256 + sl) * 144);
    wd[so][0] = bp[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) wd[so][1 + i] = bp[1 + 4 * h + i];
  }

  // ---- the wave's slice: codes and group pairs into its own LDS area
#pragma unroll
  for (int t = 0; t < TG; ++t) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int c = lane + 64 * j;
      if constexpr (STAGEQ) {
        u32 c0, c1;
        float d16, sum;
        q8_group4(xv[t][j], c0, c1, d16, sum);
        xc[wave][t][2 * c] = c0;
        xc[wave][t][2 * c + 1] = c1;
        if ((c & 3) == 0) { xm[wave][t][c >> 2][0] = d16; xm[wave][t][c >> 2][1] = sum; }
      } else {
        xc[wave][t][2 * c] = qv[t][j].x;
        xc[wave][t][2 * c + 1] = qv[t][j].y;
      }
    }
    if constexpr (!STAGEQ) {
      if (lane < NG) { xm[wave][t][lane][0] = mv[t].x; xm[wave][t][lane][1] = mv[t].y; }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- the lane's 4 groups (8 sl + 4 h + 0..3): codes and pairs into registers before the weights are awaited
  const int g0 = 8 * sl + 4 * h;
  u32 xa[TG][4][8];
  float md[TG][4], ms[TG][4];
#pragma unroll
  for (int t = 0; t < TG; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v4u p0 = *reinterpret_cast<const v4u *>(&xc[wave][t][8 * (g0 + g)]);
      const v4u p1 = *reinterpret_cast<const v4u *>(&xc[wave][t][8 * (g0 + g) + 4]);
      xa[t][g][0] = p0.x; xa[t][g][1] = p0.y; xa[t][g][2] = p0.z; xa[t][g][3] = p0.w;
      xa[t][g][4] = p1.x; xa[t][g][5] = p1.y; xa[t][g][6] = p1.z; xa[t][g][7] = p1.w;
      md[t][g] = xm[wave][t][g0 + g][0];
      ms[t][g] = xm[wave][t][g0 + g][1];
    }
#pragma unroll
  for (int t = 0; t < TG; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) asm volatile("" ::"v"(xa[t][g][i]));
      asm volatile("" ::"v"(md[t][g]), "v"(ms[t][g]));
    }

  // ---- math: pages 2h (groups g0, g0 + 1) and 2h + 1 (groups g0 + 2, g0 + 3)
#pragma unroll
  for (int so = 0; so < kSSlots; ++so) {
  const v4u hd = wd[so][0];
  const float d = f16_to_f32(hd.x), dmin = f16_to_f32(hd.x >> 16);
  const u32 q[16] = {wd[so][1].x, wd[so][1].y, wd[so][1].z, wd[so][1].w, wd[so][2].x, wd[so][2].y, wd[so][2].z,
                     wd[so][2].w, wd[so][3].x, wd[so][3].y, wd[so][3].z, wd[so][3].w, wd[so][4].x, wd[so][4].y,
                     wd[so][4].z, wd[so][4].w};
  float sc[4], mn[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    u32 s_, m_;
    q4k_scale_min(hd.y, hd.z, hd.w, 4 * h + g, s_, m_);
    sc[g] = d * (float)s_;
    mn[g] = dmin * (float)m_;
  }
  float part[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    float p = 0.f;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      int ia = 0, ib = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32 Q = q[8 * pg + i];
        ia = sdot4(Q & 0x0F0F0F0Fu, xa[t][2 * pg][i], ia);
        ib = sdot4((Q >> 4) & 0x0F0F0F0Fu, xa[t][2 * pg + 1][i], ib);
      }
      p += ((float)ia * sc[2 * pg] - ms[t][2 * pg] * mn[2 * pg]) * md[t][2 * pg];
      p += ((float)ib * sc[2 * pg + 1] - ms[t][2 * pg + 1] * mn[2 * pg + 1]) * md[t][2 * pg + 1];
    }
    // the row's IPR lanes of this slice: a butterfly leaves the slice sum in every one of them
    p += xshfl<1>(p);
    p += xshfl<2>(p);
    if constexpr (IPR == 8) p += xshfl<4>(p);
    part[t] = p;
  }
  if (it == 0) {
#pragma unroll
    for (int t = 0; t < TG; ++t) red[wave][r + RG * so][t] = part[t];
  }
  }
  __syncthreads();
  if (tid < RW * TG) {
    const int rr = tid / TG, t = tid % TG;
    float tot = 0.f;
#pragma unroll
    for (int wv = 0; wv < kSWaves; ++wv) tot += red[wv][rr][t];
    const int64_t row = row0 + rr, tok = t0 + t;
    if (row < n && tok < tokens) {
      float *py = y + tok * n + row;
      *py = accumulate ? *py + tot : tot;
    }
  }
}

template <int TG, int KB, bool STAGEQ>
int launch_sliced(int64_t n, int64_t tokens, int accumulate, const void *x, int bf, const void *w, float *y,
                  hipStream_t s) {
  constexpr int RW = 16 / KB * kSSlots;
  const dim3 grid((unsigned)((n + RW - 1) / RW), (unsigned)((tokens + TG - 1) / TG));
  mv_q4k_q8s_kernel<TG, KB, STAGEQ><<<grid, kSWaves * 64, 0, s>>>(n, tokens, accumulate, x, bf,
                                                                  static_cast<const u8 *>(w), y);
  return launch_status();
}

template <int KB, bool STAGEQ>
int launch_fast_tg(int64_t n, int64_t tokens, int accumulate, const void *x, int bf, const void *w, float *y,
                   hipStream_t s) {
  return tokens >= 2 ? launch_sliced<2, KB, STAGEQ>(n, tokens, accumulate, x, bf, w, y, s)
                     : launch_sliced<1, KB, STAGEQ>(n, tokens, accumulate, x, bf, w, y, s);
}

}  // namespace

extern "C" int qmm_quant_q8(int64_t rows, int64_t k, const void *x, int x_dtype, void *xq, qmm_stream_t stream) {
  if (!x || !xq) return QMM_ERR_NULL;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (rows <= 0 || k <= 0 || k % 32 || rows > (1ll << 24)) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(xq, 16)) return QMM_ERR_ALIGN;
  const int64_t chunks = rows * (k / 8);
  quant_q8_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      rows, k, x, x_dtype == QMM_BF16, static_cast<u8 *>(xq));
  return launch_status();
}

int qmm_mv_q4kt_q8(int fmt, int mode, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                   int x_dtype, const void *w, const void *w2, float *y, float *y2, hipStream_t s);

namespace {
// the generic (GGUF-layout, planar Q8_1) matvec of one format in one mode
template <class P, int MODE>
int launch_generic(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w, const void *w2,
                   int64_t rb, float *y, float *y2, hipStream_t s, const void *ws = nullptr,
                   const void *ws2 = nullptr) {
  constexpr int TG = 2, RW = MODE == kPlain ? 4 : 2;
  const u8 *codes = static_cast<const u8 *>(x);
  const float *meta = reinterpret_cast<const float *>(codes + tokens * k);
  const dim3 grid((unsigned)((tokens + TG - 1) / TG), (unsigned)((n + kWaves * RW - 1) / (kWaves * RW)));
  if (grid.x > 2147483647u || grid.y > 65535u) return QMM_ERR_SHAPE;
  const int items = P::items(k);
  int lpr = items <= 16 ? 16 : (items <= 32 ? 32 : 64);   // lanes a row, at least 64 / RW
  lpr = lpr < 64 / RW ? 64 / RW : lpr;
  auto go = [&](auto lc) {
    mv_q8_kernel<P, TG, MODE, RW, decltype(lc)::value><<<grid, 256, 0, s>>>(
        n, tokens, k, accumulate, codes, meta, static_cast<const u8 *>(w), static_cast<const u8 *>(w2), rb,
        static_cast<const u8 *>(ws), static_cast<const u8 *>(ws2), k / 32, y, y2);
    return launch_status();
  };
  if constexpr (RW >= 4) { if (lpr == 16) return go(std::integral_constant<int, 16>{}); }
  if (lpr == 32) return go(std::integral_constant<int, 32>{});
  return go(std::integral_constant<int, 64>{});
}

template <int MODE>
int generic_fmt(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w,
                const void *w2, float *y, float *y2, hipStream_t s) {
  const int64_t rb = row_bytes(fmt, k);
  if (fmt == QMM_Q4_K) return launch_generic<Q4K8, MODE>(k, n, tokens, accumulate, x, w, w2, rb, y, y2, s);
  if (fmt == QMM_Q6_K) return launch_generic<Q6K8, MODE>(k, n, tokens, accumulate, x, w, w2, rb, y, y2, s);
  return launch_generic<Q408, MODE>(k, n, tokens, accumulate, x, w, w2, rb, y, y2, s);
}

// checks shared by the int8 matvec entry points: formats with integer codes (GGUF Q4_K / Q4_0 / Q6_K, tiled Q4_K / Q4_0)
int check_q8(int fmt, int64_t k, int64_t n, int64_t tokens, const void *x, int x_dtype, const void *w, const float *y) {
  if (!x || !w || !y) return QMM_ERR_NULL;
  if (fmt != QMM_Q4_K && fmt != QMM_Q4_0 && fmt != QMM_Q4_KT && fmt != QMM_Q6_K && fmt != QMM_Q4_0T)
    return QMM_ERR_FORMAT;
  if (x_dtype != QMM_Q8 && x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (k <= 0 || n <= 0 || tokens <= 0 || n > (1ll << 30) || tokens > (1ll << 24) || k > (1ll << 20))
    return QMM_ERR_SHAPE;
  if ((fmt == QMM_Q4_K || fmt == QMM_Q6_K) && k % 256) return QMM_ERR_SHAPE;
  if (fmt == QMM_Q4_0 && k % 64) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, fmt == QMM_Q6_K ? 4 : 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  return QMM_OK;
}
}  // namespace

extern "C" int qmm_mv_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                         const void *w, float *y, qmm_stream_t stream) {
  if (int st = check_q8(fmt, k, n, tokens, x, x_dtype, w, y)) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (fmt == QMM_Q4_KT || fmt == QMM_Q4_0T)
    return qmm_mv_q4kt_q8(fmt, kPlain, k, n, tokens, accumulate, x, x_dtype, w, nullptr, y, nullptr, s);
  const bool fast = fmt == QMM_Q4_K && (k == 4096 || k == 8192) && tokens <= 65535ll * 2;
  if (x_dtype != QMM_Q8) {
    // f32 / bf16 rows are quantized while staged; only the fast path stages (others take planar Q8 from
    // qmm_quant_q8)
    if (!fast) return QMM_ERR_SHAPE;
    const int bf = x_dtype == QMM_BF16;
    return k == 4096 ? launch_fast_tg<1, true>(n, tokens, accumulate, x, bf, w, y, s)
                     : launch_fast_tg<2, true>(n, tokens, accumulate, x, bf, w, y, s);
  }
  if (fast)
    return k == 4096 ? launch_fast_tg<1, false>(n, tokens, accumulate, x, 0, w, y, s)
                     : launch_fast_tg<2, false>(n, tokens, accumulate, x, 0, w, y, s);
  return generic_fmt<kPlain>(fmt, k, n, tokens, accumulate, x, w, nullptr, y, nullptr, s);
}

// The two-matrix int8 matvecs (mode kSwiglu / kPair): the tiled kernel takes planar Q8_1 or f32 / bf16 rows, the
// GGUF layouts planar Q8_1.
static int mv2_q8(int mode, int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                  const void *w, const void *w2, float *y, float *y2, qmm_stream_t stream) {
  if (int st = check_q8(fmt, k, n, tokens, x, x_dtype, w, y)) return st;
  if (!w2 || (mode == kPair && !y2)) return QMM_ERR_NULL;
  if (!aligned(w2, fmt == QMM_Q6_K ? 4 : 16) || (y2 && !aligned(y2, 4))) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (fmt == QMM_Q4_KT || fmt == QMM_Q4_0T)
    return qmm_mv_q4kt_q8(fmt, mode, k, n, tokens, accumulate, x, x_dtype, w, w2, y, y2, s);
  if (x_dtype != QMM_Q8) return QMM_ERR_DTYPE;   // GGUF layouts: the planar Q8_1 buffer of qmm_quant_q8
  return mode == kSwiglu ? generic_fmt<kSwiglu>(fmt, k, n, tokens, accumulate, x, w, w2, y, nullptr, s)
                         : generic_fmt<kPair>(fmt, k, n, tokens, accumulate, x, w, w2, y, y2, s);
}

extern "C" int qmm_mv_swiglu_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                                int x_dtype, const void *w, const void *w2, float *y, qmm_stream_t stream) {
  return mv2_q8(kSwiglu, fmt, k, n, tokens, accumulate, x, x_dtype, w, w2, y, nullptr, stream);
}

extern "C" int qmm_mv_pair_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                              int x_dtype, const void *w, const void *w2, float *y, float *y2, qmm_stream_t stream) {
  return mv2_q8(kPair, fmt, k, n, tokens, accumulate, x, x_dtype, w, w2, y, y2, stream);
}

namespace {
template <class P>
int launch_expert_q8(bool gu, int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids,
                     const void *x, const void *w, const void *w2, int64_t rb, int64_t ebytes, const float *bias,
                     const float *bias2, int act, float *y, hipStream_t s, const void *ws = nullptr,
                     const void *ws2 = nullptr, int64_t sebytes = 0) {
  const u8 *s1 = static_cast<const u8 *>(ws), *s2 = static_cast<const u8 *>(ws2);
  const int64_t x_rows = gu ? assignments / KU : assignments;
  const u8 *codes = static_cast<const u8 *>(x);
  const float *meta = reinterpret_cast<const float *>(codes + x_rows * k);
  const int items = P::items(k);
  const int lpr = items <= 16 ? 16 : (items <= 32 ? 32 : 64);   // lanes a row: the item count's power of two
  const int64_t rows_wg = kWaves * (64 / lpr);
  const dim3 grid((unsigned)assignments, (unsigned)((n + rows_wg - 1) / rows_wg));
  if (grid.y > 65535u) return QMM_ERR_SHAPE;
  auto go = [&](auto lc) {
    constexpr int L = decltype(lc)::value;
    if (gu)
      expert_mv_q8_kernel<P, true, L><<<grid, 256, 0, s>>>(n, assignments, KU, E, k, ids, codes, meta,
                                                           static_cast<const u8 *>(w), static_cast<const u8 *>(w2),
                                                           rb, ebytes, s1, s2, k / 32, sebytes, bias, bias2, act, y);
    else
      expert_mv_q8_kernel<P, false, L><<<grid, 256, 0, s>>>(n, assignments, KU, E, k, ids, codes, meta,
                                                            static_cast<const u8 *>(w), nullptr, rb, ebytes, s1,
                                                            nullptr, k / 32, sebytes, bias, nullptr, act, y);
  };
  if (lpr == 16) go(std::integral_constant<int, 16>{});
  else if (lpr == 32) go(std::integral_constant<int, 32>{});
  else go(std::integral_constant<int, 64>{});
  return launch_status();
}
}  // namespace

extern "C" int qmm_moe_expert_mv_q8(int fmt, int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                    int64_t assignments, const int32_t *ids, const void *x, const void *w,
                                    const void *w2, const float *bias, const float *bias2, float *y,
                                    qmm_stream_t stream) {
  if (fmt != QMM_Q4_K && fmt != QMM_Q4_0 && fmt != QMM_Q6_K) return QMM_ERR_FORMAT;
  if (mode != 0 && mode != 1) return QMM_ERR_RANGE;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!ids || !x || !w || !y) return QMM_ERR_NULL;
  const bool gu = mode == 0;
  if (gu && !fused && !w2) return QMM_ERR_NULL;
  const int64_t rb = row_bytes(fmt, k);
  if (n <= 0 || assignments <= 0 || assignments > (1 << 24) || rb == 0 || n > (1 << 24)) return QMM_ERR_SHAPE;
  if (fmt == QMM_Q4_0 && k % 64) return QMM_ERR_SHAPE;
  if (gu && assignments % KU) return QMM_ERR_SHAPE;
  const int wal = fmt == QMM_Q4_K ? 16 : 4;
  if (!aligned(x, 16) || !aligned(w, wal) || (w2 && !aligned(w2, wal)) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  if (!aligned(bias, 4) || !aligned(bias2, 4)) return QMM_ERR_ALIGN;
  // a fused [E, 2n, k] gate_up tensor: expert e's n gate rows, then its n up rows (S/gen_moe.py:538)
  const int64_t ebytes = rb * n * (gu && fused ? 2 : 1);
  const void *wu = gu && fused ? static_cast<const void *>(static_cast<const u8 *>(w) + rb * n) : w2;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (fmt == QMM_Q4_K)
    return launch_expert_q8<Q4K8>(gu, k, n, E, KU, assignments, ids, x, w, wu, rb, ebytes, bias, bias2, act, y, s);
  if (fmt == QMM_Q6_K)
    return launch_expert_q8<Q6K8>(gu, k, n, E, KU, assignments, ids, x, w, wu, rb, ebytes, bias, bias2, act, y, s);
  return launch_expert_q8<Q408>(gu, k, n, E, KU, assignments, ids, x, w, wu, rb, ebytes, bias, bias2, act, y, s);
}

// The opt-in int8 decode of MXFP4 split planes (MXFP4S_Q8, S/formats.py:26-28): g_mv_mxfp4s_k{K}[_swiglu|_pair]
// [_t{TG}]_q8 (S/gen_llm.py:1288-1301 with @g_mxfp4s_icodes, S/gen_mxfp4s.py:1113-1160) and the MOE_Q8 expert
// matvecs of mxfp4s experts (S/gen_moe.py:535-727), over the generic item walk (MX4S8).
extern "C" int qmm_mv_mxfp4s_q8(int mode, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                                int x_dtype, const void *w, const void *ws, const void *w2, const void *ws2, float *y,
                                float *y2, qmm_stream_t stream) {
  if (mode != kPlain && mode != kSwiglu && mode != kPair) return QMM_ERR_RANGE;
  if (!x || !w || !ws || !y) return QMM_ERR_NULL;
  if (mode != kPlain && (!w2 || !ws2)) return QMM_ERR_NULL;
  if (mode == kPair && !y2) return QMM_ERR_NULL;
  if (x_dtype != QMM_Q8) return QMM_ERR_DTYPE;   // the planar Q8_1 buffer of qmm_quant_q8
  if (k <= 0 || n <= 0 || tokens <= 0 || k % 64 || n > (1ll << 30) || tokens > (1ll << 24) || k > (1ll << 20))
    return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(ws, 2) || (w2 && !aligned(w2, 16)) || (ws2 && !aligned(ws2, 2)) ||
      !aligned(y, 4) || (y2 && !aligned(y2, 4)))
    return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t rb = k / 2;
  if (mode == kSwiglu) return launch_generic<MX4S8, kSwiglu>(k, n, tokens, accumulate, x, w, w2, rb, y, nullptr, s, ws, ws2);
  if (mode == kPair) return launch_generic<MX4S8, kPair>(k, n, tokens, accumulate, x, w, w2, rb, y, y2, s, ws, ws2);
  return launch_generic<MX4S8, kPlain>(k, n, tokens, accumulate, x, w, nullptr, rb, y, nullptr, s, ws, nullptr);
}

extern "C" int qmm_moe_expert_mv_mxfp4s_q8(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                           int64_t assignments, const int32_t *ids, const void *x, const void *w,
                                           const void *ws, const void *w2, const void *ws2, const float *bias,
                                           const float *bias2, float *y, qmm_stream_t stream) {
  if (mode != 0 && mode != 1) return QMM_ERR_RANGE;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!ids || !x || !w || !ws || !y) return QMM_ERR_NULL;
  const bool gu = mode == 0;
  if (gu && !fused && (!w2 || !ws2)) return QMM_ERR_NULL;
  if (k <= 0 || k % 64 || n <= 0 || assignments <= 0 || assignments > (1 << 24) || n > (1 << 24) || k > (1 << 20))
    return QMM_ERR_SHAPE;
  if (gu && assignments % KU) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(ws, 2) || (w2 && !aligned(w2, 16)) || (ws2 && !aligned(ws2, 2)) ||
      !aligned(y, 4) || !aligned(bias, 4) || !aligned(bias2, 4))
    return QMM_ERR_ALIGN;
  // a fused [E, 2n, k] gate_up tensor (both planes): expert e's n gate rows, then its n up rows
  const int64_t rb = k / 2, sb = k / 32;
  const int64_t ebytes = rb * n * (gu && fused ? 2 : 1), sebytes = sb * n * (gu && fused ? 2 : 1);
  const void *wu = gu && fused ? static_cast<const void *>(static_cast<const u8 *>(w) + rb * n) : w2;
  const void *wsu = gu && fused ? static_cast<const void *>(static_cast<const u8 *>(ws) + sb * n) : ws2;
  return launch_expert_q8<MX4S8>(gu, k, n, E, KU, assignments, ids, x, w, wu, rb, ebytes, bias, bias2, act, y,
                                 reinterpret_cast<hipStream_t>(stream), ws, wsu, sebytes);
}
