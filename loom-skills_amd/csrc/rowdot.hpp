// Per-format lane math of the decode matvecs: a weight row is split into "items" (one per lane and pass),
// each item carries its own scales so a lane's partial dot product needs no other lane. The dense GEMV
// (S/gen_llm.py:1159-1378) and the MoE expert matvecs (S/gen_moe.py:535-727) are both built on these.
//
//   format  item                                   bytes per item      values per item
//   Q4_K    (super-block b, page j): header+page   16 + 32 (3 x b128)  64 (sub-blocks 2j, 2j+1)
//   Q4_0    pair of blocks (36 B, 9 dwords)        36                  64
//   MXFP4   one 17-byte GGUF block                 17 (byte loads)     32
//   MXFP4S  one 16-byte nibble chunk + scale byte  16 + 1              32
//   Q6_K    (super-block b, half, jh): groups      64 ql + 32 qh + 4   64 (groups 4 half + 2 jh, + 1)
//           4 half + 2 jh and + 1 of the block     scale bytes + d
//
// bf16 activations: 4-bit codes become bf16 (128 + q) with one or into the exponent field and v_dot2_f32_bf16
// multiplies two codes with two activations per lane op; the +128 is removed with the item's sum of x.
// E2M1 codes are converted with v_cvt_scalef32_pk_bf16_fp4 (scale 1: exact), and the E8M0 block scale is applied
// to the f32 partial. f32 activations use f32 FMAs.
#pragma once
#include "common.hpp"

namespace qmm {

constexpr u32 kNib2 = 0x000F000Fu;
constexpr u32 kBf16_128 = 0x43004300u;   // bf16(128) in both halves

__device__ __forceinline__ u32 pair02(u32 d0, u32 d1) { return __builtin_amdgcn_perm(d1, d0, 0x05040100u); }
__device__ __forceinline__ u32 pair13(u32 d0, u32 d1) { return __builtin_amdgcn_perm(d1, d0, 0x07060302u); }

__device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

__device__ __forceinline__ void load16(const void *p, bool live, u32 (&d)[4]) {
  const uint4 v = live ? *reinterpret_cast<const uint4 *>(p) : make_uint4(0, 0, 0, 0);
  d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
}

// ------------------------------------------------------------------------------------ activation fragments
// bf16 halves A and B of NDW code dwords each: pairs (x[4i], x[4i+2]) and (x[4i+1], x[4i+3]) per dword i.
template <int NDW>
struct XB {
  u32 a02[NDW], a13[NDW], b02[NDW], b13[NDW];
  float sa, sb;
};

// d: 2*NDW dwords of half A then 2*NDW dwords of half B (bf16 pairs in element order).
template <int NDW>
__device__ __forceinline__ void xb_from_dwords(const u32 *d, XB<NDW> &x) {
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const u32 a0 = d[2 * i], a1 = d[2 * i + 1], b0 = d[2 * NDW + 2 * i], b1 = d[2 * NDW + 2 * i + 1];
    x.a02[i] = pair02(a0, a1);
    x.a13[i] = pair13(a0, a1);
    x.b02[i] = pair02(b0, b1);
    x.b13[i] = pair13(b0, b1);
    sa += (bf16_to_f32(a0 & 0xFFFFu) + bf16_to_f32(a0 >> 16)) + (bf16_to_f32(a1 & 0xFFFFu) + bf16_to_f32(a1 >> 16));
    sb += (bf16_to_f32(b0 & 0xFFFFu) + bf16_to_f32(b0 >> 16)) + (bf16_to_f32(b1 & 0xFFFFu) + bf16_to_f32(b1 >> 16));
  }
  x.sa = sa;
  x.sb = sb;
}

// P_A = sum (128 + low nibble) x_A, P_B = sum (128 + high nibble) x_B over NDW code dwords.
template <int NDW>
__device__ __forceinline__ void nib_dot_bf16(const u32 *q, const XB<NDW> &x, float &pa, float &pb) {
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const u32 Q = q[i];
    a0 = dot2((Q & kNib2) | kBf16_128, x.a02[i], a0);
    a1 = dot2(((Q >> 8) & kNib2) | kBf16_128, x.a13[i], a1);
    b0 = dot2(((Q >> 4) & kNib2) | kBf16_128, x.b02[i], b0);
    b1 = dot2(((Q >> 12) & kNib2) | kBf16_128, x.b13[i], b1);
  }
  pa = a0 + a1;
  pb = b0 + b1;
}

template <int NDW>
struct XF {
  float a[4 * NDW], b[4 * NDW];
  float sa, sb;
};

template <int NDW>
__device__ __forceinline__ void xf_load(const float *p, bool live, XF<NDW> &x) {
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const float4 va = live ? reinterpret_cast<const float4 *>(p)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 vb = live ? reinterpret_cast<const float4 *>(p)[NDW + i] : make_float4(0.f, 0.f, 0.f, 0.f);
    x.a[4 * i] = va.x; x.a[4 * i + 1] = va.y; x.a[4 * i + 2] = va.z; x.a[4 * i + 3] = va.w;
    x.b[4 * i] = vb.x; x.b[4 * i + 1] = vb.y; x.b[4 * i + 2] = vb.z; x.b[4 * i + 3] = vb.w;
    sa += (va.x + va.y) + (va.z + va.w);
    sb += (vb.x + vb.y) + (vb.z + vb.w);
  }
  x.sa = sa;
  x.sb = sb;
}

template <int NDW>
__device__ __forceinline__ void nib_dot_f32(const u32 *q, const XF<NDW> &x, float &pa, float &pb) {
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const u32 Q = q[i];
    const u32 lo = Q & 0x0F0F0F0Fu, hi = (Q >> 4) & 0x0F0F0F0Fu;
    a0 = __builtin_fmaf((float)(lo & 0xFFu), x.a[4 * i + 0], a0);
    a1 = __builtin_fmaf((float)((lo >> 8) & 0xFFu), x.a[4 * i + 1], a1);
    a0 = __builtin_fmaf((float)((lo >> 16) & 0xFFu), x.a[4 * i + 2], a0);
    a1 = __builtin_fmaf((float)(lo >> 24), x.a[4 * i + 3], a1);
    b0 = __builtin_fmaf((float)(hi & 0xFFu), x.b[4 * i + 0], b0);
    b1 = __builtin_fmaf((float)((hi >> 8) & 0xFFu), x.b[4 * i + 1], b1);
    b0 = __builtin_fmaf((float)((hi >> 16) & 0xFFu), x.b[4 * i + 2], b0);
    b1 = __builtin_fmaf((float)(hi >> 24), x.b[4 * i + 3], b1);
  }
  pa = a0 + a1;
  pb = b0 + b1;
}

template <int NDW>
__device__ __forceinline__ void xb_load(const u16 *p, bool live, XB<NDW> &x) {
  u32 d[4 * NDW];
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    u32 v[4];
    load16(p + 8 * i, live, v);
    d[4 * i] = v[0]; d[4 * i + 1] = v[1]; d[4 * i + 2] = v[2]; d[4 * i + 3] = v[3];
  }
  xb_from_dwords<NDW>(d, x);
}

// ------------------------------------------------------------------------------------------------- Q4_K
// item = 4 * block + page; values of the item: sub-block 2j = x[256b + 64j .. +32), 2j+1 = the next 32.
template <bool BF16X>
struct Q4K {
  static constexpr int kValues = 64;
  using X = typename std::conditional<BF16X, XB<8>, XF<8>>::type;
  struct W { u32 h[4], q[8]; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 256) * 4; }
  static __device__ __forceinline__ void load_x(const void *xrow, int item, bool live, X &x) {
    const int64_t off = (int64_t)(item >> 2) * 256 + 64 * (item & 3);
    if constexpr (BF16X) xb_load<8>(static_cast<const u16 *>(xrow) + off, live, x);
    else xf_load<8>(static_cast<const float *>(xrow) + off, live, x);
  }
  static __device__ __forceinline__ void load_w(const u8 *row, const u8 *, int item, bool live, W &w) {
    const u8 *b = row + (int64_t)(item >> 2) * 144;
    const int j = item & 3;
    load16(b, live, w.h);
    u32 a[4], c[4];
    load16(b + 16 + 32 * j, live, a);
    load16(b + 32 + 32 * j, live, c);
#pragma unroll
    for (int i = 0; i < 4; ++i) { w.q[i] = a[i]; w.q[4 + i] = c[i]; }
  }
  static __device__ __forceinline__ float dot(const W &w, const X &x, int item) {
    const int j = item & 3;
    u32 sc0, m0, sc1, m1;
    q4k_scale_min(w.h[1], w.h[2], w.h[3], 2 * j, sc0, m0);
    q4k_scale_min(w.h[1], w.h[2], w.h[3], 2 * j + 1, sc1, m1);
    const float d = f16_to_f32(w.h[0]), dmin = f16_to_f32(w.h[0] >> 16);
    const float dsc0 = d * (float)sc0, dsc1 = d * (float)sc1;
    float ma = dmin * (float)m0, mb = dmin * (float)m1;
    float pa, pb;
    if constexpr (BF16X) {
      nib_dot_bf16<8>(w.q, x, pa, pb);
      ma = __builtin_fmaf(128.f, dsc0, ma);
      mb = __builtin_fmaf(128.f, dsc1, mb);
    } else {
      nib_dot_f32<8>(w.q, x, pa, pb);
    }
    return __builtin_fmaf(dsc0, pa, dsc1 * pb) - __builtin_fmaf(ma, x.sa, mb * x.sb);
  }
};

// ------------------------------------------------------------------------------------------------- Q4_0
// item = pair of blocks p: 36 bytes at 36p of the row (4-byte aligned when K % 64 == 0), x[64p .. 64p+64).
template <bool BF16X>
struct Q40 {
  static constexpr int kValues = 64;
  using XH = typename std::conditional<BF16X, XB<4>, XF<4>>::type;
  struct X { XH blk[2]; };
  struct W { u32 v[9]; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 64); }
  static __device__ __forceinline__ void load_x(const void *xrow, int item, bool live, X &x) {
    const int64_t off = (int64_t)item * 64;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      if constexpr (BF16X) xb_load<4>(static_cast<const u16 *>(xrow) + off + 32 * blk, live, x.blk[blk]);
      else xf_load<4>(static_cast<const float *>(xrow) + off + 32 * blk, live, x.blk[blk]);
    }
  }
  static __device__ __forceinline__ void load_w(const u8 *row, const u8 *, int item, bool live, W &w) {
    const u32 *p = reinterpret_cast<const u32 *>(row + (int64_t)item * 36);
#pragma unroll
    for (int i = 0; i < 9; ++i) w.v[i] = live ? p[i] : 0u;
  }
  static __device__ __forceinline__ float dot(const W &w, const X &x, int) {
    const float d[2] = {f16_to_f32(w.v[0]), f16_to_f32(w.v[4] >> 16)};
    const u32 q0[4] = {__builtin_amdgcn_alignbit(w.v[1], w.v[0], 16), __builtin_amdgcn_alignbit(w.v[2], w.v[1], 16),
                       __builtin_amdgcn_alignbit(w.v[3], w.v[2], 16), __builtin_amdgcn_alignbit(w.v[4], w.v[3], 16)};
    const u32 q1[4] = {w.v[5], w.v[6], w.v[7], w.v[8]};
    float pa0, pb0, pa1, pb1;
    float bias;
    if constexpr (BF16X) {
      nib_dot_bf16<4>(q0, x.blk[0], pa0, pb0);
      nib_dot_bf16<4>(q1, x.blk[1], pa1, pb1);
      bias = 136.f;   // value d (q - 8); the codes carry +128
    } else {
      nib_dot_f32<4>(q0, x.blk[0], pa0, pb0);
      nib_dot_f32<4>(q1, x.blk[1], pa1, pb1);
      bias = 8.f;
    }
    const float s0 = x.blk[0].sa + x.blk[0].sb, s1 = x.blk[1].sa + x.blk[1].sb;
    return __builtin_fmaf(d[0], (pa0 + pb0) - bias * s0, d[1] * ((pa1 + pb1) - bias * s1));
  }
};

// ------------------------------------------------------------------------------------------------ MXFP4
// item = one 32-value block. GGUF (SPLIT = false): 17-byte blocks, e then codes in split16 order (value j < 16:
// low nibble of code byte j, j >= 16: high nibble of byte j - 16). Split planes (SPLIT = true): 16 code bytes
// in pairs order (byte j: values 2j, 2j+1) at 16b of the row, E8M0 byte b of the scale row.
// The x fragment holds, for code byte j, the activation pair its two nibbles multiply.
template <bool BF16X, bool SPLIT>
struct MXFP4 {
  static constexpr int kValues = 32;
  struct XBm { u32 p[16]; };
  struct XFm { float lo[16], hi[16]; };
  using X = typename std::conditional<BF16X, XBm, XFm>::type;
  struct W { u32 q[4]; u32 e; };
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 32); }
  static __device__ __forceinline__ void load_x(const void *xrow, int item, bool live, X &x) {
    const int64_t off = (int64_t)item * 32;
    if constexpr (BF16X) {
      u32 d[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32 v[4];
        load16(static_cast<const u16 *>(xrow) + off + 8 * i, live, v);
        d[4 * i] = v[0]; d[4 * i + 1] = v[1]; d[4 * i + 2] = v[2]; d[4 * i + 3] = v[3];
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if constexpr (SPLIT) x.p[j] = d[j];   // (x[2j], x[2j+1])
        else x.p[j] = (j & 1) ? pair13(d[j >> 1], d[8 + (j >> 1)]) : pair02(d[j >> 1], d[8 + (j >> 1)]);  // (x[j], x[j+16])
      }
    } else {
      float v[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 f = live ? reinterpret_cast<const float4 *>(static_cast<const float *>(xrow) + off)[i]
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        x.lo[j] = SPLIT ? v[2 * j] : v[j];
        x.hi[j] = SPLIT ? v[2 * j + 1] : v[j + 16];
      }
    }
  }
  static __device__ __forceinline__ void load_w(const u8 *row, const u8 *srow, int item, bool live, W &w) {
    if constexpr (SPLIT) {
      load16(row + (int64_t)item * 16, live, w.q);
      w.e = live ? srow[item] : 127u;
    } else {
      const u8 *b = row + (int64_t)item * 17;
      w.e = live ? b[0] : 127u;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w.q[i] = live ? ((u32)b[1 + 4 * i] | ((u32)b[2 + 4 * i] << 8) | ((u32)b[3 + 4 * i] << 16) | ((u32)b[4 + 4 * i] << 24)) : 0u;
    }
  }
  template <int SEL>
  static __device__ __forceinline__ void byte_dot(u32 dw, const X &x, int j, float &p) {
    if constexpr (BF16X) {
      const bf16x2 v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(dw, 1.0f, SEL);
      p = __builtin_amdgcn_fdot2_f32_bf16(v, __builtin_bit_cast(bf16x2, x.p[j]), p, false);
    } else {
      typedef __attribute__((ext_vector_type(2))) float f32x2;
      const f32x2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(dw, 1.0f, SEL);
      p = __builtin_fmaf(v.y, x.hi[j], __builtin_fmaf(v.x, x.lo[j], p));
    }
  }
  static __device__ __forceinline__ float dot(const W &w, const X &x, int) {
    float p0 = 0.f, p1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      byte_dot<0>(w.q[i], x, 4 * i + 0, p0);
      byte_dot<1>(w.q[i], x, 4 * i + 1, p1);
      byte_dot<2>(w.q[i], x, 4 * i + 2, p0);
      byte_dot<3>(w.q[i], x, 4 * i + 3, p1);
    }
    return (p0 + p1) * e8m0_scale(w.e);
  }
};

// ------------------------------------------------------------------------------------------------- Q6_K
// item = 4 b + 2 half + jh: groups j = 2 jh and 2 jh + 1 of half `half` of super-block b, the 64 values
// 256 b + 128 half + 64 jh .. + 64. Group j's code l: ((ql[64 half + 32 (j % 2) + l] >> 4 (j / 2)) & 15) |
// (((qh[32 half + l] >> 2 j) & 3) << 4); so the item needs the half's 64 ql bytes (nibble jh), its 32 qh bytes
// (fields 2 jh, 2 jh + 1), the 4 scale bytes at 8 half + 4 jh and d (S/gen_llm.py:320-325). Super-blocks are
// 210 bytes, so with 4-byte aligned weights a block starts on a 4-byte or a 2-byte boundary: the loader reads
// dwords from the aligned address below and shifts every dword pair by the block's misalignment (alignbit), never
// reading past the block (d comes as a 16-bit load).
struct Q6W {
  u32 l[16], h[8], sc, d;
};

__device__ __forceinline__ void q6k_load(const u8 *row, int item, bool live, Q6W &w) {
  const u8 *b = row + (int64_t)(item >> 2) * 210;
  const int half = (item >> 1) & 1, jh = item & 1;
  const uintptr_t a = reinterpret_cast<uintptr_t>(b);
  const u32 sh = (u32)(a & 2u) * 8u;
  const u32 *p = reinterpret_cast<const u32 *>(a & ~(uintptr_t)3);
  u32 t[17], u[9];
#pragma unroll
  for (int i = 0; i < 17; ++i) t[i] = live ? p[16 * half + i] : 0u;
#pragma unroll
  for (int i = 0; i < 9; ++i) u[i] = live ? p[32 + 8 * half + i] : 0u;
  const u32 c0 = live ? p[48 + 2 * half + jh] : 0u;
  const u32 c1 = (live && sh) ? p[49 + 2 * half + jh] : 0u;   // only a misaligned block's scales straddle
#pragma unroll
  for (int i = 0; i < 16; ++i) w.l[i] = __builtin_amdgcn_alignbit(t[i + 1], t[i], sh);
#pragma unroll
  for (int i = 0; i < 8; ++i) w.h[i] = __builtin_amdgcn_alignbit(u[i + 1], u[i], sh);
  w.sc = __builtin_amdgcn_alignbit(c1, c0, sh);
  w.d = live ? (u32)*reinterpret_cast<const u16 *>(b + 208) : 0u;
}

// the 6-bit codes of the item's groups as bytes: ca (values 0..31), cb (values 32..63)
__device__ __forceinline__ void q6k_codes(const Q6W &w, int jh, u32 (&ca)[8], u32 (&cb)[8]) {
  const u32 ls = 4u * (u32)jh;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ca[i] = ((w.l[i] >> ls) & 0x0F0F0F0Fu) | (((w.h[i] >> ls) & 0x03030303u) << 4);
    cb[i] = ((w.l[8 + i] >> ls) & 0x0F0F0F0Fu) | (((w.h[i] >> (ls + 2u)) & 0x03030303u) << 4);
  }
}

// the four 16-value scales f32(d) * sc of the item, exact
__device__ __forceinline__ void q6k_scales(const Q6W &w, float (&s)[4]) {
  const float d = f16_to_f32(w.d);
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = d * (float)(signed char)((w.sc >> (8 * i)) & 0xFFu);
}

template <bool BF16X>
struct Q6K {
  static constexpr int kValues = 64;
  struct X {
    typename std::conditional<BF16X, XB<8>, XF<8>>::type v;
    float s16[4];   // sums of the four 16-value runs
  };
  using W = Q6W;
  static __host__ __device__ __forceinline__ int items(int64_t k) { return (int)(k / 256) * 4; }
  static __device__ __forceinline__ void load_x(const void *xrow, int item, bool live, X &x) {
    const int64_t off = (int64_t)item * 64;
    if constexpr (BF16X) {
      xb_load<8>(static_cast<const u16 *>(xrow) + off, live, x.v);
      constexpr u32 kOnes = 0x3F803F80u;   // bf16 (1, 1)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float sa = 0.f, sb = 0.f;
#pragma unroll
        for (int i = 4 * q; i < 4 * q + 4; ++i) {
          sa = dot2(kOnes, x.v.a02[i], dot2(kOnes, x.v.a13[i], sa));
          sb = dot2(kOnes, x.v.b02[i], dot2(kOnes, x.v.b13[i], sb));
        }
        x.s16[q] = sa;
        x.s16[2 + q] = sb;
      }
    } else {
      xf_load<8>(static_cast<const float *>(xrow) + off, live, x.v);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float sa = 0.f, sb = 0.f;
#pragma unroll
        for (int i = 16 * q; i < 16 * q + 16; ++i) {
          sa += x.v.a[i];
          sb += x.v.b[i];
        }
        x.s16[q] = sa;
        x.s16[2 + q] = sb;
      }
    }
  }
  static __device__ __forceinline__ void load_w(const u8 *row, const u8 *, int item, bool live, W &w) {
    q6k_load(row, item, live, w);
  }
  // sum over the four runs of s_run (sum (q - 32) x): the run sum of (128 + q) x (bf16: codes or-ed into bf16 128)
  // or q x (f32), less 160 or 32 times the run's sum of x
  static __device__ __forceinline__ float dot(const W &w, const X &x, int item) {
    u32 ca[8], cb[8];
    q6k_codes(w, item & 1, ca, cb);
    float s[4];
    q6k_scales(w, s);
    float p[4];
    if constexpr (BF16X) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
        for (int i = 4 * q; i < 4 * q + 4; ++i) {
          a0 = dot2((ca[i] & 0x00FF00FFu) | kBf16_128, x.v.a02[i], a0);
          a1 = dot2(((ca[i] >> 8) & 0x00FF00FFu) | kBf16_128, x.v.a13[i], a1);
          b0 = dot2((cb[i] & 0x00FF00FFu) | kBf16_128, x.v.b02[i], b0);
          b1 = dot2(((cb[i] >> 8) & 0x00FF00FFu) | kBf16_128, x.v.b13[i], b1);
        }
        p[q] = __builtin_fmaf(-160.f, x.s16[q], a0 + a1);
        p[2 + q] = __builtin_fmaf(-160.f, x.s16[2 + q], b0 + b1);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
        for (int i = 4 * q; i < 4 * q + 4; ++i) {
          a0 = __builtin_fmaf((float)(ca[i] & 0xFFu), x.v.a[4 * i + 0], a0);
          a1 = __builtin_fmaf((float)((ca[i] >> 8) & 0xFFu), x.v.a[4 * i + 1], a1);
          a0 = __builtin_fmaf((float)((ca[i] >> 16) & 0xFFu), x.v.a[4 * i + 2], a0);
          a1 = __builtin_fmaf((float)(ca[i] >> 24), x.v.a[4 * i + 3], a1);
          b0 = __builtin_fmaf((float)(cb[i] & 0xFFu), x.v.b[4 * i + 0], b0);
          b1 = __builtin_fmaf((float)((cb[i] >> 8) & 0xFFu), x.v.b[4 * i + 1], b1);
          b0 = __builtin_fmaf((float)((cb[i] >> 16) & 0xFFu), x.v.b[4 * i + 2], b0);
          b1 = __builtin_fmaf((float)(cb[i] >> 24), x.v.b[4 * i + 3], b1);
        }
        p[q] = __builtin_fmaf(-32.f, x.s16[q], a0 + a1);
        p[2 + q] = __builtin_fmaf(-32.f, x.s16[2 + q], b0 + b1);
      }
    }
    return __builtin_fmaf(s[0], p[0], s[1] * p[1]) + __builtin_fmaf(s[2], p[2], s[3] * p[3]);
  }
};

}  // namespace qmm
