// f16 staging of GGUF-block weights for the f16 MFMA kernels, and the expert activation: shared by the prefill GEMM /
// grouped GEMMs over 64-row tiles (gemm_q4k.hip) and the grouped GEMMs over expert tiles of few rows
// (grouped_q4k_narrow.hip). The staging is the reference's: Q4_K w = fma_f16(f16(q), f16(d sc), f16(-dmin m))
// (S/gen_gemm.py:499-530), Q4_0 w = f16(d (q - 8)) with one rounding (S/moe_q4_0.py:11-38).
#pragma once

#include "common.hpp"

namespace qmm {

typedef __attribute__((ext_vector_type(2))) _Float16 h2;

__device__ __forceinline__ h2 as_h2(u32 v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ u32 as_u32(h2 v) { return __builtin_bit_cast(u32, v); }

// 8 f16 weights of one column in K order from two code dwords (values 0..3 and 4..7 of the run) of one nibble
// plane: bytes become (1024 + q) f16 pairs with one v_perm each, the 1024 is removed exactly, then one rounding
// fma with the sub-block's f16 scale and negated minimum.
__device__ __forceinline__ f16x8 deq8_codes(u32 n0, u32 n1, h2 dsc, h2 nmn) {
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
template <bool HI>
__device__ __forceinline__ f16x8 deq8(u32 q0, u32 q1, h2 dsc, h2 nmn) {
  return deq8_codes(HI ? (q0 >> 4) & 0x0F0F0F0Fu : q0 & 0x0F0F0F0Fu, HI ? (q1 >> 4) & 0x0F0F0F0Fu : q1 & 0x0F0F0F0Fu,
                    dsc, nmn);
}
// The same 8 weights with the codes converted by the FP8 converter: a code byte 0000qqqq read as OCP E4M3 is
// q 2^-9 exactly, so v_cvt_scalef32_pk_f16_fp8 with scale 512 gives two f16 codes an instruction (where the
// (1024 + q) route takes a v_perm and an add); then the same one rounding fma.
template <bool HI>
__device__ __forceinline__ f16x8 deq8_e4m3(u32 q0, u32 q1, h2 dsc, h2 nmn) {
  const u32 n0 = HI ? (q0 >> 4) & 0x0F0F0F0Fu : q0 & 0x0F0F0F0Fu;
  const u32 n1 = HI ? (q1 >> 4) & 0x0F0F0F0Fu : q1 & 0x0F0F0F0Fu;
  const h2 c[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n0, 512.0f, false),
                   __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n0, 512.0f, true),
                   __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n1, 512.0f, false),
                   __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n1, 512.0f, true)};
  u32 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = as_u32(__builtin_elementwise_fma(c[i], dsc, nmn));
  typedef __attribute__((ext_vector_type(4))) u32 u32x4;
  return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}
// Q4_0: 8 f16 weights from two code dwords: (1024 + q) - 1032 = q - 8 exactly, then one rounding f16 multiply by d
// (f16(d (q - 8)), the reference's staging, also where -8 d would overflow f16)
template <bool HI>
__device__ __forceinline__ f16x8 deq8_q40(u32 q0, u32 q1, h2 d) {
  const u32 n0 = HI ? (q0 >> 4) & 0x0F0F0F0Fu : q0 & 0x0F0F0F0Fu, n1 = HI ? (q1 >> 4) & 0x0F0F0F0Fu : q1 & 0x0F0F0F0Fu;
  const u32 k64 = 0x64646464u;
  const h2 m1032 = __builtin_bit_cast(h2, 0xE408E408u);
  const u32 t[4] = {__builtin_amdgcn_perm(k64, n0, 0x04010400u), __builtin_amdgcn_perm(k64, n0, 0x04030402u),
                    __builtin_amdgcn_perm(k64, n1, 0x04010400u), __builtin_amdgcn_perm(k64, n1, 0x04030402u)};
  u32 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __builtin_bit_cast(u32, (__builtin_bit_cast(h2, t[i]) + m1032) * d);
  typedef __attribute__((ext_vector_type(4))) u32 u32x4;
  return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

// Q6_K (210-byte super-blocks, only 2-byte aligned): 16-byte pieces are loaded at any even address (the HSA
// runtime runs the GPU in unaligned access mode; the compiler emits global_load_dwordx4 for them).
typedef uint4 uint4_a2 __attribute__((aligned(2)));
typedef u32 u32_a2 __attribute__((aligned(2)));
__device__ __forceinline__ uint4 ld16u(const u8 *p) { return *reinterpret_cast<const uint4_a2 *>(p); }
__device__ __forceinline__ u32 ld4u(const u8 *p) { return *reinterpret_cast<const u32_a2 *>(p); }

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

}  // namespace qmm
