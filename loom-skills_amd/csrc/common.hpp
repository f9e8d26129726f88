// Shared helpers of libqmm (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/qmm.h"

namespace qmm {

constexpr int kWave = 64;

typedef uint32_t u32;
typedef uint16_t u16;
typedef uint8_t u8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(8))) int i32x8;
typedef __attribute__((ext_vector_type(4))) int i32x4;

// ------------------------------------------------------------------------------------------- number formats
__device__ __forceinline__ float f16_to_f32(u32 bits16) {
  return (float)__builtin_bit_cast(_Float16, (u16)(bits16 & 0xFFFFu));
}
__device__ __forceinline__ float bf16_to_f32(u32 bits16) { return __builtin_bit_cast(float, bits16 << 16); }
__device__ __forceinline__ u32 f32_to_bf16_rne(float f) {
  u32 u = __builtin_bit_cast(u32, f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float u32_as_f32(u32 u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ u32 f32_as_u32(float f) { return __builtin_bit_cast(u32, f); }

// 2^(e - 127) for an E8M0 byte (e = 0 gives the subnormal 2^-127).
__device__ __forceinline__ float e8m0_scale(u32 e) { return u32_as_f32(e == 0 ? 0x00400000u : (e << 23)); }
// ggml's GGML_E8M0_TO_FP32_HALF: 2^(e - 128).
__device__ __forceinline__ float e8m0_half(u32 e) { return u32_as_f32(e < 2 ? (0x00200000u << e) : ((e - 1) << 23)); }

// Q4_K 6-bit (scale, minimum) of sub-block g (0..7) from the three packed-scale dwords
// s0 = S[0..3], s1 = S[4..7], s2 = S[8..11] (ggml get_scale_min_k4).
__device__ __forceinline__ void q4k_scale_min(u32 s0, u32 s1, u32 s2, int g, u32 &sc, u32 &mn) {
  const int sh = 8 * (g & 3);
  const u32 a1 = (s0 >> sh) & 0xFFu, a2 = (s1 >> sh) & 0xFFu, a3 = (s2 >> sh) & 0xFFu;
  const bool hi = g >= 4;
  sc = hi ? ((a3 & 15u) | ((a1 >> 6) << 4)) : (a1 & 63u);
  mn = hi ? ((a3 >> 4) | ((a2 >> 6) << 4)) : (a2 & 63u);
}

// OCP MX E8M0 exponent of a 32-value block whose largest magnitude is amax: s = clamp(floor(log2(amax)) - 7, -127,
// 127) (-127 for amax = 0), which keeps every |x| 2^-s below 256, under the E4M3 maximum 448. The scale byte is
// s + 127.
__device__ __forceinline__ int mxfp8_exponent(float amax) {
  int sx = -127;
  if (amax > 0.f) {
    int ex;
    frexpf(amax, &ex);        // amax = f 2^ex, f in [0.5, 1)
    sx = min(max(ex - 1 - 7, -127), 127);
  }
  return sx;
}
// E4M3 codes of (a, b) x 2^-sx in bytes 0-1 (HI = false) or 2-3 (HI = true) of w: v_cvt_pk_fp8_f32, round to
// nearest even, OCP E4M3FN on gfx950.
template <bool HI>
__device__ __forceinline__ int e4m3_pack2(float a, float b, int sx, int w) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(a, -sx), ldexpf(b, -sx), w, HI);
}

// The expert activations (S/gen_moe.py:27-46): silu(g) u = g / (1 + e^-g) u, and gpt-oss's swiglu_oai
// min(g, 7) sigmoid(1.702 min(g, 7)) (clamp(u, -7, 7) + 1).
__device__ __forceinline__ float act_fn(int act, float g, float u) {
  if (act == QMM_ACT_SWIGLU_OAI) {
    const float xg = fminf(g, 7.0f);
    const float yu = fminf(fmaxf(u, -7.0f), 7.0f);
    return xg / (1.0f + expf(-1.702f * xg)) * (yu + 1.0f);
  }
  return g / (1.0f + expf(-g)) * u;
}

// ----------------------------------------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// ------------------------------------------------------------------------------------------- host helpers
inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? QMM_OK : QMM_ERR_LAUNCH;
}

// Raises kernel fn's dynamic-LDS limit to `bytes` (the largest any launch of it asks for) on the current device, once
// per device: `done` holds one bit per device id (ids >= 32 are raised on every call, which is harmless).
inline int raise_dyn_lds(const void *fn, int bytes, std::atomic<unsigned> &done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return QMM_ERR_LAUNCH;
  const unsigned bit = dev < 32 ? 1u << dev : 0u;
  if (bit && (done.load(std::memory_order_relaxed) & bit)) return QMM_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return QMM_ERR_LAUNCH;
  done.fetch_or(bit, std::memory_order_relaxed);
  return QMM_OK;
}

// QMM_GATE_UP(gate, up): the gate matrix's format and the up matrix's (the gate's when the call names one format)
inline int fmt_gate(int fmt) { return fmt < 0 ? fmt : fmt & 0xFF; }
inline int fmt_up(int fmt) {
  if (fmt < 0) return fmt;
  const int u = (fmt >> 8) & 0xFF;
  return u ? u - 1 : (fmt & 0xFF);
}
inline bool fmt_mixed(int fmt) { return fmt >= 0 && fmt_gate(fmt) != fmt_up(fmt); }
// a format code is one format or a gate/up pair, nothing more
inline bool fmt_code_ok(int fmt) { return fmt >= 0 && (fmt >> 16) == 0; }

inline int64_t block_values(int fmt) {
  switch (fmt) {
    case QMM_Q4_0: return 32;
    case QMM_Q4_K: return 256;
    case QMM_MXFP4: return 32;
    case QMM_MXFP4S: return 32;
    case QMM_MXFP4T: return 32;
    case QMM_Q4_KT: return 256;
    case QMM_Q6_K: return 256;
    case QMM_Q4_0T: return 512;
    default: return 0;
  }
}
inline int64_t block_bytes(int fmt) {
  switch (fmt) {
    case QMM_Q4_0: return 18;
    case QMM_Q4_K: return 144;
    case QMM_MXFP4: return 17;
    case QMM_MXFP4S: return 16;
    case QMM_MXFP4T: return 16;
    case QMM_Q4_KT: return 144;
    case QMM_Q6_K: return 210;
    case QMM_Q4_0T: return 288;
    default: return 0;
  }
}
inline int64_t row_bytes(int fmt, int64_t k) {
  const int64_t bv = block_values(fmt);
  if (bv == 0 || k <= 0 || k % bv) return 0;
  return k / bv * block_bytes(fmt);
}

}  // namespace qmm
