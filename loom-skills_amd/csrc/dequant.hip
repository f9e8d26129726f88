// Bit-exact dequantization kernels (parity / debug path) and the library's small host entry points.
//
// Each thread decodes one 32-value group into f32, with the single rounding of the reference's value helpers:
//   Q4_0   w = f32(d) * (q - 8)                       S/quant_values.loom:386-408
//   Q4_K   w = (f32(d) * sc) * q - f32(dmin) * m      S/gen_llm.py:269-326
//   Q6_K   w = (f32(d) * sc) * (q - 32)               S/gen_llm.py:320-397 (super-blocks 2-byte aligned)
//   MXFP4  w = kvalues[code] * 2^(e - 128)            S/gen_llm.py:786-841 (code 8 -> +0)
//   MXFP4S w = E2M1(code) * 2^(e - 127)               S/st_tensors.py:26-33 (code 8 -> -0)
//   MXFP4T the same values from MFMA-tiled planes (grouped_mxfp4.hip)
//   Q4_KT  the Q4_K values from the tiled GEMV layout (gemv_q4kt.hip)
//   Q4_0T  the Q4_0 values from the tiled GEMV layout (gemv_q4kt.hip)
#include "common.hpp"

using namespace qmm;

int qmm_dequant_mxfp4t(const void *w, const void *ws, int64_t rows, int64_t k, float *out, hipStream_t s);
int qmm_dequant_q4kt(const void *w, int64_t rows, int64_t k, float *out, hipStream_t s);
int qmm_dequant_q40t(const void *w, int64_t rows, int64_t k, float *out, hipStream_t s);

namespace {

__constant__ float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
__constant__ signed char kKvalues[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

__global__ void dequant_q4_0_kernel(const u8 *__restrict__ w, int64_t groups, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const u8 *b = w + gi * 18;
  const float d = f16_to_f32((u32)b[0] | ((u32)b[1] << 8));
  float *o = out + gi * 32;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const u32 q = b[2 + j];
    o[j] = d * (float)((int)(q & 15u) - 8);
    o[j + 16] = d * (float)((int)(q >> 4) - 8);
  }
}

__global__ void dequant_q4_k_kernel(const u8 *__restrict__ w, int64_t groups, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // one 32-value sub-block
  if (gi >= groups) return;
  const int64_t blk = gi >> 3;
  const int g = (int)(gi & 7);
  const u32 *h = reinterpret_cast<const u32 *>(w + blk * 144);
  const u32 h0 = h[0], s0 = h[1], s1 = h[2], s2 = h[3];
  u32 sc, mn;
  q4k_scale_min(s0, s1, s2, g, sc, mn);
  const float scale = f16_to_f32(h0) * (float)sc;
  const float minimum = f16_to_f32(h0 >> 16) * (float)mn;
  const u8 *qs = w + blk * 144 + 16 + 32 * (g >> 1);
  const int shift = 4 * (g & 1);
  float *o = out + gi * 32;
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    const float q = (float)((qs[l] >> shift) & 15u);
    o[l] = __fsub_rn(__fmul_rn(scale, q), minimum);
  }
}

// One 32-value group g = 4 half + j of a Q6_K super-block: code q = ((ql[64 half + 32 (j % 2) + l] >> 4 (j / 2)) &
// 15) | (((qh[32 half + l] >> 2 j) & 3) << 4), scale sc[8 half + 2 j + l / 16]. Byte loads: blocks are 210 bytes.
__global__ void dequant_q6_k_kernel(const u8 *__restrict__ w, int64_t groups, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const u8 *b = w + (gi >> 3) * 210;
  const int g = (int)(gi & 7), half = g >> 2, j = g & 3;
  const float d = f16_to_f32((u32)b[208] | ((u32)b[209] << 8));
  const float s0 = d * (float)(signed char)b[192 + 8 * half + 2 * j];
  const float s1 = d * (float)(signed char)b[192 + 8 * half + 2 * j + 1];
  const u8 *ql = b + 64 * half + 32 * (j & 1), *qh = b + 128 + 32 * half;
  const int ls = 4 * (j >> 1), hs = 2 * j;
  float *o = out + gi * 32;
#pragma unroll
  for (int l = 0; l < 32; ++l) {
    const int q = (int)(((ql[l] >> ls) & 15u) | (((qh[l] >> hs) & 3u) << 4));
    o[l] = __fmul_rn(l < 16 ? s0 : s1, (float)(q - 32));
  }
}

__global__ void dequant_mxfp4_kernel(const u8 *__restrict__ w, int64_t groups, float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const u8 *b = w + gi * 17;
  const float half = e8m0_half(b[0]);
  float *o = out + gi * 32;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const u32 q = b[1 + j];
    o[j] = (float)kKvalues[q & 15u] * half;
    o[j + 16] = (float)kKvalues[q >> 4] * half;
  }
}

__global__ void dequant_mxfp4s_kernel(const u8 *__restrict__ nib, const u8 *__restrict__ sc, int64_t groups,
                                      float *__restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const float s = e8m0_scale(sc[gi]);
  const u8 *b = nib + gi * 16;
  float *o = out + gi * 32;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const u32 q = b[j];
    const u32 lo = q & 15u, hi = q >> 4;
    const float vlo = kE2M1[lo & 7u] * s, vhi = kE2M1[hi & 7u] * s;
    o[2 * j] = (lo & 8u) ? -vlo : vlo;
    o[2 * j + 1] = (hi & 8u) ? -vhi : vhi;
  }
}

}  // namespace

extern "C" {

int qmm_version(void) { return 100; }

const char *qmm_strerror(int status) {
  switch (status) {
    case QMM_OK: return "ok";
    case QMM_ERR_FORMAT: return "unsupported weight format";
    case QMM_ERR_SHAPE: return "invalid shape";
    case QMM_ERR_ALIGN: return "misaligned pointer";
    case QMM_ERR_NULL: return "null pointer";
    case QMM_ERR_RANGE: return "argument out of range";
    case QMM_ERR_DTYPE: return "unsupported dtype";
    case QMM_ERR_LAUNCH: return "kernel launch failed";
    case QMM_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

int64_t qmm_row_bytes(int fmt, int64_t k) { return row_bytes(fmt, k); }

int qmm_dequant(int fmt, const void *w, const void *ws, int64_t rows, int64_t k, float *out, qmm_stream_t stream) {
  if (fmt < QMM_Q4_0 || fmt > QMM_Q4_0T) return QMM_ERR_FORMAT;
  if (!w || !out || ((fmt == QMM_MXFP4S || fmt == QMM_MXFP4T) && !ws)) return QMM_ERR_NULL;
  if (rows <= 0 || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (fmt == QMM_MXFP4T) return qmm_dequant_mxfp4t(w, ws, rows, k, out, reinterpret_cast<hipStream_t>(stream));
  if (fmt == QMM_Q4_KT) return qmm_dequant_q4kt(w, rows, k, out, reinterpret_cast<hipStream_t>(stream));
  if (fmt == QMM_Q4_0T) return qmm_dequant_q40t(w, rows, k, out, reinterpret_cast<hipStream_t>(stream));
  if (fmt == QMM_Q4_K && !aligned(w, 4)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t groups = rows * (k / 32);
  const int threads = 256;
  const unsigned grid = (unsigned)((groups + threads - 1) / threads);
  const u8 *wb = static_cast<const u8 *>(w);
  switch (fmt) {
    case QMM_Q4_0: dequant_q4_0_kernel<<<grid, threads, 0, s>>>(wb, groups, out); break;
    case QMM_Q4_K: dequant_q4_k_kernel<<<grid, threads, 0, s>>>(wb, groups, out); break;
    case QMM_MXFP4: dequant_mxfp4_kernel<<<grid, threads, 0, s>>>(wb, groups, out); break;
    case QMM_Q6_K: dequant_q6_k_kernel<<<grid, threads, 0, s>>>(wb, groups, out); break;
    default: dequant_mxfp4s_kernel<<<grid, threads, 0, s>>>(wb, static_cast<const u8 *>(ws), groups, out); break;
  }
  return launch_status();
}

}  // extern "C"
