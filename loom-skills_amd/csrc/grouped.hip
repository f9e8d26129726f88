// qmm_moe_grouped: argument checks shared by the grouped expert GEMMs and the dispatch to the GGUF-block (Q4_K, Q6_K,
// Q4_0: f16 MFMA, gemm_q4k.hip) and MXFP4 split-plane / MFMA-tiled (scaled f8f6f4 MFMA, grouped_mxfp4.hip) kernels.
// The runtime arguments keep the order of the reference's launches of g_moe_ggu_* / g_moe_gdn_*:
// (max_rows, k, n, xrows, tile_info, rowmap, x16, scales, w [, w2] [, biases], y) (S/gen_llm.py:5376-5378).
#include "common.hpp"

int qmm_grouped_q4k(int fmt, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E, int KU,
                    const int32_t *tile_info, const int32_t *rowmap, const void *x, const float *x_scales,
                    int64_t x_rows, const void *w, const void *w2, const float *bias, const float *bias2, float *y,
                    hipStream_t s);
int qmm_grouped_mxfp4(int tiled, int mode, int fused, int act, int64_t max_tiles, int64_t k, int64_t n, int E, int KU,
                      const int32_t *tile_info, const int32_t *rowmap, const void *x, const void *x_scales,
                      int64_t x_rows, const void *w, const void *ws, const void *w2, const void *ws2,
                      const float *bias, const float *bias2, float *y, uint8_t *y8, uint8_t *ys8, hipStream_t s);

namespace {
// the checks both grouped entry points share; max_rows = max_tiles * 64
int check_grouped(int act, int E, int KU, int64_t max_rows, int64_t k, int64_t n, int64_t x_rows,
                  const int32_t *tile_info, const int32_t *rowmap, const void *x, const void *w) {
  using namespace qmm;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!tile_info || !rowmap || !x || !w) return QMM_ERR_NULL;
  if (max_rows <= 0 || max_rows % 64 || max_rows > (int64_t(1) << 24)) return QMM_ERR_SHAPE;
  if (k <= 0 || n <= 0 || k > (1 << 20) || n > (1 << 20) || x_rows <= 0) return QMM_ERR_SHAPE;
  return QMM_OK;
}
}  // namespace

extern "C" int qmm_moe_grouped(int fmt, int mode, int fused, int act, int E, int KU, int64_t max_rows, int64_t k,
                               int64_t n, int64_t x_rows, const int32_t *tile_info, const int32_t *rowmap,
                               const void *x, int x_dtype, const void *x_scales, const void *w, const void *ws,
                               const void *w2, const void *ws2, const float *bias, const float *bias2, float *y,
                               qmm_stream_t stream) {
  using namespace qmm;
  if (!fmt_code_ok(fmt)) return QMM_ERR_FORMAT;
  const bool mixed = fmt_mixed(fmt);   // QMM_GATE_UP(gate, up): GGUF gate / up tensors in two formats
  const int fg = fmt_gate(fmt);
  if (fg != QMM_Q4_K && fg != QMM_Q4_KT && fg != QMM_Q6_K && fg != QMM_Q4_0 && fg != QMM_MXFP4S && fg != QMM_MXFP4T)
    return QMM_ERR_FORMAT;
  if (mixed && (mode != 0 || fused)) return QMM_ERR_FORMAT;   // one up tensor in its own format, gate/up only
  if (mode != 0 && mode != 1) return QMM_ERR_RANGE;
  if (int st = check_grouped(act, E, KU, max_rows, k, n, x_rows, tile_info, rowmap, x, w)) return st;
  if (!y) return QMM_ERR_NULL;
  // an unfused gate/up needs its up matrix on every kernel path (the narrow and 64-row Q4_K kernels, MXFP4)
  if (mode == 0 && !fused && !w2) return QMM_ERR_NULL;
  if (mode == 1 && x_rows < max_rows) return QMM_ERR_SHAPE;   // the down GEMM reads its sorted rows in place
  if (!aligned(y, 4) || !aligned(bias, 4) || !aligned(bias2, 4)) return QMM_ERR_ALIGN;
  const int64_t max_tiles = max_rows / 64;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (mixed || fmt == QMM_Q4_K || fmt == QMM_Q4_KT || fmt == QMM_Q6_K || fmt == QMM_Q4_0) {
    if (x_dtype != QMM_F16) return QMM_ERR_DTYPE;
    return qmm_grouped_q4k(fmt, mode, fused, act, max_tiles, k, n, E, KU, tile_info, rowmap, x,
                           static_cast<const float *>(x_scales), x_rows, w, w2, bias, bias2, y, s);
  }
  if (x_dtype != QMM_MXFP8) return QMM_ERR_DTYPE;
  return qmm_grouped_mxfp4(fmt == QMM_MXFP4T, mode, fused, act, max_tiles, k, n, E, KU, tile_info, rowmap, x,
                           x_scales, x_rows, w, ws, w2, ws2, bias, bias2, y, nullptr, nullptr, s);
}

extern "C" int qmm_moe_grouped_mxfp8(int fmt, int fused, int act, int E, int KU, int64_t max_rows, int64_t k,
                                     int64_t n, int64_t x_rows, const int32_t *tile_info, const int32_t *rowmap,
                                     const void *x, const void *x_scales, const void *w, const void *ws,
                                     const void *w2, const void *ws2, const float *bias, const float *bias2,
                                     uint8_t *codes, uint8_t *scales, qmm_stream_t stream) {
  using namespace qmm;
  if (fmt != QMM_MXFP4S && fmt != QMM_MXFP4T) return QMM_ERR_FORMAT;
  if (int st = check_grouped(act, E, KU, max_rows, k, n, x_rows, tile_info, rowmap, x, w)) return st;
  if (!codes || !scales) return QMM_ERR_NULL;
  if (!fused && (!w2 || !ws2)) return QMM_ERR_NULL;
  if (n % 32) return QMM_ERR_SHAPE;
  if (!aligned(bias, 4) || !aligned(bias2, 4)) return QMM_ERR_ALIGN;
  return qmm_grouped_mxfp4(fmt == QMM_MXFP4T, 0, fused, act, max_rows / 64, k, n, E, KU, tile_info, rowmap, x,
                           x_scales, x_rows, w, ws, w2, ws2, bias, bias2, nullptr, codes, scales,
                           reinterpret_cast<hipStream_t>(stream));
}
