// Grouped expert GEMM (MFMA); in progress.
#include "common.hpp"

extern "C" int qmm_moe_grouped(int, int, int, int, int64_t, int64_t, int64_t, int, int, const int32_t *,
                               const int32_t *, const void *, int, const void *, int64_t, const void *, const void *,
                               const void *, const void *, const float *, float *, qmm_stream_t) {
  return QMM_ERR_FORMAT;
}
