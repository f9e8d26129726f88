// qmm_moe_routed_static: qmm_moe_routed (moe_chain.hip) for callers that cannot allocate device memory -- code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. The chain's intermediates go to `scratch`,
// a file-scope device array of kScratchBytes that every GPU the library runs on holds until the process ends; its
// address on the current device is taken once per device (hipGetSymbolAddress) and kept. Every call on one GPU uses
// that GPU's one array: calls that overlap on one GPU (two streams, two host threads) race on it. No intermediate of
// the chain needs to start at zero (each is written in full before it is read), so nothing is cleared between calls.
#include <mutex>

#include "common.hpp"

using namespace qmm;

namespace {
// 16 MiB: the decode chain of a model with H + FE <= 8192 and top-8 routing on given logits at up to 63 tokens on
// f32 / bf16 activations, and up to 48 tokens on the Q8_1 path (QMM_MOE_Q8 adds the quantized input and gate/up rows)
constexpr int64_t kScratchBytes = int64_t(16) << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];   // the array's address on each device (host-side stand-in `scratch` is never used)

int scratch_on_current_device(void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return QMM_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return QMM_ERR_RANGE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return QMM_ERR_LAUNCH;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return QMM_OK;
}
}  // namespace

extern "C" int qmm_moe_routed_static(int fmt, int fmt_down, int fused, int act, int gating, int norm, float scale,
                                     int flags, int E, int KU, int64_t tokens, int64_t H, int64_t FE, const void *x,
                                     int x_dtype, const float *logits, const void *w_router, int w_router_dtype,
                                     const float *router_bias, const float *down_scale, const void *w_gate,
                                     const void *ws_gate, const void *w_up, const void *ws_up, const void *w_down,
                                     const void *ws_down, const float *bias_gate, const float *bias_up,
                                     const float *bias_down, const float *sg, int accumulate, float *y,
                                     qmm_stream_t stream) {
  const int64_t need = qmm_moe_routed_workspace_size(fmt, flags, E, KU, tokens, H, FE, logits == nullptr);
  if (need > kScratchBytes) return QMM_ERR_WORKSPACE;   // larger than the static array: use qmm_moe_routed
  void *ws = nullptr;
  if (int st = scratch_on_current_device(&ws)) return st;
  return qmm_moe_routed(fmt, fmt_down, fused, act, gating, norm, scale, flags, E, KU, tokens, H, FE, x, x_dtype,
                        logits, w_router, w_router_dtype, router_bias, down_scale, w_gate, ws_gate, w_up, ws_up,
                        w_down, ws_down, bias_gate, bias_up, bias_down, sg, accumulate, y, ws, kScratchBytes, stream);
}
