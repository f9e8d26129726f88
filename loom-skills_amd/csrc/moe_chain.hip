// qmm_moe_routed: the routed experts of one MoE layer as one call, the command sequence the reference's moe_routed
// emits (S/gen_llm.py:5324-5385) run on one stream with a caller-passed workspace for its intermediates (the buffers
// moe_alloc allocates, S/gen_llm.py:5388-5432):
//
//   prefill (tokens >= 64): route (router matvec + top-k, or top-k of given logits; with given logits and bf16 rows
//     the top-k launch also writes the activation operand), [wscale], bucket into 64-row
//     expert tiles, the activation operand (GGUF formats: row-scaled f16; MXFP4: MXFP8), grouped gate/up GEMM with the
//     activation, its output's operand, grouped down GEMM, combine of the sorted rows;
//   decode (tokens < 64): route, [wscale], gate/up expert matvecs, down expert matvecs (f32 / bf16 activations, or
//     with QMM_MOE_Q8 the int8 path: the input and the gate/up output quantized to Q8_1), combine in assignment order.
//
// Every step is one of this library's entry points, so the chain computes what the separate calls compute, bit for
// bit. The workspace is carved into 256-byte aligned pieces by moe_plan, the single description of its layout that
// qmm_moe_routed_workspace_size reports.
#include "common.hpp"

using namespace qmm;

namespace {

constexpr int kTile = 64;
constexpr int kMinPrefillTokens = 64;   // %gemm: epochs of 64+ tokens take the grouped chain (S/gen_llm.py:6107-6126)

int64_t up256(int64_t b) { return (b + 255) / 256 * 256; }
int64_t q8_bytes(int64_t rows, int64_t k) { return rows * k + rows * (k / 32) * 8; }
bool gguf_blocks(int fmt) { return fmt == QMM_Q4_K || fmt == QMM_Q6_K || fmt == QMM_Q4_0; }
bool mx_planes(int fmt) { return fmt == QMM_MXFP4S || fmt == QMM_MXFP4T; }

// byte offsets of the chain's intermediates in the workspace (0-sized pieces are unused)
struct Plan {
  bool prefill, q8, mx;
  int64_t max_tiles, max_rows, A;
  int64_t logits, ids, wts, tile_info, rowmap, pos, xa, xs, act, a2, as, ys, total;
};

Plan moe_plan(int fmt, int flags, int E, int KU, int64_t T, int64_t H, int64_t FE, bool router) {
  fmt = fmt_gate(fmt);   // a QMM_GATE_UP pair plans as its gate format (GGUF blocks either way)
  Plan p{};
  p.prefill = T >= kMinPrefillTokens;
  p.q8 = !p.prefill && (flags & QMM_MOE_Q8);
  p.mx = mx_planes(fmt);
  p.A = T * KU;
  p.max_tiles = p.A / kTile + E;
  p.max_rows = p.max_tiles * kTile;
  int64_t at = 0;
  auto take = [&](int64_t bytes) { const int64_t o = at; at += up256(bytes); return o; };
  p.logits = take(router ? T * E * 4 : 0);
  p.ids = take(p.A * 4);
  p.wts = take(p.A * 4);
  if (p.prefill) {
    p.tile_info = take(p.max_tiles * 2 * 4);
    p.rowmap = take(p.max_rows * 4);
    p.pos = take(p.A * 4);
    if (p.mx) {                    // MXFP8 operands: E4M3 codes + E8M0 per 32
      p.xa = take(T * H);
      p.xs = take(T * (H / 32));
      p.act = take(p.max_rows * FE);
      p.as = take(p.max_rows * (FE / 32));
    } else {                       // row-scaled f16 operands + (2^-e, 2^e) per row
      p.xa = take(T * H * 2);
      p.xs = take(T * 2 * 4);
      p.act = take(p.max_rows * FE * 4);
      p.a2 = take(p.max_rows * FE * 2);
      p.as = take(p.max_rows * 2 * 4);
    }
    p.ys = take(p.max_rows * H * 4);
  } else {
    if (p.q8) p.xa = take(q8_bytes(T, H));
    p.act = take(p.A * FE * 4);
    if (p.q8) p.a2 = take(q8_bytes(p.A, FE));
    p.ys = take(p.A * H * 4);
  }
  p.total = at;
  return p;
}

int check_chain(int fmt, int fmt_down, int flags, int E, int KU, int64_t T, int64_t H, int64_t FE) {
  if (E <= 0 || E > 256 || KU <= 0 || KU > 8 || KU > E) return QMM_ERR_RANGE;
  if (!fmt_code_ok(fmt) || fmt_mixed(fmt_down)) return QMM_ERR_FORMAT;
  if (fmt_mixed(fmt)) {
    // QMM_GATE_UP(gate, up): GGUF gate / up tensors in two formats (two tensors), f32 / bf16 decode activations (the
    // reference's int8 expert matvecs take one format, S/gen_moe.py:545)
    if (!gguf_blocks(fmt_gate(fmt)) || !gguf_blocks(fmt_up(fmt)) || (flags & QMM_MOE_Q8)) return QMM_ERR_FORMAT;
    fmt = fmt_gate(fmt);
  }
  if (flags & ~QMM_MOE_Q8) return QMM_ERR_RANGE;
  if (T <= 0 || T > 65536 || H <= 0 || FE <= 0 || H > (1 << 20) || FE > (1 << 20)) return QMM_ERR_SHAPE;
  const bool prefill = T >= kMinPrefillTokens;
  if (prefill) {   // the tiled Q4_K layout: the grouped GEMMs read it (prefill only, like the MXFP4 tiled planes)
    const bool g = gguf_blocks(fmt) || fmt == QMM_Q4_KT, d = gguf_blocks(fmt_down) || fmt_down == QMM_Q4_KT;
    if (g && d) return QMM_OK;
    if (mx_planes(fmt) && fmt_down == fmt) return QMM_OK;
    return QMM_ERR_FORMAT;
  }
  if (flags & QMM_MOE_Q8) return gguf_blocks(fmt) && gguf_blocks(fmt_down) ? QMM_OK : QMM_ERR_FORMAT;
  if (fmt == QMM_Q4_KT || fmt_down == QMM_Q4_KT) return QMM_ERR_FORMAT;   // the expert matvecs read GGUF blocks
  if ((fmt == QMM_MXFP4S) != (fmt_down == QMM_MXFP4S) || (fmt == QMM_MXFP4T) != (fmt_down == QMM_MXFP4T))
    return QMM_ERR_FORMAT;
  return QMM_OK;
}

}  // namespace

extern "C" int64_t qmm_moe_routed_workspace_size(int fmt, int flags, int E, int KU, int64_t tokens, int64_t H,
                                                 int64_t FE, int router) {
  if (check_chain(fmt, fmt_gate(fmt), flags, E, KU, tokens, H, FE) != QMM_OK) return -1;
  return moe_plan(fmt, flags, E, KU, tokens, H, FE, router != 0).total;
}

extern "C" int qmm_moe_routed(int fmt, int fmt_down, int fused, int act, int gating, int norm, float scale, int flags,
                              int E, int KU, int64_t tokens, int64_t H, int64_t FE, const void *x, int x_dtype,
                              const float *logits, const void *w_router, int w_router_dtype,
                              const float *router_bias, const float *down_scale, const void *w_gate,
                              const void *ws_gate, const void *w_up, const void *ws_up, const void *w_down,
                              const void *ws_down, const float *bias_gate, const float *bias_up,
                              const float *bias_down, const float *sg, int accumulate, float *y, void *workspace,
                              int64_t workspace_bytes, qmm_stream_t stream) {
  if (fmt_down < 0) fmt_down = fmt_gate(fmt);
  if (int st = check_chain(fmt, fmt_down, flags, E, KU, tokens, H, FE)) return st;
  if (!x || !y || !w_gate || !w_down || (!logits && !w_router)) return QMM_ERR_NULL;
  if (!fused && !w_up) return QMM_ERR_NULL;   // an unfused gate/up reads its up matrix in every chain
  if (fused && fmt_mixed(fmt)) return QMM_ERR_FORMAT;   // one fused gate_up tensor has one format
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  const Plan p = moe_plan(fmt, flags, E, KU, tokens, H, FE, logits == nullptr);
  if (!workspace) return QMM_ERR_NULL;
  if (workspace_bytes < p.total) return QMM_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QMM_ERR_ALIGN;
  char *ws = static_cast<char *>(workspace);
  auto at = [&](int64_t off) { return static_cast<void *>(ws + off); };
  int32_t *ids = static_cast<int32_t *>(at(p.ids));
  float *wts = static_cast<float *>(at(p.wts));
  const int64_t T = tokens;

  // ---- route; a prefill batch with given logits and bf16 rows also gets the gate/up operand in the same launch
  int st;
  const bool operand = p.prefill && logits && x_dtype == QMM_BF16 && H <= 4096 && H % (p.mx ? 32 : 8) == 0;
  // decode with given logits on f32 / bf16 activations, one key slot a lane and few assignments: the routing runs
  // inside the gate/up matvecs (every workgroup ranks its token itself: gpt-oss-20b at one token 25.0 -> 23.9 us;
  // slower with 128 experts or eight tokens)
  const bool route_gu = !p.prefill && !p.q8 && logits && E <= 64 && p.A <= 8 && !fmt_mixed(fmt);
  if (route_gu)
    st = mx_planes(fmt)
             ? qmm_moe_topk_expert_mv(logits, T, E, KU, gating, norm, scale, router_bias, ids, wts, fmt, fused, act, H,
                                      FE, x, x_dtype, w_gate, ws_gate, w_up, ws_up, bias_gate, bias_up,
                                      static_cast<float *>(at(p.act)), stream)
             : qmm_moe_topk_expert_mv(logits, T, E, KU, gating, norm, scale, router_bias, ids, wts, fmt, fused, act, H,
                                      FE, x, x_dtype, w_gate, nullptr, w_up, nullptr, bias_gate, bias_up,
                                      static_cast<float *>(at(p.act)), stream);
  else if (operand)
    st = qmm_moe_topk_operand(logits, T, E, KU, gating, norm, scale, router_bias, ids, wts, H, x, x_dtype,
                              p.mx ? QMM_MXFP8 : QMM_F16, at(p.xa), at(p.xs), stream);
  else if (logits)
    st = qmm_moe_topk(logits, T, E, KU, gating, norm, scale, router_bias, ids, wts, stream);
  else
    st = qmm_moe_route(T, H, E, KU, gating, norm, scale, x, x_dtype, w_router, w_router_dtype, router_bias, nullptr,
                       static_cast<float *>(at(p.logits)), ids, wts, stream);
  if (st) return st;
  if (down_scale && (st = qmm_moe_wscale(T, KU, E, ids, down_scale, wts, stream))) return st;
  float *ys = static_cast<float *>(at(p.ys));

  if (!p.prefill) {
    // ---- decode: per-assignment expert matvecs, combine in assignment order
    float *a = static_cast<float *>(at(p.act));
    if (p.q8) {
      void *xq = at(p.xa), *aq = at(p.a2);
      if ((st = qmm_quant_q8(T, H, x, x_dtype, xq, stream))) return st;
      if ((st = qmm_moe_expert_mv_q8(fmt, 0, fused, act, H, FE, E, KU, p.A, ids, xq, w_gate, w_up, bias_gate,
                                     bias_up, a, stream)))
        return st;
      if ((st = qmm_quant_q8(p.A, FE, a, QMM_F32, aq, stream))) return st;
      st = qmm_moe_expert_mv_q8(fmt_down, 1, 0, act, FE, H, E, KU, p.A, ids, aq, w_down, nullptr, bias_down, nullptr,
                                ys, stream);
      if (st) return st;
      return sg ? qmm_moe_combine_gated(T, p.A, H, KU, ys, nullptr, wts, sg, y, stream)
                : qmm_moe_combine(T, p.A, H, KU, ys, nullptr, wts, accumulate, y, stream);
    }
    if (route_gu)
      st = QMM_OK;   // the gate/up matvecs ran with the routing
    else if (fmt == QMM_MXFP4S)
      st = qmm_moe_expert_mv_split(0, fused, act, H, FE, E, KU, p.A, ids, x, x_dtype, w_gate, ws_gate, w_up, ws_up,
                                   bias_gate, bias_up, a, stream);
    else if (fmt == QMM_MXFP4T)
      st = qmm_moe_expert_mv_tiled(0, fused, act, H, FE, E, KU, p.A, ids, x, x_dtype, w_gate, ws_gate, w_up, ws_up,
                                   bias_gate, bias_up, a, stream);
    else
      st = qmm_moe_expert_mv(fmt, 0, fused, act, H, FE, E, KU, p.A, ids, x, x_dtype, w_gate, w_up, bias_gate,
                             bias_up, a, stream);
    if (st) return st;
    // the down matvecs and the combine in one launch (the ys rows are not written)
    return qmm_moe_expert_mv_combine(fmt_down, FE, H, E, KU, T, ids, wts, a, QMM_F32, w_down, ws_down, bias_down,
                                     accumulate, sg, y, stream);
  }

  // ---- prefill: bucket, grouped GEMMs, combine of the sorted rows
  int32_t *ti = static_cast<int32_t *>(at(p.tile_info)), *rm = static_cast<int32_t *>(at(p.rowmap));
  int32_t *pos = static_cast<int32_t *>(at(p.pos));
  if ((st = qmm_moe_bucket(T, KU, E, p.max_tiles, nullptr, ids, ti, rm, pos, stream))) return st;
  if (p.mx) {
    uint8_t *x8 = static_cast<uint8_t *>(at(p.xa)), *xs8 = static_cast<uint8_t *>(at(p.xs));
    uint8_t *a8 = static_cast<uint8_t *>(at(p.act)), *as8 = static_cast<uint8_t *>(at(p.as));
    if (!operand && (st = qmm_quant_mxfp8(T, H, x, x_dtype, nullptr, x8, xs8, stream))) return st;
    if ((st = qmm_moe_grouped_mxfp8(fmt, fused, act, E, KU, p.max_rows, H, FE, T, ti, rm, x8, xs8, w_gate, ws_gate,
                                    w_up, ws_up, bias_gate, bias_up, a8, as8, stream)))
      return st;
    st = qmm_moe_grouped(fmt, 1, 0, act, E, KU, p.max_rows, FE, H, p.max_rows, ti, rm, a8, QMM_MXFP8, as8, w_down,
                         ws_down, nullptr, nullptr, bias_down, nullptr, ys, stream);
  } else {
    void *x16 = at(p.xa), *a16 = at(p.a2);
    float *xsc = static_cast<float *>(at(p.xs)), *asc = static_cast<float *>(at(p.as));
    float *a = static_cast<float *>(at(p.act));
    if (!operand && (st = qmm_row_scale_f16(T, H, x, x_dtype, xsc, x16, nullptr, stream))) return st;
    if ((st = qmm_moe_grouped(fmt, 0, fused, act, E, KU, p.max_rows, H, FE, T, ti, rm, x16, QMM_F16, xsc, w_gate,
                              nullptr, w_up, nullptr, bias_gate, bias_up, a, stream)))
      return st;
    // the down GEMM's operand over the assignments' rows (the rows the tile-wise producer covers)
    if ((st = FE % 8 == 0 && FE <= 8192 ? qmm_row_scale_f16_rows(p.A, pos, FE, a, QMM_F32, asc, a16, stream)
                                         : qmm_row_scale_f16(p.max_rows, FE, a, QMM_F32, asc, a16, ti, stream)))
      return st;
    st = qmm_moe_grouped(fmt_down, 1, 0, act, E, KU, p.max_rows, FE, H, p.max_rows, ti, rm, a16, QMM_F16, asc,
                         w_down, nullptr, nullptr, nullptr, bias_down, nullptr, ys, stream);
  }
  if (st) return st;
  return sg ? qmm_moe_combine_gated(T, p.max_rows, H, KU, ys, pos, wts, sg, y, stream)
            : qmm_moe_combine(T, p.max_rows, H, KU, ys, pos, wts, accumulate, y, stream);
}
