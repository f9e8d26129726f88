// Decode matvecs with fused weight dequantization:
//   qmm_mv             y[t, r] (+)= sum_k x[t, k] W[r, k]        g_mv_{fmt}_k{K}[_t{TG}][_r{R}], S/gen_llm.py:1159-1378
//   qmm_moe_expert_mv  gu: act[a] = act(Wg[e] x[a/KU], Wu[e] x[a/KU]); dn: ys[a] = Wd[e] x[a]
//                                                                 g_moe_gu_* / g_moe_dn_*, S/gen_moe.py:535-727
//   qmm_moe_expert_mv_combine  the dn matvecs and the combine in one launch     + g_moe_combine, S/gen_moe.py:730-762
//
// Launch shape (wave64): a workgroup is 4 waves, each wave owns RW consecutive weight rows. A wave walks the row
// in passes of 64 items (rowdot.hpp), keeps the lane's activation fragments of its TG tokens in registers for all
// RW rows, issues every row's 128-bit loads before the math, and folds each row's 64 lane partials with a
// butterfly. Every token runs the same per-lane arithmetic and the same butterfly, so a call's result for one
// token does not depend on how many tokens the call carries (multi-token == one-token, bit for bit).
#include <type_traits>

#include "rowdot.hpp"
#include "topk.hpp"

using namespace qmm;

namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kRW = 4;
// Output rows a wave of the expert matvecs: four weight rows in flight a wave, i.e. two gate / up row pairs for
// gate/up (measured: MXFP4 gpt-oss-20b T = 1 gate/up 11.5 -> 10.4 us, Q4_K Qwen3-30B-A3B 10.6 -> 8.5 us; the down
// matvec is slower with two rows and with eight)
template <bool GU>
constexpr int expert_rw() { return GU ? 2 : 4; }

template <int RW, int TG>
__device__ __forceinline__ void reduce_all(float (&acc)[RW][TG]) {
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int t = 0; t < TG; ++t) acc[r][t] = wave_sum(acc[r][t]);
}

template <class P, int TG, int RW>
__global__ __launch_bounds__(256) void mv_kernel(int64_t n, int64_t tokens, int64_t k, int accumulate,
                                                 const u8 *__restrict__ x, int64_t x_row_bytes,
                                                 const u8 *__restrict__ w, const u8 *__restrict__ ws, int64_t rb,
                                                 int64_t srb, float *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * TG;
  const int64_t row0 = ((int64_t)blockIdx.y * kWavesPerBlock + wave) * RW;
  if (row0 >= n) return;
  const int nitems = P::items(k);
  float acc[RW][TG];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int t = 0; t < TG; ++t) acc[r][t] = 0.f;

  for (int it0 = 0; it0 < nitems; it0 += 64) {
    const int item = it0 + lane;
    const bool live = item < nitems;
    typename P::X xs[TG];
#pragma unroll
    for (int t = 0; t < TG; ++t) P::load_x(x + (t0 + t) * x_row_bytes, item, live && (t0 + t) < tokens, xs[t]);
    typename P::W wv[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r)
      P::load_w(w + (row0 + r) * rb, ws + (row0 + r) * srb, item, live && (row0 + r) < n, wv[r]);
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int t = 0; t < TG; ++t) acc[r][t] += P::dot(wv[r], xs[t], item);
  }
  reduce_all<RW, TG>(acc);
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      const int64_t row = row0 + r, tok = t0 + t;
      if (lane == r * TG + t && row < n && tok < tokens) {
        float *p = y + tok * n + row;
        *p = accumulate ? *p + acc[r][t] : acc[r][t];
      }
    }
}

// One assignment per workgroup row (blockIdx.x), RW output rows per wave. LPR lanes a row (the row's item count
// rounded up to a power of two, at least 64 / RW): lane (group rg, sub) takes items sub, sub + LPR, ... of rows
// rg, rg + 64 / LPR, ... of the wave's RW, and a row's LPR lanes meet in the butterfly of wave_sum restricted to
// their group. With one item a lane up to LPR items, the lanes a full-wave butterfly would add past the group hold
// zeros, so the row sums are the same for every LPR.
template <class P, int RW, bool GU, int NS = 0, int LPR = 64>
__global__ __launch_bounds__(256) void expert_mv_kernel(int64_t n, int64_t assignments, int KU, int E, int64_t k,
                                                        const int32_t *__restrict__ ids, const u8 *__restrict__ x,
                                                        int64_t x_row_bytes, const u8 *__restrict__ w,
                                                        const u8 *__restrict__ ws, const u8 *__restrict__ w2,
                                                        const u8 *__restrict__ ws2, int64_t rb, int64_t srb,
                                                        int64_t ebytes, int64_t esbytes, const float *__restrict__ bias,
                                                        const float *__restrict__ bias2, int act, int accumulate,
                                                        float *__restrict__ y, RouteArgs route = {}) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t a = blockIdx.x;
  const int64_t row0 = ((int64_t)blockIdx.y * kWavesPerBlock + wave) * RW;
  if constexpr (NS > 0) {
    if (a >= assignments) return;
  } else {
    if (row0 >= n || a >= assignments) return;
  }
  int e;
  if constexpr (NS > 0) {
    __shared__ __align__(16) uint64_t keys[kWavesPerBlock][64 * NS];
    int rank[NS];
    float wo[NS];
    bool pick[NS];
    const int64_t t = a / KU;
    topk_select<NS>(route.logits + t * E, E, KU, route.gating, route.norm, route.scale, route.bias, keys[wave], rank,
                    wo, pick);
    float wt;
    topk_pick<NS>(rank, wo, pick, (int)(a % KU), e, wt);
    if (blockIdx.y == 0 && wave == 0 && lane == 0) {
      route.ids[a] = e;
      route.wts[a] = wt;
    }
    if (row0 >= n) return;
  } else {
    e = ids ? ids[a] : 0;                    // no ids: one expert (the dense swiglu matvec)
  }
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);   // ids are clamped into range as the reference does (S/gen_moe.py:592-596)
  const u8 *xr = x + (GU ? a / KU : a) * x_row_bytes;
  const u8 *we = w + e * ebytes, *wse = ws + e * esbytes;
  const u8 *w2e = w2 + e * ebytes, *ws2e = ws2 + e * esbytes;
  const int nitems = P::items(k);
  constexpr int G = 64 / LPR, RL = RW / G;   // row groups a wave, rows a lane
  static_assert(RL >= 1 && RW % G == 0, "LPR below 64 / RW");
  const int sub = lane % LPR, rg = lane / LPR;
  float ag[RL], au[RL];
#pragma unroll
  for (int r = 0; r < RL; ++r) ag[r] = au[r] = 0.f;
  for (int it0 = 0; it0 < nitems; it0 += LPR) {
    const int item = it0 + sub;
    const bool live = item < nitems;
    typename P::X xs;
    P::load_x(xr, item, live, xs);
    typename P::W wg[RL], wu[GU ? RL : 1];
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int64_t row = row0 + rg + G * r;
      const bool rl = live && row < n;
      P::load_w(we + row * rb, wse + row * srb, item, rl, wg[r]);
      if constexpr (GU) P::load_w(w2e + row * rb, ws2e + row * srb, item, rl, wu[r]);
    }
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      ag[r] += P::dot(wg[r], xs, item);
      if constexpr (GU) au[r] += P::dot(wu[r], xs, item);
    }
  }
#pragma unroll
  for (int r = 0; r < RL; ++r)
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) {
      ag[r] += __shfl_xor(ag[r], off, kWave);
      if constexpr (GU) au[r] += __shfl_xor(au[r], off, kWave);
    }
#pragma unroll
  for (int r = 0; r < RL; ++r) {
    const int64_t row = row0 + rg + G * r;
    if (sub == 0 && row < n) {
      float g = ag[r];
      if (bias) g += bias[e * n + row];
      float v = g;
      if constexpr (GU) {
        float u = au[r];
        if (bias2) u += bias2[e * n + row];
        v = act_fn(act, g, u);
      }
      y[a * n + row] = accumulate ? y[a * n + row] + v : v;
    }
  }
}

// The gate/up expert matvecs with gate and up in different formats (the reference's "GATE+UP" expert tensors,
// g_moe_gu_{fg}_{fu}_k{K}_r{R}, S/gen_moe.py:535-552; with no ids one expert: the dense swiglu matvec): the gate
// rows are walked in the gate format's items and the up rows in the up format's, each with the one-format kernel's
// per-lane arithmetic and butterfly, then act_fn(g + bg, u + bu) as there.
template <class PG, class PU, int RW>
__global__ __launch_bounds__(256) void expert_mv_mixed_kernel(int64_t n, int64_t assignments, int KU, int E, int64_t k,
                                                              const int32_t *__restrict__ ids, const u8 *__restrict__ x,
                                                              int64_t x_row_bytes, const u8 *__restrict__ w,
                                                              const u8 *__restrict__ w2, int64_t rbg, int64_t rbu,
                                                              const float *__restrict__ bias,
                                                              const float *__restrict__ bias2, int act, int accumulate,
                                                              float *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t a = blockIdx.x;
  const int64_t row0 = ((int64_t)blockIdx.y * kWavesPerBlock + wave) * RW;
  if (row0 >= n || a >= assignments) return;
  int e = ids ? ids[a] : 0;
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);
  const u8 *xr = x + (a / KU) * x_row_bytes;
  const u8 *we = w + e * (rbg * n), *w2e = w2 + e * (rbu * n);
  float ag[RW], au[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) ag[r] = au[r] = 0.f;
  const int ng = PG::items(k), nu = PU::items(k);
  for (int it0 = 0; it0 < ng; it0 += 64) {
    const int item = it0 + lane;
    const bool live = item < ng;
    typename PG::X xs;
    PG::load_x(xr, item, live, xs);
    typename PG::W wg[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) PG::load_w(we + (row0 + r) * rbg, we, item, live && (row0 + r) < n, wg[r]);
#pragma unroll
    for (int r = 0; r < RW; ++r) ag[r] += PG::dot(wg[r], xs, item);
  }
  for (int it0 = 0; it0 < nu; it0 += 64) {
    const int item = it0 + lane;
    const bool live = item < nu;
    typename PU::X xs;
    PU::load_x(xr, item, live, xs);
    typename PU::W wu[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) PU::load_w(w2e + (row0 + r) * rbu, w2e, item, live && (row0 + r) < n, wu[r]);
#pragma unroll
    for (int r = 0; r < RW; ++r) au[r] += PU::dot(wu[r], xs, item);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    ag[r] = wave_sum(ag[r]);
    au[r] = wave_sum(au[r]);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int64_t row = row0 + r;
    if (lane == r && row < n) {
      float g = ag[r], u = au[r];
      if (bias) g += bias[e * n + row];
      if (bias2) u += bias2[e * n + row];
      const float v = act_fn(act, g, u);
      y[a * n + row] = accumulate ? y[a * n + row] + v : v;
    }
  }
}

// The decode chain's down matvecs and combine in one launch: workgroup (row block, token t) runs one wave per
// routed slot j of t, all over the same RW rows. Each wave does expert_mv_kernel's per-lane arithmetic and
// butterfly for its assignment t*KU + j (so its row sums are the separate call's ys, bit for bit); one lane a
// row then folds the KU sums with the combine's fma chain in slot order.
template <class P, int RW, int LPR = 64>
__global__ __launch_bounds__(512) void expert_mv_combine_kernel(int64_t n, int KU, int E, int64_t k,
                                                                const int32_t *__restrict__ ids,
                                                                const float *__restrict__ wts,
                                                                const u8 *__restrict__ x, int64_t x_row_bytes,
                                                                const u8 *__restrict__ w, const u8 *__restrict__ ws,
                                                                int64_t rb, int64_t srb, int64_t ebytes,
                                                                int64_t esbytes, const float *__restrict__ bias,
                                                                int accumulate, const float *__restrict__ sg,
                                                                float *__restrict__ y) {
  __shared__ float part[8][RW];
  __shared__ float slot_w[8];
  const int lane = threadIdx.x & 63;
  const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: ids / wts / expert in SGPRs
  const int64_t t = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * RW;
  const int64_t a = t * KU + j;
  int e = ids[a];
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);
  const float wj = wts[a];
  // the combine's starting value, loaded ahead of the weights (lane r: row row0 + r)
  float y0 = 0.f;
  if (accumulate && j == 0 && lane < RW && row0 + lane < n) {
    y0 = y[t * n + row0 + lane];
    if (sg) y0 = y0 * sg[t];
  }
  const u8 *xr = x + a * x_row_bytes;
  const u8 *we = w + e * ebytes, *wse = ws + e * esbytes;
  const int nitems = P::items(k);
  constexpr int G = 64 / LPR, RL = RW / G;   // row groups a wave, rows a lane (expert_mv_kernel's lane map)
  static_assert(RL >= 1 && RW % G == 0, "LPR below 64 / RW");
  const int sub = lane % LPR, rg = lane / LPR;
  float ag[RL];
#pragma unroll
  for (int r = 0; r < RL; ++r) ag[r] = 0.f;
  for (int it0 = 0; it0 < nitems; it0 += LPR) {
    const int item = it0 + sub;
    const bool live = item < nitems;
    typename P::X xs;
    P::load_x(xr, item, live, xs);
    typename P::W wg[RL];
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int64_t row = row0 + rg + G * r;
      P::load_w(we + row * rb, wse + row * srb, item, live && row < n, wg[r]);
    }
#pragma unroll
    for (int r = 0; r < RL; ++r) ag[r] += P::dot(wg[r], xs, item);
  }
#pragma unroll
  for (int r = 0; r < RL; ++r)
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) ag[r] += __shfl_xor(ag[r], off, kWave);
#pragma unroll
  for (int r = 0; r < RL; ++r) {
    const int rl = rg + G * r;   // the row's place in the workgroup's RW
    const int64_t row = row0 + rl;
    if (sub == 0) {
      float g = ag[r];
      if (bias && row < n) g += bias[e * n + row];
      part[j][rl] = g;
    }
  }
  if (lane == 0) slot_w[j] = wj;
  __syncthreads();
  if (threadIdx.x < RW && row0 + threadIdx.x < n) {
    float acc = y0;
    for (int i = 0; i < KU; ++i) acc = __builtin_fmaf(slot_w[i], part[i][threadIdx.x], acc);
    y[t * n + row0 + threadIdx.x] = acc;
  }
}

template <class P, int TG>
int launch_mv(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int64_t x_row_bytes,
              const void *w, const void *ws, int64_t rb, int64_t srb, float *y, hipStream_t s) {
  const dim3 grid((unsigned)((tokens + TG - 1) / TG), (unsigned)((n + kWavesPerBlock * kRW - 1) / (kWavesPerBlock * kRW)));
  mv_kernel<P, TG, kRW><<<grid, 256, 0, s>>>(n, tokens, k, accumulate, static_cast<const u8 *>(x), x_row_bytes,
                                            static_cast<const u8 *>(w), static_cast<const u8 *>(ws), rb, srb, y);
  return launch_status();
}

// token group: 4 (bf16 activations) or 2 (f32 activations) tokens share every weight load
template <template <bool> class P>
int dispatch_mv(bool bf, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w,
                const void *ws, int64_t rb, int64_t srb, float *y, hipStream_t s) {
  if (bf) {
    const int64_t xb = k * 2;
    if (tokens >= 4) return launch_mv<P<true>, 4>(k, n, tokens, accumulate, x, xb, w, ws, rb, srb, y, s);
    if (tokens >= 2) return launch_mv<P<true>, 2>(k, n, tokens, accumulate, x, xb, w, ws, rb, srb, y, s);
    return launch_mv<P<true>, 1>(k, n, tokens, accumulate, x, xb, w, ws, rb, srb, y, s);
  }
  const int64_t xb = k * 4;
  if (tokens >= 2) return launch_mv<P<false>, 2>(k, n, tokens, accumulate, x, xb, w, ws, rb, srb, y, s);
  return launch_mv<P<false>, 1>(k, n, tokens, accumulate, x, xb, w, ws, rb, srb, y, s);
}

template <bool B> using MXG = MXFP4<B, false>;
template <bool B> using MXS = MXFP4<B, true>;

// no GEMV here on the tiled layouts (the grouped GEMM's MXFP4 tiles; tiled Q4_K has its own int8 GEMV)
bool valid_fmt(int fmt) { return (fmt >= QMM_Q4_0 && fmt <= QMM_MXFP4S) || fmt == QMM_Q6_K; }

// Alignment the row engine needs: 16-byte rows for Q4_K / MXFP4S, 4-byte rows for Q4_0 pairs, a 4-byte aligned
// tensor for Q6_K (its 210-byte super-blocks then start on even addresses the loader can realign).
int check_weights(int fmt, int64_t k, const void *w, const void *ws) {
  if (!w || (fmt == QMM_MXFP4S && !ws)) return QMM_ERR_NULL;
  if (fmt == QMM_Q4_0 && k % 64) return QMM_ERR_SHAPE;
  if ((fmt == QMM_Q4_K || fmt == QMM_MXFP4S) && !aligned(w, 16)) return QMM_ERR_ALIGN;
  if ((fmt == QMM_Q4_0 || fmt == QMM_Q6_K) && !aligned(w, 4)) return QMM_ERR_ALIGN;
  return QMM_OK;
}

}  // namespace

int qmm_mv_q4k_fast(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w, float *y,
                    hipStream_t s);
int qmm_topk_expert_mv_tiled(const RouteArgs &r, int E, int KU, int64_t tokens, int fused, int act, int64_t k,
                             int64_t n, const void *x, int x_dtype, const void *w, const void *ws, const void *w2,
                             const void *ws2, const float *bias, const float *bias2, float *y, hipStream_t s);
int qmm_expert_mv_combine_tiled(int64_t k, int64_t n, int E, int KU, int64_t tokens, const int32_t *ids,
                                const float *wts, const void *x, int x_dtype, const void *w, const void *ws,
                                const float *bias, int accumulate, const float *sg, float *y, hipStream_t s);

int qmm_mv_q40t_f32(int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype, const void *w,
                    float *y, hipStream_t s);

extern "C" int qmm_mv(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                      const void *w, const void *ws, float *y, qmm_stream_t stream) {
  if (fmt == QMM_Q4_0T) {   // the tiled Q4_0 units of qmm_tile_q40 (gemv_q4kt.hip)
    if (!x || !w || !y) return QMM_ERR_NULL;
    if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
    if (n <= 0 || tokens <= 0 || k <= 0 || n > (1ll << 30) || k > (1ll << 20)) return QMM_ERR_SHAPE;
    if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
    return qmm_mv_q40t_f32(k, n, tokens, accumulate, x, x_dtype, w, y, reinterpret_cast<hipStream_t>(stream));
  }
  if (!valid_fmt(fmt)) return QMM_ERR_FORMAT;
  if (!x || !y) return QMM_ERR_NULL;
  if (n <= 0 || tokens <= 0 || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (n > (1ll << 30) || tokens > (1ll << 20) || k > (1ll << 24)) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (int st = check_weights(fmt, k, w, ws)) return st;
  if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  const int64_t rb = row_bytes(fmt, k), srb = fmt == QMM_MXFP4S ? k / 32 : 0;
  switch (fmt) {
    case QMM_Q4_K:
      if (bf) {
        const int st = qmm_mv_q4k_fast(k, n, tokens, accumulate, x, w, y, s);
        if (st != 1) return st;
      }
      return dispatch_mv<Q4K>(bf, k, n, tokens, accumulate, x, w, w, rb, 0, y, s);
    case QMM_Q4_0: return dispatch_mv<Q40>(bf, k, n, tokens, accumulate, x, w, w, rb, 0, y, s);
    case QMM_Q6_K: return dispatch_mv<Q6K>(bf, k, n, tokens, accumulate, x, w, w, rb, 0, y, s);
    case QMM_MXFP4: return dispatch_mv<MXG>(bf, k, n, tokens, accumulate, x, w, w, rb, 0, y, s);
    default: return dispatch_mv<MXS>(bf, k, n, tokens, accumulate, x, w, ws, rb, srb, y, s);
  }
}

namespace {
// Lanes a row for the expert matvecs: the item count rounded up to a power of two, at least 64 / RW
inline int expert_lpr(int items, int rw) {
  int l = items <= 16 ? 16 : (items <= 32 ? 32 : 64);
  return l < 64 / rw ? 64 / rw : l;
}
// the kernel instantiation for lpr; MAXL: the largest lpr the caller's rows can have (no kernel is built past it)
template <int RW, int MAXL = 64, class F>
int with_lpr(int lpr, F &&f) {
  if constexpr (64 / RW <= 16) { if (lpr == 16) return f(std::integral_constant<int, 16>{}); }
  if constexpr (MAXL == 32) return f(std::integral_constant<int, 32>{});
  else {
    if constexpr (64 / RW <= 32) { if (lpr == 32) return f(std::integral_constant<int, 32>{}); }
    return f(std::integral_constant<int, 64>{});
  }
}

template <class P, bool GU>
int launch_expert(int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids, const void *x,
                  int64_t x_row_bytes, const void *w, const void *ws, const void *w2, const void *ws2, int64_t rb,
                  int64_t srb, int64_t ebytes, int64_t esbytes, const float *bias, const float *bias2, int act,
                  float *y, hipStream_t s, int accumulate = 0) {
  constexpr int RW = expert_rw<GU>();
  const dim3 grid((unsigned)assignments, (unsigned)((n + kWavesPerBlock * RW - 1) / (kWavesPerBlock * RW)));
  return with_lpr<RW>(expert_lpr(P::items(k), RW), [&](auto lc) {
    expert_mv_kernel<P, RW, GU, 0, decltype(lc)::value><<<grid, 256, 0, s>>>(
        n, assignments, KU, E, k, ids, static_cast<const u8 *>(x), x_row_bytes, static_cast<const u8 *>(w),
        static_cast<const u8 *>(ws), static_cast<const u8 *>(w2), static_cast<const u8 *>(ws2), rb, srb, ebytes,
        esbytes, bias, bias2, act, accumulate, y);
    return launch_status();
  });
}

// The gate/up expert matvecs routing their own tokens (NS = ceil(E / 64) key slots a lane).
template <class P, int NS>
int launch_expert_route(int64_t k, int64_t n, int E, int KU, int64_t assignments, const RouteArgs &r, const void *x,
                        int64_t x_row_bytes, const void *w, const void *ws, const void *w2, const void *ws2,
                        int64_t rb, int64_t srb, int64_t ebytes, int64_t esbytes, const float *bias,
                        const float *bias2, int act, float *y, hipStream_t s) {
  constexpr int RW = expert_rw<true>();
  const dim3 grid((unsigned)assignments, (unsigned)((n + kWavesPerBlock * RW - 1) / (kWavesPerBlock * RW)));
  return with_lpr<RW>(expert_lpr(P::items(k), RW), [&](auto lc) {
    expert_mv_kernel<P, RW, true, NS, decltype(lc)::value><<<grid, 256, 0, s>>>(
        n, assignments, KU, E, k, nullptr, static_cast<const u8 *>(x), x_row_bytes, static_cast<const u8 *>(w),
        static_cast<const u8 *>(ws), static_cast<const u8 *>(w2), static_cast<const u8 *>(ws2), rb, srb, ebytes,
        esbytes, bias, bias2, act, 0, y, r);
    return launch_status();
  });
}

template <template <bool> class P>
int dispatch_route(bool bf, int64_t k, int64_t n, int E, int KU, int64_t assignments, const RouteArgs &r,
                   const void *x, const void *w, const void *ws, const void *w2, const void *ws2, int64_t rb,
                   int64_t srb, int64_t ebytes, int64_t esbytes, const float *bias, const float *bias2, int act,
                   float *y, hipStream_t s) {
  const int64_t xb = k * (bf ? 2 : 4);
#define QMM_ROUTE(NS)                                                                                                \
  (bf ? launch_expert_route<P<true>, NS>(k, n, E, KU, assignments, r, x, xb, w, ws, w2, ws2, rb, srb, ebytes,        \
                                         esbytes, bias, bias2, act, y, s)                                             \
      : launch_expert_route<P<false>, NS>(k, n, E, KU, assignments, r, x, xb, w, ws, w2, ws2, rb, srb, ebytes,       \
                                          esbytes, bias, bias2, act, y, s))
  if (E <= 64) return QMM_ROUTE(1);
  if (E <= 128) return QMM_ROUTE(2);
  if (E <= 192) return QMM_ROUTE(3);
  return QMM_ROUTE(4);
#undef QMM_ROUTE
}

// The dense swiglu matvec: the gate/up expert kernel with one expert (no ids) and one token a row of x.
template <template <bool> class P>
int launch_swiglu(bool bf, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, const void *w,
                  const void *w2, int64_t rb, float *y, hipStream_t s) {
  const int64_t xb = k * (bf ? 2 : 4);
  if (bf)
    return launch_expert<P<true>, true>(k, n, 1, 1, tokens, nullptr, x, xb, w, w, w2, w2, rb, 0, rb * n, 0, nullptr,
                                        nullptr, QMM_ACT_SILU, y, s, accumulate);
  return launch_expert<P<false>, true>(k, n, 1, 1, tokens, nullptr, x, xb, w, w, w2, w2, rb, 0, rb * n, 0, nullptr,
                                       nullptr, QMM_ACT_SILU, y, s, accumulate);
}

template <template <bool> class P>
int dispatch_expert(bool gu, bool bf, int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids,
                    const void *x, const void *w, const void *ws, const void *w2, const void *ws2, int64_t rb,
                    int64_t srb, int64_t ebytes, int64_t esbytes, const float *bias, const float *bias2, int act,
                    float *y, hipStream_t s) {
  const int64_t xb = k * (bf ? 2 : 4);
  if (gu) {
    return bf ? launch_expert<P<true>, true>(k, n, E, KU, assignments, ids, x, xb, w, ws, w2, ws2, rb, srb, ebytes, esbytes, bias, bias2, act, y, s)
              : launch_expert<P<false>, true>(k, n, E, KU, assignments, ids, x, xb, w, ws, w2, ws2, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
  }
  return bf ? launch_expert<P<true>, false>(k, n, E, KU, assignments, ids, x, xb, w, ws, w2, ws2, rb, srb, ebytes, esbytes, bias, bias2, act, y, s)
            : launch_expert<P<false>, false>(k, n, E, KU, assignments, ids, x, xb, w, ws, w2, ws2, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
}

template <class PG, class PU>
int launch_mixed(int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids, const void *x,
                 int64_t x_row_bytes, const void *w, const void *w2, int64_t rbg, int64_t rbu, const float *bias,
                 const float *bias2, int act, int accumulate, float *y, hipStream_t s) {
  constexpr int RW = expert_rw<true>();
  const dim3 grid((unsigned)assignments, (unsigned)((n + kWavesPerBlock * RW - 1) / (kWavesPerBlock * RW)));
  expert_mv_mixed_kernel<PG, PU, RW><<<grid, 256, 0, s>>>(
      n, assignments, KU, E, k, ids, static_cast<const u8 *>(x), x_row_bytes, static_cast<const u8 *>(w),
      static_cast<const u8 *>(w2), rbg, rbu, bias, bias2, act, accumulate, y);
  return launch_status();
}

// gate format PG, then the up format from its code (GGUF blocks: Q4_0, Q4_K, Q6_K, MXFP4)
template <template <bool> class PG, bool B>
int dispatch_mixed_up(int fu, int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids,
                      const void *x, const void *w, const void *w2, int64_t rbg, int64_t rbu, const float *bias,
                      const float *bias2, int act, int accumulate, float *y, hipStream_t s) {
  const int64_t xb = k * (B ? 2 : 4);
  switch (fu) {
    case QMM_Q4_K: return launch_mixed<PG<B>, Q4K<B>>(k, n, E, KU, assignments, ids, x, xb, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    case QMM_Q6_K: return launch_mixed<PG<B>, Q6K<B>>(k, n, E, KU, assignments, ids, x, xb, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    case QMM_Q4_0: return launch_mixed<PG<B>, Q40<B>>(k, n, E, KU, assignments, ids, x, xb, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    default: return launch_mixed<PG<B>, MXG<B>>(k, n, E, KU, assignments, ids, x, xb, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
  }
}

template <bool B>
int dispatch_mixed(int fg, int fu, int64_t k, int64_t n, int E, int KU, int64_t assignments, const int32_t *ids,
                   const void *x, const void *w, const void *w2, const float *bias, const float *bias2, int act,
                   int accumulate, float *y, hipStream_t s) {
  const int64_t rbg = row_bytes(fg, k), rbu = row_bytes(fu, k);
  switch (fg) {
    case QMM_Q4_K: return dispatch_mixed_up<Q4K, B>(fu, k, n, E, KU, assignments, ids, x, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    case QMM_Q6_K: return dispatch_mixed_up<Q6K, B>(fu, k, n, E, KU, assignments, ids, x, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    case QMM_Q4_0: return dispatch_mixed_up<Q40, B>(fu, k, n, E, KU, assignments, ids, x, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
    default: return dispatch_mixed_up<MXG, B>(fu, k, n, E, KU, assignments, ids, x, w, w2, rbg, rbu, bias, bias2, act, accumulate, y, s);
  }
}

// the formats a mixed gate/up pair takes: GGUF blocks (each matrix read in place)
bool mixed_fmt_ok(int f) { return f == QMM_Q4_0 || f == QMM_Q4_K || f == QMM_Q6_K || f == QMM_MXFP4; }

template <template <bool> class P, int RW>
int launch_expert_combine_rw(bool bf, int64_t k, int64_t n, int E, int KU, int64_t tokens, const int32_t *ids,
                             const float *wts, const void *x, const void *w, const void *ws, int64_t rb, int64_t srb,
                             const float *bias, int accumulate, const float *sg, float *y, hipStream_t s) {
  const dim3 grid((unsigned)((n + RW - 1) / RW), (unsigned)tokens);
  const int64_t xb = k * (bf ? 2 : 4);
  const u8 *xp = static_cast<const u8 *>(x), *wp = static_cast<const u8 *>(w), *wsp = static_cast<const u8 *>(ws);
  // eight rows a wave only for rows of at most 32 items (launch_expert_combine)
  return with_lpr<RW, RW == 8 ? 32 : 64>(expert_lpr(P<false>::items(k), RW), [&](auto lc) {
    constexpr int L = decltype(lc)::value;
    if (bf)
      expert_mv_combine_kernel<P<true>, RW, L><<<grid, 64 * KU, 0, s>>>(n, KU, E, k, ids, wts, xp, xb, wp, wsp, rb,
                                                                       srb, rb * n, srb * n, bias, accumulate, sg, y);
    else
      expert_mv_combine_kernel<P<false>, RW, L><<<grid, 64 * KU, 0, s>>>(n, KU, E, k, ids, wts, xp, xb, wp, wsp, rb,
                                                                        srb, rb * n, srb * n, bias, accumulate, sg, y);
    return launch_status();
  });
}

// Rows a wave: four, or eight where one pass over a row keeps at most half the wave's lanes busy (Q4_K FE = 768:
// 12 items a row), so each lane has twice the weight loads in flight (measured: Qwen3-30B-A3B Q4_K decode chain at
// one token 26.3 -> 24.8 us, at eight 149.8 -> 140.3 us; gpt-oss-20b MXFP4, 90 items a row, is slower with eight).
template <template <bool> class P>
int launch_expert_combine(bool bf, int64_t k, int64_t n, int E, int KU, int64_t tokens, const int32_t *ids,
                          const float *wts, const void *x, const void *w, const void *ws, int64_t rb, int64_t srb,
                          const float *bias, int accumulate, const float *sg, float *y, hipStream_t s) {
  if (P<false>::items(k) <= 32)
    return launch_expert_combine_rw<P, 8>(bf, k, n, E, KU, tokens, ids, wts, x, w, ws, rb, srb, bias, accumulate, sg, y, s);
  return launch_expert_combine_rw<P, 4>(bf, k, n, E, KU, tokens, ids, wts, x, w, ws, rb, srb, bias, accumulate, sg, y, s);
}
}  // namespace

// ws / ws2: for QMM_MXFP4S the scale planes come through `w2`-style pairing: w = nibble plane, bias slots unchanged.
// The split-plane expert tensors are passed as w (nibbles [E, rows, k/2]) with their scale planes in ws.
extern "C" int qmm_moe_expert_mv_split(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                       int64_t assignments, const int32_t *ids, const void *x, int x_dtype,
                                       const void *w, const void *ws, const void *w2, const void *ws2,
                                       const float *bias, const float *bias2, float *y, qmm_stream_t stream);

static int expert_mv_impl(int fmt, int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                          int64_t assignments, const int32_t *ids, const void *x, int x_dtype, const void *w,
                          const void *ws, const void *w2, const void *ws2, const float *bias, const float *bias2,
                          float *y, qmm_stream_t stream) {
  if (fmt_code_ok(fmt) && fmt_mixed(fmt)) {
    // QMM_GATE_UP(gate, up): gate/up only (the down matvec has one matrix), two tensors (a fused gate_up tensor has
    // one format)
    const int fg = fmt_gate(fmt), fu = fmt_up(fmt);
    if (!mixed_fmt_ok(fg) || !mixed_fmt_ok(fu) || mode != 0 || fused) return QMM_ERR_FORMAT;
    if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
    if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
    if (!ids || !x || !y || !w || !w2) return QMM_ERR_NULL;
    if (n <= 0 || assignments <= 0 || assignments > (1 << 24) || assignments % KU || row_bytes(fg, k) == 0 ||
        row_bytes(fu, k) == 0)
      return QMM_ERR_SHAPE;
    if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
    if (int st = check_weights(fg, k, w, nullptr)) return st;
    if (int st = check_weights(fu, k, w2, nullptr)) return st;
    if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return x_dtype == QMM_BF16
               ? dispatch_mixed<true>(fg, fu, k, n, E, KU, assignments, ids, x, w, w2, bias, bias2, act, 0, y, s)
               : dispatch_mixed<false>(fg, fu, k, n, E, KU, assignments, ids, x, w, w2, bias, bias2, act, 0, y, s);
  }
  if (!valid_fmt(fmt)) return QMM_ERR_FORMAT;
  if (mode != 0 && mode != 1) return QMM_ERR_RANGE;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!ids || !x || !y) return QMM_ERR_NULL;
  if (n <= 0 || assignments <= 0 || assignments > (1 << 24) || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (mode == 0 && assignments % KU) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (int st = check_weights(fmt, k, w, ws)) return st;
  const bool gu = mode == 0;
  if (gu && !fused && (check_weights(fmt, k, w2, ws2) != QMM_OK)) return check_weights(fmt, k, w2, ws2);
  if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  const int64_t rb = row_bytes(fmt, k), srb = fmt == QMM_MXFP4S ? k / 32 : 0;
  const int64_t ebytes = rb * n * (fused && gu ? 2 : 1), esbytes = srb * n * (fused && gu ? 2 : 1);
  const void *wu = w2, *wsu = ws2;
  if (gu && fused) {   // one [E, 2n, k] tensor: expert e's n gate rows, then its n up rows (S/gen_moe.py:538)
    wu = static_cast<const u8 *>(w) + rb * n;
    wsu = fmt == QMM_MXFP4S ? static_cast<const u8 *>(ws) + srb * n : nullptr;
  }
  if (!gu) { wu = w; wsu = ws; }
  if (!wsu) wsu = wu;
  const void *wsg = ws ? ws : w;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  switch (fmt) {
    case QMM_Q4_K: return dispatch_expert<Q4K>(gu, bf, k, n, E, KU, assignments, ids, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_Q4_0: return dispatch_expert<Q40>(gu, bf, k, n, E, KU, assignments, ids, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_MXFP4: return dispatch_expert<MXG>(gu, bf, k, n, E, KU, assignments, ids, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_Q6_K: return dispatch_expert<Q6K>(gu, bf, k, n, E, KU, assignments, ids, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    default: return dispatch_expert<MXS>(gu, bf, k, n, E, KU, assignments, ids, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
  }
}

extern "C" int qmm_mv_swiglu(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x,
                             int x_dtype, const void *w, const void *w2, float *y, qmm_stream_t stream) {
  if (fmt_code_ok(fmt) && fmt_mixed(fmt)) {   // QMM_GATE_UP(gate, up): the gate and up matrices in their own formats
    const int fg = fmt_gate(fmt), fu = fmt_up(fmt);
    if (!mixed_fmt_ok(fg) || !mixed_fmt_ok(fu)) return QMM_ERR_FORMAT;
    if (!x || !w || !w2 || !y) return QMM_ERR_NULL;
    if (n <= 0 || tokens <= 0 || tokens > (1 << 24) || row_bytes(fg, k) == 0 || row_bytes(fu, k) == 0)
      return QMM_ERR_SHAPE;
    if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
    if (int st = check_weights(fg, k, w, nullptr)) return st;
    if (int st = check_weights(fu, k, w2, nullptr)) return st;
    if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return x_dtype == QMM_BF16
               ? dispatch_mixed<true>(fg, fu, k, n, 1, 1, tokens, nullptr, x, w, w2, nullptr, nullptr, QMM_ACT_SILU,
                                      accumulate, y, s)
               : dispatch_mixed<false>(fg, fu, k, n, 1, 1, tokens, nullptr, x, w, w2, nullptr, nullptr, QMM_ACT_SILU,
                                       accumulate, y, s);
  }
  if (fmt != QMM_Q4_0 && fmt != QMM_Q4_K && fmt != QMM_MXFP4 && fmt != QMM_Q6_K) return QMM_ERR_FORMAT;
  if (!x || !w || !w2 || !y) return QMM_ERR_NULL;
  if (n <= 0 || tokens <= 0 || tokens > (1 << 24) || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (int st = check_weights(fmt, k, w, nullptr)) return st;
  if (int st = check_weights(fmt, k, w2, nullptr)) return st;
  if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  const int64_t rb = row_bytes(fmt, k);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  switch (fmt) {
    case QMM_Q4_K: return launch_swiglu<Q4K>(bf, k, n, tokens, accumulate, x, w, w2, rb, y, s);
    case QMM_Q4_0: return launch_swiglu<Q40>(bf, k, n, tokens, accumulate, x, w, w2, rb, y, s);
    case QMM_Q6_K: return launch_swiglu<Q6K>(bf, k, n, tokens, accumulate, x, w, w2, rb, y, s);
    default: return launch_swiglu<MXG>(bf, k, n, tokens, accumulate, x, w, w2, rb, y, s);
  }
}

extern "C" int qmm_moe_expert_mv(int fmt, int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                 int64_t assignments, const int32_t *ids, const void *x, int x_dtype, const void *w,
                                 const void *w2, const float *bias, const float *bias2, float *y, qmm_stream_t stream) {
  if (fmt == QMM_MXFP4S) return QMM_ERR_FORMAT;   // split planes go through qmm_moe_expert_mv_split
  return expert_mv_impl(fmt, mode, fused, act, k, n, E, KU, assignments, ids, x, x_dtype, w, nullptr, w2, nullptr,
                        bias, bias2, y, stream);
}

extern "C" int qmm_moe_expert_mv_split(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                       int64_t assignments, const int32_t *ids, const void *x, int x_dtype,
                                       const void *w, const void *ws, const void *w2, const void *ws2,
                                       const float *bias, const float *bias2, float *y, qmm_stream_t stream) {
  return expert_mv_impl(QMM_MXFP4S, mode, fused, act, k, n, E, KU, assignments, ids, x, x_dtype, w, ws, w2, ws2,
                        bias, bias2, y, stream);
}

extern "C" int qmm_moe_topk_expert_mv(const float *logits, int64_t tokens, int E, int KU, int gating, int norm,
                                      float scale, const float *router_bias, int32_t *ids, float *wts, int fmt,
                                      int fused, int act, int64_t k, int64_t n, const void *x, int x_dtype,
                                      const void *w, const void *ws, const void *w2, const void *ws2,
                                      const float *bias, const float *bias2, float *y, qmm_stream_t stream) {
  // the routing's checks (qmm_moe_topk), then the gate/up matvec's (qmm_moe_expert_mv[_split], mode 0)
  if (!logits || !ids || !wts) return QMM_ERR_NULL;
  if (E <= 0 || E > 256 || KU <= 0 || KU > 8 || KU > E) return QMM_ERR_RANGE;
  if (gating < 1 || gating > 3 || (gating == 1 && router_bias)) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens * KU > (1 << 24)) return QMM_ERR_SHAPE;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (fmt == QMM_MXFP4T)   // the MFMA-tiled planes: expert_mv_tiled.hip
    return qmm_topk_expert_mv_tiled(RouteArgs{logits, gating, norm, scale, router_bias, ids, wts}, E, KU, tokens,
                                    fused, act, k, n, x, x_dtype, w, ws, w2, ws2, bias, bias2, y,
                                    reinterpret_cast<hipStream_t>(stream));
  if (!valid_fmt(fmt)) return QMM_ERR_FORMAT;
  if (!x || !y) return QMM_ERR_NULL;
  if (n <= 0 || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (int st = check_weights(fmt, k, w, ws)) return st;
  if (!fused && check_weights(fmt, k, w2, ws2) != QMM_OK) return check_weights(fmt, k, w2, ws2);
  if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  const int64_t rb = row_bytes(fmt, k), srb = fmt == QMM_MXFP4S ? k / 32 : 0;
  const int64_t ebytes = rb * n * (fused ? 2 : 1), esbytes = srb * n * (fused ? 2 : 1);
  const void *wu = w2, *wsu = ws2;
  if (fused) {   // one [E, 2n, k] tensor: expert e's n gate rows, then its n up rows (S/gen_moe.py:538)
    wu = static_cast<const u8 *>(w) + rb * n;
    wsu = fmt == QMM_MXFP4S ? static_cast<const u8 *>(ws) + srb * n : nullptr;
  }
  if (!wsu) wsu = wu;
  const void *wsg = fmt == QMM_MXFP4S ? ws : w;
  const RouteArgs r{logits, gating, norm, scale, router_bias, ids, wts};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  const int64_t A = tokens * KU;
  switch (fmt) {
    case QMM_Q4_K: return dispatch_route<Q4K>(bf, k, n, E, KU, A, r, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_Q4_0: return dispatch_route<Q40>(bf, k, n, E, KU, A, r, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_MXFP4: return dispatch_route<MXG>(bf, k, n, E, KU, A, r, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    case QMM_Q6_K: return dispatch_route<Q6K>(bf, k, n, E, KU, A, r, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
    default: return dispatch_route<MXS>(bf, k, n, E, KU, A, r, x, w, wsg, wu, wsu, rb, srb, ebytes, esbytes, bias, bias2, act, y, s);
  }
}

extern "C" int qmm_moe_expert_mv_combine(int fmt, int64_t k, int64_t n, int E, int KU, int64_t tokens,
                                         const int32_t *ids, const float *wts, const void *x, int x_dtype,
                                         const void *w, const void *ws, const float *bias, int accumulate,
                                         const float *sg, float *y, qmm_stream_t stream) {
  if (!valid_fmt(fmt) && fmt != QMM_MXFP4T) return QMM_ERR_FORMAT;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!ids || !wts || !x || !y) return QMM_ERR_NULL;
  if (n <= 0 || tokens <= 0 || tokens > 65535 || row_bytes(fmt, k) == 0) return QMM_ERR_SHAPE;
  if (fmt == QMM_MXFP4T)   // the MFMA-tiled planes: expert_mv_tiled.hip
    return qmm_expert_mv_combine_tiled(k, n, E, KU, tokens, ids, wts, x, x_dtype, w, ws, bias, sg ? 1 : accumulate, sg,
                                       y, reinterpret_cast<hipStream_t>(stream));
  if (n > (1ll << 30)) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (int st = check_weights(fmt, k, w, ws)) return st;
  if (!aligned(x, 16) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  if (sg) accumulate = 1;   // the gated combine: y = sg[t] y[t] + sum_j ...
  const int64_t rb = row_bytes(fmt, k), srb = fmt == QMM_MXFP4S ? k / 32 : 0;
  const void *wsp = fmt == QMM_MXFP4S ? ws : w;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  switch (fmt) {
    case QMM_Q4_K: return launch_expert_combine<Q4K>(bf, k, n, E, KU, tokens, ids, wts, x, w, wsp, rb, srb, bias, accumulate, sg, y, s);
    case QMM_Q4_0: return launch_expert_combine<Q40>(bf, k, n, E, KU, tokens, ids, wts, x, w, wsp, rb, srb, bias, accumulate, sg, y, s);
    case QMM_MXFP4: return launch_expert_combine<MXG>(bf, k, n, E, KU, tokens, ids, wts, x, w, wsp, rb, srb, bias, accumulate, sg, y, s);
    case QMM_Q6_K: return launch_expert_combine<Q6K>(bf, k, n, E, KU, tokens, ids, wts, x, w, wsp, rb, srb, bias, accumulate, sg, y, s);
    default: return launch_expert_combine<MXS>(bf, k, n, E, KU, tokens, ids, wts, x, w, wsp, rb, srb, bias, accumulate, sg, y, s);
  }
}
