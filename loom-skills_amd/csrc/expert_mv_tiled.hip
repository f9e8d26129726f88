// Decode expert matvecs on MXFP4 in MFMA-tiled planes (QMM_MXFP4T, qmm_tile_mxfp4), the layout the grouped prefill
// GEMM streams, so one copy of the expert weights serves prefill and decode:
//   gate/up          act[a, r] = act(Wg[e] x[a / KU] + bg[e, r], Wu[e] x[a / KU] + bu[e, r])
//   down             ys[a, r]  = Wd[e] x[a] + bd[e, r]          (g_moe_gu_* / g_moe_dn_*, S/gen_moe.py:535-727)
//   down + combine   y[t, r]   = y0 + sum_j w[t, j] (Wd[e_j] x[t KU + j] + bd[e_j, r])   (+ g_moe_combine,
//                    S/gen_moe.py:730-762; y0 = 0, y[t, r], or sg[t] y[t, r] for the gated combine)
// with e = clamp(ids[a], 0, E - 1) (S/gen_moe.py:592-596), or the expert the gate/up launch ranks itself from the
// token's logits (topk_select, the routing kernels' arithmetic).
//
// Launch shape: a workgroup owns one block of 32 output rows (one row of tiles) for one assignment (gate/up, down) or
// one token (down + combine: one group of waves per routed slot). Its waves split the K chunks (64 values: one 1 KB
// tile a matrix, lane l = 32 h + i holding row i's values 64 c + 32 h .. +31) in whole scale groups of four chunks, so
// a wave's scale dword j serves its chunks 4 j .. 4 j + 3. A wave issues its slice of the activation row, then the tile
// loads of all its chunks and their scale dwords, before any math; it stages the activations in its own LDS area and
// each lane accumulates its row over the wave's chunks with the split-plane expert matvec's per-block arithmetic (the
// fp4 pairs widened to bf16 against bf16 activation pairs in v_dot2_f32_bf16, or two fmas a pair on f32 activations,
// two partial sums, times the block's E8M0 scale). Lanes i and 32 + i then fold, and the waves' row sums are added in
// wave order in LDS. Every assignment runs the same arithmetic whatever the token count, so a multi-token call equals
// one-token calls bit for bit.
#include "rowdot.hpp"
#include "topk.hpp"

using namespace qmm;

namespace {

typedef __attribute__((ext_vector_type(4))) u32 v4u;

constexpr int kMaxW = 16;          // waves a workgroup
constexpr int kTile = 1024;        // bytes of one 32 x 64 fp4 tile
constexpr int kScaleGroup = 256;   // bytes of one scale group (4 chunks, 64 lanes x 4 bytes)

struct MxtArgs {
  int64_t n;                      // output rows, n % 32 == 0
  int C, C4;                      // K / 64 chunks, ceil(C / 4) scale groups
  int E, KU;
  int64_t rows;                   // assignments (gate/up, down) or tokens (down + combine)
  const int32_t *ids;             // [assignments] (NULL with the routing inside)
  const float *wts;               // combine weights [tokens, KU]
  const u8 *x;                    // activation rows [*, K], f32 or bf16
  const u8 *wg, *sg, *wu, *su;    // first row block of expert 0: gate (or down) tiles / scales, up tiles / scales
  int64_t e_rb;                   // row blocks an expert spans in the tensors
  const float *bias, *bias2;      // [E, n] or NULL
  int act, accumulate;
  const float *sgate;             // gated combine: y0 = sgate[t] y[t, r]
  float *y;
  RouteArgs route;
};

// The wave's K range in scale groups [g0, g1) of the slice `part` of `parts`, its chunks [4 g0, min(4 g1, C)).
__device__ __forceinline__ void wave_range(int part, int parts, int C, int C4, int &c0, int &c1) {
  const int g0 = part * C4 / parts, g1 = (part + 1) * C4 / parts;
  c0 = 4 * g0;
  c1 = min(4 * g1, C);
}

// One wave's dot products over chunks [c0, c1) of row block `rbi`, NM matrices (1: W; 2: gate and up), activation
// row xr, for the unit of RU = 32 / R rows rsel RU .. rsel RU + RU - 1 of the block: at step s lane l (h = l / 32)
// takes tile lane 32 h + rsel RU + l % RU of chunk R s + (l % 32) / RU, so one load instruction covers R chunks of the
// unit's rows. Returns the unit's row sums in lanes 0 .. RU - 1 of acc[]. MAXG scale groups (4 MAXG chunks) a batch;
// xl is the wave's LDS area of 4 MAXG chunks of activations.
template <bool BF, int NM, int MAXG, int R>
__device__ __forceinline__ void wave_dots(const MxtArgs &a, int64_t rbi, int rsel, const u8 *__restrict__ xr, int c0,
                                          int c1, u32 *xl, float (&acc)[NM]) {
  using P = MXFP4<BF, true>;
  constexpr int MAXC = 4 * MAXG;
  constexpr int RU = 32 / R;             // rows of the unit
  constexpr int XW = BF ? 32 : 64;       // dwords of one chunk's activations
  constexpr int PPC = XW / 4;            // 16-byte pieces of one chunk's activations
  const int lane = threadIdx.x & 63, h = lane >> 5, co = (lane & 31) / RU;
  const int tl = 32 * h + RU * rsel + (lane & (RU - 1));
  const u8 *tw[2] = {a.wg + rbi * a.C * kTile + 16 * tl, a.wu + rbi * a.C * kTile + 16 * tl};
  const u8 *ts[2] = {a.sg + rbi * a.C4 * kScaleGroup + 4 * tl, a.su + rbi * a.C4 * kScaleGroup + 4 * tl};
#pragma unroll
  for (int m = 0; m < NM; ++m) acc[m] = 0.f;
  for (int cb = c0; cb < c1; cb += MAXC) {
    const int nc = min(MAXC, c1 - cb);
    // activations of the batch's chunks first (L2-resident), then every weight tile and scale dword
    v4u xv[(MAXC * PPC + 63) / 64];
#pragma unroll
    for (int i = 0; i < (MAXC * PPC + 63) / 64; ++i) {
      const int p = lane + 64 * i;
      const int pc = p < nc * PPC ? p : 0;
      xv[i] = *reinterpret_cast<const v4u *>(xr + (int64_t)64 * cb * (BF ? 2 : 4) + 16 * pc);
    }
    v4u q[NM][MAXC / R];
    u32 sc[NM][MAXG];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
#pragma unroll
      for (int st = 0; st < MAXC / R; ++st) {
        const int i = R * st + co;
        const int c = cb + (i < nc ? i : nc - 1);
        q[m][st] = *reinterpret_cast<const v4u *>(tw[m] + (int64_t)c * kTile);
      }
#pragma unroll
      for (int j = 0; j < MAXG; ++j) {
        const int g = (cb >> 2) + (4 * j < nc ? j : 0);
        sc[m][j] = *reinterpret_cast<const u32 *>(ts[m] + (int64_t)g * kScaleGroup);
      }
    }
#pragma unroll
    for (int i = 0; i < (MAXC * PPC + 63) / 64; ++i) {
      const int p = lane + 64 * i;
      if (p < nc * PPC) *reinterpret_cast<v4u *>(xl + 4 * p) = xv[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int st = 0; st < MAXC / R; ++st) {
      if (R * st < nc) {   // some lane's chunk of this step is in the batch
        const int i = R * st + co;   // the lane's chunk in the batch
        typename P::X xs;
        const u32 *xc = xl + XW * (i < nc ? i : 0) + (XW / 2) * h;   // the lane's 32 values of chunk i
        if constexpr (BF) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const v4u v = *reinterpret_cast<const v4u *>(xc + 4 * j);
            xs.p[4 * j] = v.x; xs.p[4 * j + 1] = v.y; xs.p[4 * j + 2] = v.z; xs.p[4 * j + 3] = v.w;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const v4u v = *reinterpret_cast<const v4u *>(xc + 4 * j);
            xs.lo[2 * j] = u32_as_f32(v.x); xs.hi[2 * j] = u32_as_f32(v.y);
            xs.lo[2 * j + 1] = u32_as_f32(v.z); xs.hi[2 * j + 1] = u32_as_f32(v.w);
          }
        }
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          typename P::W w;
          w.q[0] = q[m][st].x; w.q[1] = q[m][st].y; w.q[2] = q[m][st].z; w.q[3] = q[m][st].w;
          w.e = (sc[m][(R * st) >> 2] >> (8 * (i & 3))) & 0xFFu;
          const float d = P::dot(w, xs, 0);
          if (i < nc) acc[m] += d;
        }
      }
    }
    if (cb + MAXC < c1) {   // the next batch overwrites the LDS area
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  // the lanes of one row: the two K halves of a chunk (lanes l, l ^ 32) and the R chunks of a step
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    acc[m] += __shfl_xor(acc[m], 32, 64);
#pragma unroll
    for (int off = RU; off < 32; off <<= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  }
}

template <bool BF, int MAXG>
constexpr int xl_words() { return 4 * MAXG * (BF ? 32 : 64); }

// gate/up (GU) or down: workgroup (unit blockIdx.x: rows 32 / R of row block blockIdx.x / R, assignment blockIdx.y),
// blockDim / 64 waves splitting K.
template <bool BF, bool GU, int MAXG, int NS, int R, int LB>
__global__ __launch_bounds__(LB) void mxt_expert_kernel(MxtArgs a) {
  constexpr int NM = GU ? 2 : 1, RU = 32 / R;
  __shared__ __align__(16) u32 xl[kMaxW][xl_words<BF, MAXG>()];
  __shared__ float red[kMaxW][NM][RU];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int NW = (int)(blockDim.x >> 6);
  const int64_t unit = blockIdx.x, asg = blockIdx.y, rb = unit / R;
  const int rsel = (int)(unit % R);
  int e;
  if constexpr (NS > 0) {
    __shared__ __align__(8) uint64_t keys[kMaxW][64 * NS];
    int rank[NS];
    float wo[NS];
    bool pick[NS];
    const RouteArgs &r = a.route;
    topk_select<NS>(r.logits + (asg / a.KU) * a.E, a.E, a.KU, r.gating, r.norm, r.scale, r.bias, keys[wave], rank,
                    wo, pick);
    float wt;
    topk_pick<NS>(rank, wo, pick, (int)(asg % a.KU), e, wt);
    if (unit == 0 && wave == 0 && lane == 0) {
      r.ids[asg] = e;
      r.wts[asg] = wt;
    }
  } else {
    e = a.ids[asg];
  }
  e = e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
  int c0, c1;
  wave_range(wave, NW, a.C, a.C4, c0, c1);
  const int64_t xrow = GU ? asg / a.KU : asg;
  float acc[NM];
  wave_dots<BF, NM, MAXG, R>(a, (int64_t)e * a.e_rb + rb, rsel, a.x + xrow * (int64_t)a.C * 64 * (BF ? 2 : 4), c0,
                             c1, xl[wave], acc);
  if (lane < RU) {
#pragma unroll
    for (int m = 0; m < NM; ++m) red[wave][m][lane] = acc[m];
  }
  __syncthreads();
  if (threadIdx.x < RU) {
    const int i = threadIdx.x;
    float s[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      s[m] = 0.f;
      for (int w = 0; w < NW; ++w) s[m] += red[w][m][i];
    }
    const int64_t row = RU * unit + i;
    float g = s[0];
    if (a.bias) g += a.bias[e * a.n + row];
    float v = g;
    if constexpr (GU) {
      float u = s[NM - 1];
      if (a.bias2) u += a.bias2[e * a.n + row];
      v = act_fn(a.act, g, u);
    }
    a.y[asg * a.n + row] = v;
  }
}

// down + combine: workgroup (unit blockIdx.x: rows 32 / R of row block blockIdx.x / R, token blockIdx.y); waves KU
// groups of S = blockDim / 64 / KU, group j the routed slot j (assignment t KU + j), its S waves splitting K.
template <bool BF, int MAXG, int R, int LB>
__global__ __launch_bounds__(LB) void mxt_combine_kernel(MxtArgs a) {
  constexpr int RU = 32 / R;
  __shared__ __align__(16) u32 xl[kMaxW][xl_words<BF, MAXG>()];
  __shared__ float red[kMaxW][RU];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int S = (int)(blockDim.x >> 6) / a.KU;
  const int j = wave / S, part = wave % S;
  const int64_t unit = blockIdx.x, t = blockIdx.y, asg = t * a.KU + j, rb = unit / R;
  const int rsel = (int)(unit % R);
  float y0 = 0.f;   // the combine's starting value, loaded ahead of the weights
  if (threadIdx.x < RU && a.accumulate) {
    y0 = a.y[t * a.n + RU * unit + threadIdx.x];
    if (a.sgate) y0 *= a.sgate[t];
  }
  int e = a.ids[asg];
  e = e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
  int c0, c1;
  wave_range(part, S, a.C, a.C4, c0, c1);
  float acc[1];
  wave_dots<BF, 1, MAXG, R>(a, (int64_t)e * a.e_rb + rb, rsel, a.x + asg * (int64_t)a.C * 64 * (BF ? 2 : 4), c0, c1,
                            xl[wave], acc);
  if (lane < RU) red[wave][lane] = acc[0];
  __syncthreads();
  if (threadIdx.x < RU) {
    const int i = threadIdx.x;
    const int64_t row = RU * unit + i;
    float v = y0;
    for (int jj = 0; jj < a.KU; ++jj) {
      float s = 0.f;
      for (int p = 0; p < S; ++p) s += red[jj * S + p][i];
      if (a.bias) {
        int ej = a.ids[t * a.KU + jj];
        ej = ej < 0 ? 0 : (ej >= a.E ? a.E - 1 : ej);
        s += a.bias[ej * a.n + row];
      }
      v = __builtin_fmaf(a.wts[t * a.KU + jj], s, v);
    }
    a.y[t * a.n + row] = v;
  }
}

// waves a workgroup splitting `groups` scale groups (at most `cap`)
int pick_waves(int groups, int cap) { return groups < cap ? groups : cap; }

// Rows a workgroup: 32 / R. The gate/up launches read two matrices and take whole 32-row blocks (R = 1); the down
// launches (one matrix, a quarter of the bytes at gpt-oss-20b's one token: 90 32-row blocks for 256 CUs) take 16-row
// units (R = 2), so twice as many CUs stream them (measured: the down + combine launch 11.5 -> 9.5 us; gate/up is
// slower with 16-row units, 10.9 -> 12.5 us, and both are slower with 8-row units).
constexpr int kRGateUp = 1, kRDown = 2;

// Waves a workgroup: one a scale group of K up to 16 (gate/up), and up to 16 / KU a routed slot (down: the combine's
// split; gpt-oss-20b: 12 waves of one group each, 4 x 4 waves of three groups). Fewer, longer waves measured slower.
constexpr int kGuWaves = kMaxW;
int slot_waves(int KU) { return kMaxW / KU; }

// The batch of scale groups a wave loads at once is its whole K range up to 2 groups (two matrices) or 3 (one);
// larger batches (up to 3 / 6 groups) take workgroups of at most 8 waves, whose waves may hold 256 VGPRs.
template <bool BF, bool GU, int NS>
int launch_expert(const MxtArgs &a, int nw, hipStream_t s) {
  constexpr int R = GU ? kRGateUp : kRDown;
  const dim3 grid((unsigned)(a.n / 32 * R), (unsigned)a.rows);
  const int gpw = (a.C4 + nw - 1) / nw;   // scale groups of the busiest wave
  if (gpw <= 1) mxt_expert_kernel<BF, GU, 1, NS, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  else if (gpw <= 2) mxt_expert_kernel<BF, GU, 2, NS, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  else if (nw <= 8) mxt_expert_kernel<BF, GU, 3, NS, R, 512><<<grid, 64 * nw, 0, s>>>(a);
  else mxt_expert_kernel<BF, GU, 2, NS, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  return launch_status();
}

template <bool BF>
int launch_combine(const MxtArgs &a, int nw, hipStream_t s) {
  constexpr int R = kRDown;   // the down matvec's units, so each slot's sums are qmm_moe_expert_mv_tiled's
  const dim3 grid((unsigned)(a.n / 32 * R), (unsigned)a.rows);
  const int S = nw / a.KU, gpw = (a.C4 + S - 1) / S;
  if (gpw <= 1) mxt_combine_kernel<BF, 1, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  else if (gpw <= 2) mxt_combine_kernel<BF, 2, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  else if (gpw <= 3 || nw > 8) mxt_combine_kernel<BF, 3, R, 1024><<<grid, 64 * nw, 0, s>>>(a);
  else mxt_combine_kernel<BF, 6, R, 512><<<grid, 64 * nw, 0, s>>>(a);
  return launch_status();
}

// shapes and pointers shared by the entry points: rows % 32, K % 64, 16-byte tiles, 4-byte scale groups
int check_tiled(int64_t k, int64_t n, const void *x, int x_dtype, const void *w, const void *ws, const float *y) {
  if (!x || !w || !ws || !y) return QMM_ERR_NULL;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (k <= 0 || k % 64 || k > (1 << 20) || n <= 0 || n % 32 || n > (1ll << 30)) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(ws, 4) || !aligned(y, 4)) return QMM_ERR_ALIGN;
  return QMM_OK;
}

MxtArgs base_args(int64_t k, int64_t n, int E, int KU, const void *x, const void *w, const void *ws, float *y) {
  MxtArgs a{};
  a.n = n;
  a.C = (int)(k / 64);
  a.C4 = (a.C + 3) / 4;
  a.E = E;
  a.KU = KU;
  a.x = static_cast<const u8 *>(x);
  a.wg = static_cast<const u8 *>(w);
  a.sg = static_cast<const u8 *>(ws);
  a.wu = a.wg;
  a.su = a.sg;
  a.y = y;
  return a;
}

// gate / up tensors: fused [E, 2n, k] (expert e's n gate rows then its n up rows) or two [E, n, k] tensors
void gate_up_args(MxtArgs &a, int fused, const void *w, const void *ws, const void *w2, const void *ws2) {
  const int64_t nrb = a.n / 32;
  if (fused) {
    a.e_rb = 2 * nrb;
    a.wu = static_cast<const u8 *>(w) + nrb * a.C * kTile;
    a.su = static_cast<const u8 *>(ws) + nrb * a.C4 * kScaleGroup;
  } else {
    a.e_rb = nrb;
    a.wu = static_cast<const u8 *>(w2);
    a.su = static_cast<const u8 *>(ws2);
  }
}

}  // namespace

// Decode expert matvecs on MFMA-tiled planes: mode 0 gate/up (act[a] = act(Wg[e] x[a / KU], Wu[e] x[a / KU])),
// mode 1 down (ys[a] = Wd[e] x[a]).
extern "C" int qmm_moe_expert_mv_tiled(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                       int64_t assignments, const int32_t *ids, const void *x, int x_dtype,
                                       const void *w, const void *ws, const void *w2, const void *ws2,
                                       const float *bias, const float *bias2, float *y, qmm_stream_t stream) {
  if (mode != 0 && mode != 1) return QMM_ERR_RANGE;
  if (act != QMM_ACT_SILU && act != QMM_ACT_SWIGLU_OAI) return QMM_ERR_RANGE;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (!ids) return QMM_ERR_NULL;
  if (int st = check_tiled(k, n, x, x_dtype, w, ws, y)) return st;
  const bool gu = mode == 0;
  if (gu && !fused && (!w2 || !ws2)) return QMM_ERR_NULL;
  if (gu && !fused && (!aligned(w2, 16) || !aligned(ws2, 4))) return QMM_ERR_ALIGN;
  if (assignments <= 0 || assignments > 65535 || (gu && assignments % KU)) return QMM_ERR_SHAPE;
  MxtArgs a = base_args(k, n, E, KU, x, w, ws, y);
  a.rows = assignments;
  a.ids = ids;
  a.bias = bias;
  a.bias2 = bias2;
  a.act = act;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf = x_dtype == QMM_BF16;
  if (gu) {
    gate_up_args(a, fused, w, ws, w2, ws2);
    const int nw = pick_waves(a.C4, kGuWaves);
    return bf ? launch_expert<true, true, 0>(a, nw, s) : launch_expert<false, true, 0>(a, nw, s);
  }
  // the down matvec splits K as the combine launch splits it for one routed slot, so its rows are the combine's
  a.e_rb = n / 32;
  const int nw = pick_waves(a.C4, slot_waves(KU));
  return bf ? launch_expert<true, false, 0>(a, nw, s) : launch_expert<false, false, 0>(a, nw, s);
}

// The gate/up launch of qmm_moe_topk_expert_mv on tiled planes (its checks done by the caller; E <= 256).
int qmm_topk_expert_mv_tiled(const RouteArgs &r, int E, int KU, int64_t tokens, int fused, int act, int64_t k,
                             int64_t n, const void *x, int x_dtype, const void *w, const void *ws, const void *w2,
                             const void *ws2, const float *bias, const float *bias2, float *y, hipStream_t s) {
  if (int st = check_tiled(k, n, x, x_dtype, w, ws, y)) return st;
  if (!fused && (!w2 || !ws2)) return QMM_ERR_NULL;
  if (!fused && (!aligned(w2, 16) || !aligned(ws2, 4))) return QMM_ERR_ALIGN;
  if (tokens * KU > 65535) return QMM_ERR_SHAPE;
  MxtArgs a = base_args(k, n, E, KU, x, w, ws, y);
  a.rows = tokens * KU;
  a.bias = bias;
  a.bias2 = bias2;
  a.act = act;
  a.route = r;
  gate_up_args(a, fused, w, ws, w2, ws2);
  const int nw = pick_waves(a.C4, kGuWaves);
  const bool bf = x_dtype == QMM_BF16;
#define QMM_MXT_ROUTE(NS) (bf ? launch_expert<true, true, NS>(a, nw, s) : launch_expert<false, true, NS>(a, nw, s))
  if (E <= 64) return QMM_MXT_ROUTE(1);
  if (E <= 128) return QMM_MXT_ROUTE(2);
  if (E <= 192) return QMM_MXT_ROUTE(3);
  return QMM_MXT_ROUTE(4);
#undef QMM_MXT_ROUTE
}

// The down matvecs and the combine of qmm_moe_expert_mv_combine on tiled planes (its checks done by the caller).
int qmm_expert_mv_combine_tiled(int64_t k, int64_t n, int E, int KU, int64_t tokens, const int32_t *ids,
                                const float *wts, const void *x, int x_dtype, const void *w, const void *ws,
                                const float *bias, int accumulate, const float *sg, float *y, hipStream_t s) {
  if (int st = check_tiled(k, n, x, x_dtype, w, ws, y)) return st;
  MxtArgs a = base_args(k, n, E, KU, x, w, ws, y);
  a.rows = tokens;
  a.ids = ids;
  a.wts = wts;
  a.bias = bias;
  a.accumulate = accumulate;
  a.sgate = sg;
  a.e_rb = n / 32;
  const int S = pick_waves(a.C4, slot_waves(KU));   // waves a routed slot (the down matvec's split)
  return x_dtype == QMM_BF16 ? launch_combine<true>(a, S * KU, s) : launch_combine<false>(a, S * KU, s);
}
