// MoE routing, permutation and combine, plus the activation producers of the grouped GEMMs.
//
//   qmm_moe_topk       top-k of router logits + gating weights      g_moe_route[_tr], S/gen_moe.py:116-500
//   qmm_moe_route      router matvec x W_router^T, then qmm_moe_topk g_moe_route[_tr][_live], S/gen_moe.py:116-500
//   qmm_moe_shared_gate sg[t] = sigmoid(x[t] . w)                   g_moe_shared_gate, S/gen_moe.py:780-823
//   qmm_moe_wscale     wts[t, k] *= scale[ids[t, k]]                g_moe_wscale, S/gen_moe.py:1010-1045
//   qmm_moe_bucket     canonical bucket of assignments into 64-row expert tiles
//                                                                    g_moe_bucket, S/gen_moe.py:829-955
//   qmm_moe_combine    y[t] (+)= sum_k w[t,k] ys[row(t,k)]           g_moe_combine[_sorted], S/gen_moe.py:730-762, :1231-1280
//   qmm_moe_combine_gated  y[t] = sg[t] y[t] + sum_k ...             shared_gated combine, S/gen_moe.py:765-779
//   qmm_row_scale_f16  per-row power-of-two scale + f16 copy         g_row_scale_f16[_tiles], S/gen_llm.py:1843-1915
//   qmm_row_scale_f16_rows  the same over listed rows (the bucket's pos): the rows g_row_scale_f16_tiles covers
//   qmm_quant_mxfp8    E4M3 + E8M0-per-32 operand of the scaled MFMA
//   qmm_repack_mxfp4   GGUF 17-byte MXFP4 blocks -> split planes
#include "common.hpp"
#include "topk.hpp"

using namespace qmm;

namespace {

constexpr int kTile = 64;
typedef __attribute__((ext_vector_type(4))) u32 v4u;

template <int NS>
__global__ __launch_bounds__(256) void topk_kernel(const float *__restrict__ logits, int64_t tokens, int E, int KU,
                                                   int gating, int norm, float scale, const float *__restrict__ bias,
                                                   const int32_t *__restrict__ info, int32_t *__restrict__ ids,
                                                   float *__restrict__ wts) {
  __shared__ __align__(16) uint64_t keys[4][64 * NS];
  const int wv = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  if (t >= tokens) return;               // a whole wave: nothing below synchronizes the workgroup
  if (info && info[4 * t + 2] == 0) return;   // a padding token of the epoch (_live): no ids, no weights
  topk_token<NS>(logits + t * E, t, E, KU, gating, norm, scale, bias, keys[wv], ids, wts);
}

// ------------------------------------------------------------------------------ top-k + activation operand
// The prefill chain's first two steps, routing and the grouped gate/up GEMM's activation operand, are both per token
// and independent: one launch does both, a wave ranking each token while another writes its operand. OP kOpF16: the row-scaled f16 row and its (2^-e, 2^e) as qmm_row_scale_f16 computes them; kOpMx8:
// the E4M3 codes and E8M0 scales as qmm_quant_mxfp8 computes them. x: bf16 rows [tokens, H]; NP: 16-byte pieces
// (8 values) a lane, H <= 512 NP.
enum TopkOp { kOpF16 = 1, kOpMx8 = 2 };

template <int NS, int OP, int NP>
__global__ __launch_bounds__(256) void topk_operand_kernel(const float *__restrict__ logits, int64_t tokens, int E,
                                                           int KU, int gating, int norm, float scale,
                                                           const float *__restrict__ bias, int32_t *__restrict__ ids,
                                                           float *__restrict__ wts, int64_t H,
                                                           const u16 *__restrict__ x, void *__restrict__ xo,
                                                           void *__restrict__ xs) {
  __shared__ __align__(16) uint64_t keys[2][64 * NS];
  // two tokens a workgroup: waves 0 / 1 rank tokens 2 b / 2 b + 1, waves 2 / 3 write their operands meanwhile
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 2 + (wv & 1);
  if (t >= tokens) return;
  if (wv < 2) {
    topk_token<NS>(logits + t * E, t, E, KU, gating, norm, scale, bias, keys[wv], ids, wts);
    return;
  }
  const int np = (int)(H / 8);           // pieces of the row
  const v4u *xr = reinterpret_cast<const v4u *>(x + t * H);
  v4u raw[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int p = lane + 64 * i;
    raw[i] = xr[p < np ? p : np - 1];
  }
  float v[NP][8];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const u32 d[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[i][2 * j] = bf16_to_f32(d[j] & 0xFFFFu); v[i][2 * j + 1] = bf16_to_f32(d[j] >> 16); }
  }
  if constexpr (OP == kOpF16) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const bool in = lane + 64 * i < np;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, in ? fabsf(v[i][j]) : 0.f);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    const int biased = (int)((f32_as_u32(m) >> 23) & 255u);
    const int e = min(max(biased - 127 - 13, 0), 100);
    const float sc = u32_as_f32((u32)(127 - e) << 23), inv = u32_as_f32((u32)(127 + e) << 23);
    v4u *o = reinterpret_cast<v4u *>(static_cast<_Float16 *>(xo) + t * H);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int p = lane + 64 * i;
      if (p < np) {
        u32 w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = (u32)__builtin_bit_cast(u16, (_Float16)(v[i][2 * j] * sc)) |
                 ((u32)__builtin_bit_cast(u16, (_Float16)(v[i][2 * j + 1] * sc)) << 16);
        o[p] = v4u{w[0], w[1], w[2], w[3]};
      }
    }
    if (lane == 0) reinterpret_cast<float2 *>(xs)[t] = make_float2(sc, inv);
  } else {
    // a 32-value block is four consecutive lanes' pieces (np % 4 == 0, so a block never straddles the row's end)
    typedef __attribute__((ext_vector_type(2))) u32 v2u;
    u8 *codes = static_cast<u8 *>(xo) + t * H;
    u8 *scales = static_cast<u8 *>(xs) + t * (H / 32);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int p = lane + 64 * i;
      float amax = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
      amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
      const int sx = mxfp8_exponent(amax);
      if (p < np) {
        int w0 = 0, w1 = 0;
        w0 = e4m3_pack2<false>(v[i][0], v[i][1], sx, w0);
        w0 = e4m3_pack2<true>(v[i][2], v[i][3], sx, w0);
        w1 = e4m3_pack2<false>(v[i][4], v[i][5], sx, w1);
        w1 = e4m3_pack2<true>(v[i][6], v[i][7], sx, w1);
        reinterpret_cast<v2u *>(codes)[p] = v2u{(u32)w0, (u32)w1};
        if ((lane & 3) == 0) scales[p / 4] = (u8)(sx + 127);
      }
    }
  }
}

// the top-k instantiation for E experts (slots a lane: ceil(E / 64))
static void launch_topk(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                        const float *bias, const int32_t *info, int32_t *ids, float *wts, hipStream_t s) {
  const unsigned g = (unsigned)((tokens + 3) / 4);
  if (E <= 64) topk_kernel<1><<<g, 256, 0, s>>>(logits, tokens, E, KU, gating, norm, scale, bias, info, ids, wts);
  else if (E <= 128) topk_kernel<2><<<g, 256, 0, s>>>(logits, tokens, E, KU, gating, norm, scale, bias, info, ids, wts);
  else if (E <= 192) topk_kernel<3><<<g, 256, 0, s>>>(logits, tokens, E, KU, gating, norm, scale, bias, info, ids, wts);
  else topk_kernel<4><<<g, 256, 0, s>>>(logits, tokens, E, KU, gating, norm, scale, bias, info, ids, wts);
}

// ------------------------------------------------------------------------------------------------ router
// out[t, e] = sum_k x[t, k] W[e, k] with fp32 accumulation: the router matvec of g_moe_route[_tr] (S/gen_moe.py:
// 116-252, :255-460) and, with one row and the sigmoid, g_moe_shared_gate (S/gen_moe.py:780-823). One wave per
// (row e, group of kRouteTok tokens), row fastest so the waves of a token group share its x rows in L2; lane l
// reads the 4-value chunks l, l + 64, ... of the row (one 1 KB contiguous piece per wave load for f32 weights)
// and the same chunks of each token's x. The lane sums its chunks in order, then the butterfly sums the lanes.
constexpr int kRouteTok = 8;

template <bool BF>
__device__ __forceinline__ f32x4 load4(const void *p, int64_t i4) {
  if constexpr (BF) {
    const uint2 q = reinterpret_cast<const uint2 *>(p)[i4];
    return f32x4{bf16_to_f32(q.x & 0xFFFFu), bf16_to_f32(q.x >> 16), bf16_to_f32(q.y & 0xFFFFu),
                 bf16_to_f32(q.y >> 16)};
  } else {
    return reinterpret_cast<const f32x4 *>(p)[i4];
  }
}

template <bool XBF, bool WBF>
__global__ __launch_bounds__(256) void router_kernel(int64_t tokens, int64_t H, int E, const void *__restrict__ x,
                                                     const void *__restrict__ w, int sigmoid, float *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int e = (int)(gw % E);
  const int64_t t0 = gw / E * kRouteTok;
  if (t0 >= tokens) return;
  const int64_t C = H / 4;                 // 4-value chunks of a row
  int64_t xrow[kRouteTok];
#pragma unroll
  for (int r = 0; r < kRouteTok; ++r) xrow[r] = (t0 + r < tokens ? t0 + r : tokens - 1) * C;   // tail: reread
  float acc[kRouteTok];
#pragma unroll
  for (int r = 0; r < kRouteTok; ++r) acc[r] = 0.f;
  const int64_t wrow = (int64_t)e * C;
#pragma unroll 2
  for (int64_t c = lane; c < C; c += 64) {
    const f32x4 wv = load4<WBF>(w, wrow + c);
#pragma unroll
    for (int r = 0; r < kRouteTok; ++r) {
      const f32x4 xv = load4<XBF>(x, xrow[r] + c);
      acc[r] = __builtin_fmaf(wv.x, xv.x, acc[r]);
      acc[r] = __builtin_fmaf(wv.y, xv.y, acc[r]);
      acc[r] = __builtin_fmaf(wv.z, xv.z, acc[r]);
      acc[r] = __builtin_fmaf(wv.w, xv.w, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kRouteTok; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && t0 + r < tokens) out[(t0 + r) * E + e] = sigmoid ? 1.f / (1.f + expf(-v)) : v;
  }
}

// ------------------------------------------------------------------------------------------------ wscale
// wts[a] *= scale[clamp(ids[a], 0, E - 1)] (g_moe_wscale: a per-expert output scale folded into the combine weights)
__global__ __launch_bounds__(256) void wscale_kernel(int64_t n, int E, const int32_t *__restrict__ ids,
                                                     const float *__restrict__ scale, float *__restrict__ wts) {
  const int64_t a = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (a >= n) return;
  int e = ids[a];
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);
  wts[a] = wts[a] * scale[e];
}

// ------------------------------------------------------------------------------------------------ bucket
// One workgroup of 1024 threads. Counts per expert, 64-row tiles per expert in id order, then a stable scatter:
// assignments are taken in chunks of 1024 in ascending order; inside a wave the lanes with the same expert are
// found with 8 ballots (one per bit of the id) and ranked by popcount, waves are ranked through a per-wave count
// table, chunks through a running offset per expert. The row of an assignment is therefore its rank among the
// live assignments of its expert in ascending a (the canonical order), independent of thread timing.
constexpr int kBucketThreads = 1024;
constexpr int kBucketWaves = kBucketThreads / 64;
constexpr int kMaxE = 256;

__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(int64_t tokens, int KU, int E, int64_t max_tiles,
                                                                const int32_t *__restrict__ info,
                                                                const int32_t *__restrict__ ids,
                                                                int32_t *__restrict__ tile_info,
                                                                int32_t *__restrict__ rowmap, int32_t *__restrict__ pos) {
  __shared__ int count[kMaxE];
  __shared__ int base[kMaxE];
  __shared__ int running[kMaxE];
  __shared__ int wcount[kBucketWaves][kMaxE];
  __shared__ int total_tiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t A = tokens * KU;
  for (int e = tid; e < kMaxE; e += kBucketThreads) { count[e] = 0; running[e] = 0; }
  for (int i = tid; i < kBucketWaves * kMaxE; i += kBucketThreads) (&wcount[0][0])[i] = 0;
  __syncthreads();
  for (int64_t a = tid; a < A; a += kBucketThreads) {
    const int64_t t = a / KU;
    if (info && info[t * 4 + 2] == 0) continue;
    int e = ids[a];
    e = e < 0 ? 0 : (e >= E ? E - 1 : e);
    atomicAdd(&count[e], 1);
  }
  __syncthreads();
  if (wave == 0) {   // exclusive scan of tiles per expert over <= 256 experts, 4 per lane
    int tl[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      tl[i] = e < E ? (count[e] + kTile - 1) / kTile : 0;
      s += tl[i];
    }
    int incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    int b = incl - s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e < kMaxE) base[e] = b;
      b += tl[i];
    }
    if (lane == 63) total_tiles = incl;
  }
  __syncthreads();
  // tile table
  for (int e = tid; e < E; e += kBucketThreads) {
    const int tiles = (count[e] + kTile - 1) / kTile;
    for (int j = 0; j < tiles; ++j) {
      tile_info[2 * (base[e] + j)] = e;
      tile_info[2 * (base[e] + j) + 1] = min(kTile, count[e] - kTile * j);
    }
  }
  for (int64_t i = total_tiles + tid; i < max_tiles; i += kBucketThreads) {
    tile_info[2 * i] = -1;
    tile_info[2 * i + 1] = 0;
  }
  for (int64_t r = tid; r < max_tiles * kTile; r += kBucketThreads) rowmap[r] = -1;
  __syncthreads();
  // stable scatter
  for (int64_t c0 = 0; c0 < A; c0 += kBucketThreads) {
    const int64_t a = c0 + tid;
    bool live = a < A;
    int e = 0;
    if (live) {
      const int64_t t = a / KU;
      live = !(info && info[t * 4 + 2] == 0);
      e = ids[a];
      e = e < 0 ? 0 : (e >= E ? E - 1 : e);
    }
    uint64_t peers = __ballot(live);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t ones = __ballot(live && ((e >> bit) & 1));
      peers &= ((e >> bit) & 1) ? ones : ~ones;
    }
    const uint64_t lt = (1ull << lane) - 1ull;
    const int rank_w = __popcll(peers & lt);
    if (live && rank_w == 0) wcount[wave][e] = __popcll(peers);
    __syncthreads();
    for (int ex = tid; ex < E; ex += kBucketThreads) {   // per expert: exclusive offsets over waves
      int run = running[ex];
      for (int w = 0; w < kBucketWaves; ++w) {
        const int c = wcount[w][ex];
        wcount[w][ex] = run;
        run += c;
      }
      running[ex] = run;
    }
    __syncthreads();
    if (a < A) {
      if (live) {
        const int row = base[e] * kTile + wcount[wave][e] + rank_w;
        rowmap[row] = (int32_t)a;
        pos[a] = row;
      } else {
        pos[a] = -1;
      }
    }
    __syncthreads();
    for (int i = tid; i < kBucketWaves * kMaxE; i += kBucketThreads) (&wcount[0][0])[i] = 0;
    __syncthreads();
  }
}

// Many assignments (from 8192): the same rows from three launches of many workgroups. Workgroup g owns the assignments
// [g C, g C + C) (the last one also the remainder, C = kBucketChunk >= kMaxE). (1) count: per expert the live
// assignments of the range, parked in pos[g C + e] (the range's own slice of pos, which only its scatter writes
// later), and rowmap cleared. (2) scan, one workgroup: tiles per expert, the tile table, and per (g, e) the first
// row of expert e's assignments of range g, base[e] * 64 + the counts of the ranges before g, parked back in the
// same slot. (3) scatter: range g reads its row offsets, then ranks its assignments in ascending a exactly as the
// one-workgroup kernel does. Rows are therefore the one-workgroup kernel's, bit for bit.
constexpr int kBucketChunk = 1024;
static_assert(kBucketChunk >= kMaxE, "a range parks one count per expert in its own slice of pos");
constexpr int64_t kBucketSplit = 8 * kBucketChunk;   // assignments from which the three launches are faster

__device__ __forceinline__ void bucket_range(int64_t A, int G, int g, int64_t &a0, int64_t &a1) {
  a0 = (int64_t)g * kBucketChunk;
  a1 = g == G - 1 ? A : a0 + kBucketChunk;
}

__global__ __launch_bounds__(kBucketThreads) void bucket_count_kernel(int64_t tokens, int KU, int E, int64_t max_tiles,
                                                                      const int32_t *__restrict__ info,
                                                                      const int32_t *__restrict__ ids,
                                                                      int32_t *__restrict__ rowmap,
                                                                      int32_t *__restrict__ pos) {
  __shared__ int count[kMaxE];
  const int tid = threadIdx.x, G = gridDim.x, g = blockIdx.x;
  const int64_t A = tokens * KU;
  int64_t a0, a1;
  bucket_range(A, G, g, a0, a1);
  for (int e = tid; e < kMaxE; e += kBucketThreads) count[e] = 0;
  // this range's share of the row map cleared (every row; the scatter writes the live ones)
  const int64_t R = max_tiles * kTile, r0 = R * g / G, r1 = R * (g + 1) / G;
  for (int64_t r = r0 + tid; r < r1; r += kBucketThreads) rowmap[r] = -1;
  __syncthreads();
  for (int64_t a = a0 + tid; a < a1; a += kBucketThreads) {
    if (info && info[(a / KU) * 4 + 2] == 0) continue;
    int e = ids[a];
    e = e < 0 ? 0 : (e >= E ? E - 1 : e);
    atomicAdd(&count[e], 1);
  }
  __syncthreads();
  for (int e = tid; e < E; e += kBucketThreads) pos[a0 + e] = count[e];
}

__global__ __launch_bounds__(kBucketThreads) void bucket_scan_kernel(int64_t tokens, int KU, int E, int64_t max_tiles,
                                                                     int G, int32_t *__restrict__ tile_info,
                                                                     int32_t *__restrict__ pos) {
  __shared__ int total[kMaxE];
  __shared__ int base[kMaxE];
  __shared__ int total_tiles;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t A = tokens * KU;
  // per expert: the counts of the ranges become running offsets inside the expert (a thread per expert)
  for (int e = tid; e < kMaxE; e += kBucketThreads) {
    int run = 0;
    if (e < E)
      for (int g = 0; g < G; ++g) {
        int64_t a0, a1;
        bucket_range(A, G, g, a0, a1);
        const int c = pos[a0 + e];
        pos[a0 + e] = run;
        run += c;
      }
    total[e] = run;
  }
  __syncthreads();
  if (wave == 0) {   // exclusive scan of tiles per expert over <= 256 experts, 4 per lane
    int tl[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      tl[i] = e < E ? (total[e] + kTile - 1) / kTile : 0;
      sum += tl[i];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    int b = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      base[lane * 4 + i] = b;
      b += tl[i];
    }
    if (lane == 63) total_tiles = incl;
  }
  __syncthreads();
  for (int e = tid; e < E; e += kBucketThreads) {
    const int tiles = (total[e] + kTile - 1) / kTile;
    for (int j = 0; j < tiles; ++j) {
      tile_info[2 * (base[e] + j)] = e;
      tile_info[2 * (base[e] + j) + 1] = min(kTile, total[e] - kTile * j);
    }
  }
  for (int64_t i = total_tiles + tid; i < max_tiles; i += kBucketThreads) {
    tile_info[2 * i] = -1;
    tile_info[2 * i + 1] = 0;
  }
  // the first row of each (range, expert): the expert's first tile row plus the running offset
  for (int64_t i = tid; i < (int64_t)G * E; i += kBucketThreads) {
    const int g = (int)(i / E), e = (int)(i % E);
    int64_t a0, a1;
    bucket_range(A, G, g, a0, a1);
    pos[a0 + e] += base[e] * kTile;
  }
}

__global__ __launch_bounds__(kBucketThreads) void bucket_scatter_kernel(int64_t tokens, int KU, int E,
                                                                        const int32_t *__restrict__ info,
                                                                        const int32_t *__restrict__ ids,
                                                                        int32_t *__restrict__ rowmap,
                                                                        int32_t *__restrict__ pos) {
  __shared__ int first[kMaxE];
  __shared__ int wcount[kBucketWaves][kMaxE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, G = gridDim.x, g = blockIdx.x;
  const int64_t A = tokens * KU;
  int64_t a0, a1;
  bucket_range(A, G, g, a0, a1);
  for (int e = tid; e < E; e += kBucketThreads) first[e] = pos[a0 + e];
  for (int i = tid; i < kBucketWaves * kMaxE; i += kBucketThreads) (&wcount[0][0])[i] = 0;
  __syncthreads();   // the offsets are read before this range's pos entries are written
  for (int64_t c0 = a0; c0 < a1; c0 += kBucketThreads) {
    const int64_t a = c0 + tid;
    bool live = a < a1;
    int e = 0;
    if (live) {
      live = !(info && info[(a / KU) * 4 + 2] == 0);
      e = ids[a];
      e = e < 0 ? 0 : (e >= E ? E - 1 : e);
    }
    uint64_t peers = __ballot(live);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t ones = __ballot(live && ((e >> bit) & 1));
      peers &= ((e >> bit) & 1) ? ones : ~ones;
    }
    const int rank_w = __popcll(peers & ((1ull << lane) - 1ull));
    if (live && rank_w == 0) wcount[wave][e] = __popcll(peers);
    __syncthreads();
    for (int ex = tid; ex < E; ex += kBucketThreads) {   // per expert: exclusive offsets over waves
      int run = first[ex];
      for (int w = 0; w < kBucketWaves; ++w) {
        const int c = wcount[w][ex];
        wcount[w][ex] = run;
        run += c;
      }
      first[ex] = run;
    }
    __syncthreads();
    if (a < a1) {
      if (live) {
        const int row = wcount[wave][e] + rank_w;
        rowmap[row] = (int32_t)a;
        pos[a] = row;
      } else {
        pos[a] = -1;
      }
    }
    __syncthreads();
    for (int i = tid; i < kBucketWaves * kMaxE; i += kBucketThreads) (&wcount[0][0])[i] = 0;
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------------------------- combine
// One workgroup per token, 256-channel blocks; the fma chain runs in k order (S/gen_moe.py:1231-1280).
__global__ __launch_bounds__(256) void combine_kernel(int64_t tokens, int64_t rows, int64_t H, int KU,
                                                      const float *__restrict__ ys, const int32_t *__restrict__ pos,
                                                      const float *__restrict__ wts, int accumulate,
                                                      const float *__restrict__ sg, float *__restrict__ y) {
  const int64_t t = blockIdx.x;
  int64_t row[8];
  float w[8];
  for (int k = 0; k < KU; ++k) {
    row[k] = pos ? pos[t * KU + k] : t * KU + k;
    w[k] = wts[t * KU + k];
  }
  const float g = sg ? sg[t] : 1.f;
  for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
    float acc = accumulate ? (sg ? y[t * H + c] * g : y[t * H + c]) : 0.f;
    for (int k = 0; k < KU; ++k) {
      const float v = (row[k] >= 0 && row[k] < rows) ? ys[row[k] * H + c] : 0.f;
      acc = __builtin_fmaf(w[k], v, acc);
    }
    y[t * H + c] = acc;
  }
}

// ------------------------------------------------------------------------------------------ row scale f16
// One workgroup per row: e = clamp(exponent(max |x|) - 13, 0, 100), x16 = f16(x 2^-e) (round to nearest even),
// scales = (2^-e, 2^e). x is f32 or bf16.
// The same with 16-byte accesses, for H % 4 == 0 and 16-byte aligned ys / y: workgroup (t, part) covers 1024
// values of token t, thread c four of them, and every one of the KU rows is loaded before the fma chain (same
// order, same arithmetic as combine_kernel).
__global__ __launch_bounds__(256) void combine_vec_kernel(int64_t tokens, int64_t rows, int64_t H, int KU,
                                                          const float *__restrict__ ys, const int32_t *__restrict__ pos,
                                                          const float *__restrict__ wts, int accumulate,
                                                          const float *__restrict__ sg, float *__restrict__ y) {
  const int64_t t = blockIdx.y;
  const int64_t c4 = (int64_t)blockIdx.x * 256 + threadIdx.x;   // float4 index within the row
  if (c4 * 4 >= H) return;
  int64_t row[8];
  float w[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < KU) {
      row[k] = pos ? pos[t * KU + k] : t * KU + k;
      w[k] = wts[t * KU + k];
    }
  }
  f32x4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < KU) v[k] = (row[k] >= 0 && row[k] < rows) ? reinterpret_cast<const f32x4 *>(ys + row[k] * H)[c4] : f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 acc = accumulate ? reinterpret_cast<const f32x4 *>(y + t * H)[c4] : f32x4{0.f, 0.f, 0.f, 0.f};
  if (sg) {                                // the shared experts' output in y, scaled by the token's gate first
    const float g = sg[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = acc[j] * g;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < KU) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(w[k], v[k][j], acc[j]);
    }
  reinterpret_cast<f32x4 *>(y + t * H)[c4] = acc;
}

__device__ __forceinline__ float load_act(const void *x, int bf, int64_t i) {
  return bf ? bf16_to_f32(static_cast<const u16 *>(x)[i]) : static_cast<const float *>(x)[i];
}

// A padding row (info != NULL and info[row, 2] == 0, the reference's g_row_scale_f16_live) gets scale and inverse 0
// and zero f16 values without its x row being read; the prefill GEMM skips a 64-row tile whose scales are all 0.
__device__ __forceinline__ bool pad_row(const int32_t *info, int64_t r, int64_t k, float *scales, _Float16 *x16) {
  if (!info || info[4 * r + 2] != 0) return false;
  for (int64_t c = threadIdx.x; c < k; c += 256) x16[r * k + c] = (_Float16)0.f;
  if (threadIdx.x == 0) {
    scales[2 * r] = 0.f;
    scales[2 * r + 1] = 0.f;
  }
  return true;
}

__global__ __launch_bounds__(256) void row_scale_kernel(int64_t rows, int64_t k, const void *__restrict__ x, int bf,
                                                        float *__restrict__ scales, _Float16 *__restrict__ x16,
                                                        const int32_t *__restrict__ tile_info,
                                                        const int32_t *__restrict__ info) {
  const int64_t r = blockIdx.x;
  if (tile_info && (tile_info[2 * (r / kTile)] < 0 || r % kTile >= tile_info[2 * (r / kTile) + 1])) return;
  if (pad_row(info, r, k, scales, x16)) return;
  __shared__ float wmax[4];
  float m = 0.f;
  for (int64_t c = threadIdx.x; c < k; c += 256) m = fmaxf(m, fabsf(load_act(x, bf, r * k + c)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const int biased = (int)((f32_as_u32(m) >> 23) & 255u);
  const int e = min(max(biased - 127 - 13, 0), 100);
  const float sc = u32_as_f32((u32)(127 - e) << 23), inv = u32_as_f32((u32)(127 + e) << 23);
  for (int64_t c = threadIdx.x; c < k; c += 256) x16[r * k + c] = (_Float16)(load_act(x, bf, r * k + c) * sc);
  if (threadIdx.x == 0) {
    scales[2 * r] = sc;
    scales[2 * r + 1] = inv;
  }
}

// 16-byte accesses for the wave-per-row kernel below
constexpr int kRsMaxChunks = 16;   // 8-value chunks a lane: rows of up to 64 x 8 x 16 = 8192 values
typedef __attribute__((ext_vector_type(4))) u32 v4u;

template <bool BF>
__device__ __forceinline__ void load8(const void *x, int64_t i8, float (&v)[8]) {
  if constexpr (BF) {
    const v4u q = reinterpret_cast<const v4u *>(x)[i8];
    const u32 d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_to_f32(d[j] & 0xFFFFu); v[2 * j + 1] = bf16_to_f32(d[j] >> 16); }
  } else {
    const v4u a = reinterpret_cast<const v4u *>(x)[2 * i8], b = reinterpret_cast<const v4u *>(x)[2 * i8 + 1];
    const u32 d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = u32_as_f32(d[j]);
  }
}

// One wave per row (four rows a workgroup): lane l handles the 8-value chunks l, l + 64, ... (NCH of them at most,
// held in registers between the row maximum and the conversion); the maximum is a wave butterfly, so the row needs no
// workgroup barrier or LDS. Rows up to 64 x 8 x NCH values; the host takes the scalar kernel above for wider,
// misaligned or k % 8 != 0 rows.
template <bool BF, int NCH>
__global__ __launch_bounds__(256) void row_scale_wave_kernel(int64_t rows, int64_t k, const void *__restrict__ x,
                                                             float *__restrict__ scales, _Float16 *__restrict__ x16,
                                                             const int32_t *__restrict__ tile_info,
                                                             const int32_t *__restrict__ info,
                                                             const int32_t *__restrict__ ridx = nullptr) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= rows) return;
  const int64_t r = ridx ? ridx[i] : i;   // ridx: the listed rows only (rows = entries of the list)
  if (r < 0) return;
  if (tile_info && (tile_info[2 * (r / kTile)] < 0 || r % kTile >= tile_info[2 * (r / kTile) + 1])) return;
  const int64_t nch = k / 8, base = r * nch;
  if (info && info[4 * r + 2] == 0) {   // a padding row of the epoch: zero values, scale and inverse 0
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t c = lane + 64 * i;
      if (c < nch) reinterpret_cast<v4u *>(x16)[base + c] = v4u{0u, 0u, 0u, 0u};
    }
    if (lane == 0) {
      scales[2 * r] = 0.f;
      scales[2 * r + 1] = 0.f;
    }
    return;
  }
  // every chunk load is issued before any is used (a lane past the row reloads its last chunk and ignores it), so
  // the row costs one memory latency, not one per chunk
  float v[NCH][8];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = lane + 64 * i;
    load8<BF>(x, base + (c < nch ? c : nch - 1), v[i]);
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const bool in = lane + 64 * i < nch;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, in ? fabsf(v[i][j]) : 0.f);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  const int biased = (int)((f32_as_u32(m) >> 23) & 255u);
  const int e = min(max(biased - 127 - 13, 0), 100);
  const float sc = u32_as_f32((u32)(127 - e) << 23), inv = u32_as_f32((u32)(127 + e) << 23);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = lane + 64 * i;
    if (c < nch) {
      u32 o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = (u32)__builtin_bit_cast(u16, (_Float16)(v[i][2 * j] * sc)) |
               ((u32)__builtin_bit_cast(u16, (_Float16)(v[i][2 * j + 1] * sc)) << 16);
      reinterpret_cast<v4u *>(x16)[base + c] = v4u{o[0], o[1], o[2], o[3]};
    }
  }
  if (lane == 0) {
    scales[2 * r] = sc;
    scales[2 * r + 1] = inv;
  }
}

// ---------------------------------------------------------------------------------------------- MXFP8 quant
// OCP MX: one E8M0 scale per 32 values along a row, E4M3 codes (mxfp8_exponent, e4m3_pack2). Consecutive lanes take consecutive 16-byte pieces of the rows (4 f32 or 8 bf16 values); a
// block is the group of 8 (f32) or 4 (bf16) lanes holding it, whose maximum comes from a butterfly inside the group.
constexpr int kMxBlock = 32;

template <bool BF>
__global__ __launch_bounds__(256) void quant_mxfp8_vec_kernel(int64_t rows, int64_t k, const void *__restrict__ xv,
                                                              const int32_t *__restrict__ tile_info,
                                                              u8 *__restrict__ codes, u8 *__restrict__ scales) {
  constexpr int VPL = BF ? 8 : 4, LPB = kMxBlock / VPL;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // 16-byte piece of the input
  const int64_t pieces = rows * (k / VPL);
  const bool in = g < pieces;
  const int64_t gg = in ? g : pieces - 1;
  const int64_t r = gg / (k / VPL);
  const bool live = in && !(tile_info && tile_info[2 * (r / kTile)] < 0);
  float v[VPL];
  if constexpr (BF) {
    const v4u q = reinterpret_cast<const v4u *>(xv)[gg];
    const u32 d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_to_f32(d[j] & 0xFFFFu); v[2 * j + 1] = bf16_to_f32(d[j] >> 16); }
  } else {
    const f32x4 q = reinterpret_cast<const f32x4 *>(xv)[gg];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = q[j];
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int off = 1; off < LPB; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const int sx = mxfp8_exponent(amax);
  if (!live) return;
  u32 out[VPL / 4];
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    int w = 0;
    w = e4m3_pack2<false>(v[4 * i], v[4 * i + 1], sx, w);
    w = e4m3_pack2<true>(v[4 * i + 2], v[4 * i + 3], sx, w);
    out[i] = (u32)w;
  }
  if constexpr (BF) {
    typedef __attribute__((ext_vector_type(2))) u32 v2u;
    reinterpret_cast<v2u *>(codes)[g] = v2u{out[0], out[1]};
  } else {
    reinterpret_cast<u32 *>(codes)[g] = out[0];
  }
  if ((threadIdx.x & (LPB - 1)) == 0) scales[g / LPB] = (u8)(sx + 127);
}

__global__ __launch_bounds__(256) void repack_mxfp4_kernel(int64_t groups, const u8 *__restrict__ w,
                                                           u8 *__restrict__ nib, u8 *__restrict__ sc) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  const u8 *b = w + g * 17;
  u32 code[32];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const u32 q = b[1 + j];
    code[j] = q & 15u;
    code[j + 16] = q >> 4;
  }
  u32 out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32 v = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) v |= (code[8 * i + 2 * j] | (code[8 * i + 2 * j + 1] << 4)) << (8 * j);
    out[i] = v;
  }
  reinterpret_cast<uint4 *>(nib)[g] = make_uint4(out[0], out[1], out[2], out[3]);
  sc[g] = b[0];
}

}  // namespace

extern "C" {

int qmm_moe_topk_operand(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                         const float *bias, int32_t *ids, float *wts, int64_t H, const void *x, int x_dtype,
                         int op_dtype, void *xo, void *xo_scales, qmm_stream_t stream) {
  if (!logits || !ids || !wts || !x || !xo || !xo_scales) return QMM_ERR_NULL;
  if (E <= 0 || E > 256 || KU <= 0 || KU > 8 || KU > E) return QMM_ERR_RANGE;
  if (gating < 1 || gating > 3 || (gating == 1 && bias)) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  if (x_dtype != QMM_BF16 || (op_dtype != QMM_F16 && op_dtype != QMM_MXFP8)) return QMM_ERR_DTYPE;
  if (H <= 0 || H > 4096 || H % (op_dtype == QMM_F16 ? 8 : 32)) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(xo, op_dtype == QMM_F16 ? 16 : 8) || !aligned(xo_scales, 8)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned g = (unsigned)((tokens + 1) / 2);
  const int NS = (E + 63) / 64;
  const u16 *xb = static_cast<const u16 *>(x);
  auto go = [&](auto kern) {
    kern<<<g, 256, 0, s>>>(logits, tokens, E, KU, gating, norm, scale, bias, ids, wts, H, xb, xo, xo_scales);
    return launch_status();
  };
#define QMM_TOPK_OP(NSV)                                                                                            \
  if (NS == NSV) {                                                                                                  \
    if (op_dtype == QMM_F16)                                                                                        \
      return H <= 2048 ? go(topk_operand_kernel<NSV, kOpF16, 4>) : go(topk_operand_kernel<NSV, kOpF16, 8>);       \
    return H <= 2048 ? go(topk_operand_kernel<NSV, kOpMx8, 4>) : go(topk_operand_kernel<NSV, kOpMx8, 8>);         \
  }
  QMM_TOPK_OP(1)
  QMM_TOPK_OP(2)
  QMM_TOPK_OP(3)
  QMM_TOPK_OP(4)
#undef QMM_TOPK_OP
  return QMM_ERR_RANGE;
}

int qmm_moe_topk(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                 const float *bias, int32_t *ids, float *wts, qmm_stream_t stream) {
  if (!logits || !ids || !wts) return QMM_ERR_NULL;
  if (E <= 0 || E > 256 || KU <= 0 || KU > 8 || KU > E) return QMM_ERR_RANGE;
  if (gating < 1 || gating > 3 || (gating == 1 && bias)) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  launch_topk(logits, tokens, E, KU, gating, norm, scale, bias, nullptr, ids, wts, s);
  return launch_status();
}

static int router(int64_t tokens, int64_t H, int E, const void *x, int x_dtype, const void *w, int w_dtype,
                  int sigmoid, float *out, hipStream_t s) {
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (w_dtype != QMM_F32 && w_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (H <= 0 || H % 4 || H > (1 << 20)) return QMM_ERR_SHAPE;
  const bool xb = x_dtype == QMM_BF16, wb = w_dtype == QMM_BF16;
  if (!aligned(x, xb ? 8 : 16) || !aligned(w, wb ? 8 : 16) || !aligned(out, 4)) return QMM_ERR_ALIGN;
  const int64_t waves = (int64_t)E * ((tokens + kRouteTok - 1) / kRouteTok);
  const unsigned grid = (unsigned)((waves + 3) / 4);
  if (xb) {
    if (wb) router_kernel<true, true><<<grid, 256, 0, s>>>(tokens, H, E, x, w, sigmoid, out);
    else router_kernel<true, false><<<grid, 256, 0, s>>>(tokens, H, E, x, w, sigmoid, out);
  } else {
    if (wb) router_kernel<false, true><<<grid, 256, 0, s>>>(tokens, H, E, x, w, sigmoid, out);
    else router_kernel<false, false><<<grid, 256, 0, s>>>(tokens, H, E, x, w, sigmoid, out);
  }
  return launch_status();
}

int qmm_moe_route(int64_t tokens, int64_t H, int E, int KU, int gating, int norm, float scale, const void *x,
                  int x_dtype, const void *w, int w_dtype, const float *bias, const int32_t *info, float *logits,
                  int32_t *ids, float *wts, qmm_stream_t stream) {
  if (!x || !w || !logits || !ids || !wts) return QMM_ERR_NULL;
  if (E <= 0 || E > 256 || KU <= 0 || KU > 8 || KU > E) return QMM_ERR_RANGE;
  if (gating < 1 || gating > 3 || (gating == 1 && bias)) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (int st = router(tokens, H, E, x, x_dtype, w, w_dtype, 0, logits, s)) return st;
  launch_topk(logits, tokens, E, KU, gating, norm, scale, bias, info, ids, wts, s);
  return launch_status();
}

int qmm_moe_shared_gate(int64_t tokens, int64_t H, const void *x, int x_dtype, const void *w, int w_dtype, float *sg,
                        qmm_stream_t stream) {
  if (!x || !w || !sg) return QMM_ERR_NULL;
  if (tokens <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  return router(tokens, H, 1, x, x_dtype, w, w_dtype, 1, sg, reinterpret_cast<hipStream_t>(stream));
}

int qmm_moe_wscale(int64_t tokens, int KU, int E, const int32_t *ids, const float *scale, float *wts,
                   qmm_stream_t stream) {
  if (!ids || !scale || !wts) return QMM_ERR_NULL;
  if (E <= 0 || E > 1024 || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  const int64_t n = tokens * KU;
  wscale_kernel<<<(unsigned)((n + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(n, E, ids, scale, wts);
  return launch_status();
}

int qmm_moe_bucket(int64_t tokens, int KU, int E, int64_t max_tiles, const int32_t *info, const int32_t *ids,
                   int32_t *tile_info, int32_t *rowmap, int32_t *pos, qmm_stream_t stream) {
  if (!ids || !tile_info || !rowmap || !pos) return QMM_ERR_NULL;
  if (E <= 0 || E > kMaxE || KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (tokens <= 0 || tokens > 65536) return QMM_ERR_SHAPE;
  if (max_tiles < tokens * KU / kTile + E || max_tiles > (1 << 24)) return QMM_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t A = tokens * KU;
  if (A < kBucketSplit) {   // three launches cost about 15 us; the one-workgroup kernel about 2 us per 1024
    bucket_kernel<<<1, kBucketThreads, 0, s>>>(tokens, KU, E, max_tiles, info, ids, tile_info, rowmap, pos);
    return launch_status();
  }
  const int G = (int)(A / kBucketChunk);   // ranges of kBucketChunk assignments, the last with the remainder
  bucket_count_kernel<<<G, kBucketThreads, 0, s>>>(tokens, KU, E, max_tiles, info, ids, rowmap, pos);
  bucket_scan_kernel<<<1, kBucketThreads, 0, s>>>(tokens, KU, E, max_tiles, G, tile_info, pos);
  bucket_scatter_kernel<<<G, kBucketThreads, 0, s>>>(tokens, KU, E, info, ids, rowmap, pos);
  return launch_status();
}

static int combine(int64_t tokens, int64_t rows, int64_t H, int KU, const float *ys, const int32_t *pos,
                   const float *wts, int accumulate, const float *sg, float *y, qmm_stream_t stream) {
  if (!ys || !wts || !y) return QMM_ERR_NULL;
  if (KU <= 0 || KU > 8) return QMM_ERR_RANGE;
  if (tokens <= 0 || H <= 0 || rows <= 0 || tokens > (1ll << 24)) return QMM_ERR_SHAPE;
  if (!pos && rows < tokens * KU) return QMM_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (H % 4 == 0 && aligned(ys, 16) && aligned(y, 16) && tokens <= 65535)
    combine_vec_kernel<<<dim3((unsigned)((H / 4 + 255) / 256), (unsigned)tokens), 256, 0, s>>>(
        tokens, rows, H, KU, ys, pos, wts, accumulate, sg, y);
  else
    combine_kernel<<<(unsigned)tokens, 256, 0, s>>>(tokens, rows, H, KU, ys, pos, wts, accumulate, sg, y);
  return launch_status();
}

int qmm_moe_combine(int64_t tokens, int64_t rows, int64_t H, int KU, const float *ys, const int32_t *pos,
                    const float *wts, int accumulate, float *y, qmm_stream_t stream) {
  return combine(tokens, rows, H, KU, ys, pos, wts, accumulate, nullptr, y, stream);
}

int qmm_moe_combine_gated(int64_t tokens, int64_t rows, int64_t H, int KU, const float *ys, const int32_t *pos,
                          const float *wts, const float *sg, float *y, qmm_stream_t stream) {
  if (!sg) return QMM_ERR_NULL;
  return combine(tokens, rows, H, KU, ys, pos, wts, 1, sg, y, stream);
}

static int row_scale(int64_t rows, int64_t k, const void *x, int x_dtype, float *scales, void *x16,
                     const int32_t *tile_info, const int32_t *info, hipStream_t s, const int32_t *ridx = nullptr) {
  if (!x || !scales || !x16) return QMM_ERR_NULL;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (rows <= 0 || k <= 0 || rows > (1ll << 24)) return QMM_ERR_SHAPE;
  if (tile_info && rows % kTile) return QMM_ERR_SHAPE;
  _Float16 *o = static_cast<_Float16 *>(x16);
  const bool wave_path = k % 8 == 0 && k <= 8 * 64 * kRsMaxChunks && aligned(x, 16) && aligned(x16, 16);
  if (ridx && !wave_path) return k % 8 || k > 8 * 64 * kRsMaxChunks ? QMM_ERR_SHAPE : QMM_ERR_ALIGN;
  if (wave_path) {
    const unsigned grid = (unsigned)((rows + 3) / 4);
    const int64_t per = (k / 8 + 63) / 64;   // chunks a lane
    const bool bf = x_dtype == QMM_BF16;
#define QMM_RS(N)                                                                                                   \
  (bf ? (row_scale_wave_kernel<true, N><<<grid, 256, 0, s>>>(rows, k, x, scales, o, tile_info, info, ridx), 0)    \
      : (row_scale_wave_kernel<false, N><<<grid, 256, 0, s>>>(rows, k, x, scales, o, tile_info, info, ridx), 0))
    if (per <= 1) QMM_RS(1);
    else if (per <= 2) QMM_RS(2);
    else if (per <= 4) QMM_RS(4);
    else if (per <= 8) QMM_RS(8);
    else QMM_RS(16);
#undef QMM_RS
  } else {
    row_scale_kernel<<<(unsigned)rows, 256, 0, s>>>(rows, k, x, x_dtype == QMM_BF16, scales, o, tile_info, info);
  }
  return launch_status();
}

int qmm_row_scale_f16(int64_t rows, int64_t k, const void *x, int x_dtype, float *scales, void *x16,
                      const int32_t *tile_info, qmm_stream_t stream) {
  return row_scale(rows, k, x, x_dtype, scales, x16, tile_info, nullptr, reinterpret_cast<hipStream_t>(stream));
}

int qmm_row_scale_f16_rows(int64_t n, const int32_t *rows, int64_t k, const void *x, int x_dtype, float *scales,
                           void *x16, qmm_stream_t stream) {
  if (!rows) return QMM_ERR_NULL;
  return row_scale(n, k, x, x_dtype, scales, x16, nullptr, nullptr, reinterpret_cast<hipStream_t>(stream), rows);
}

int qmm_row_scale_f16_live(int64_t rows, const int32_t *info, int64_t k, const void *x, int x_dtype, float *scales,
                           void *x16, qmm_stream_t stream) {
  if (!info) return QMM_ERR_NULL;
  return row_scale(rows, k, x, x_dtype, scales, x16, nullptr, info, reinterpret_cast<hipStream_t>(stream));
}

int qmm_quant_mxfp8(int64_t rows, int64_t k, const void *x, int x_dtype, const int32_t *tile_info, uint8_t *codes,
                    uint8_t *scales, qmm_stream_t stream) {
  if (!x || !codes || !scales) return QMM_ERR_NULL;
  if (x_dtype != QMM_F32 && x_dtype != QMM_BF16) return QMM_ERR_DTYPE;
  if (rows <= 0 || k <= 0 || k % kMxBlock || rows > (1ll << 24)) return QMM_ERR_SHAPE;
  if (tile_info && rows % kTile) return QMM_ERR_SHAPE;
  if (!aligned(x, 16) || !aligned(codes, 16)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == QMM_BF16) {
    const int64_t pieces = rows * (k / 8);
    quant_mxfp8_vec_kernel<true><<<(unsigned)((pieces + 255) / 256), 256, 0, s>>>(rows, k, x, tile_info, codes, scales);
  } else {
    const int64_t pieces = rows * (k / 4);
    quant_mxfp8_vec_kernel<false><<<(unsigned)((pieces + 255) / 256), 256, 0, s>>>(rows, k, x, tile_info, codes, scales);
  }
  return launch_status();
}

int qmm_repack_mxfp4(const void *w, int64_t rows, int64_t k, uint8_t *nibbles, uint8_t *scales, qmm_stream_t stream) {
  if (!w || !nibbles || !scales) return QMM_ERR_NULL;
  if (rows <= 0 || k <= 0 || k % 32) return QMM_ERR_SHAPE;
  if (!aligned(nibbles, 16)) return QMM_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t groups = rows * (k / 32);
  repack_mxfp4_kernel<<<(unsigned)((groups + 255) / 256), 256, 0, s>>>(groups, static_cast<const u8 *>(w), nibbles,
                                                                       scales);
  return launch_status();
}

}  // extern "C"
