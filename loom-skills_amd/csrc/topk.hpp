// Top-k routing of one token by one wave (g_moe_route, S/gen_moe.py:116-500): shared by the routing kernels
// (moe_route.hip) and the decode gate/up expert matvec that routes its own token (gemv.hip).
#pragma once

#include "common.hpp"

namespace qmm {

constexpr float kNormFloor = 6.103515625e-05f;

// ------------------------------------------------------------------------------------------------- top-k
// One wave per token; lane l holds experts l, l + 64, ... (NS = ceil(E / 64) slots). The selection is a ranking: the
// wave writes each expert's selection key to LDS and every lane counts, for each of its experts, how many experts
// beat it; an expert of rank r < KU is pick r. A key orders (score, expert) as the reference's workgroup max then
// min-index does (S/gen_moe.py:219-235): the score's bits mapped to an order-preserving u32 (after -0 -> +0, so equal
// scores tie) in the high word and 0xFFFFFFFF - expert in the low word, so "higher score, ties to the lower id" is one
// unsigned 64-bit compare. The score is the logit (+ bias) for gating 1 and 3 and for gating 2 without a bias: those
// selections are monotone in the logit, so choosing on the exact f32 logit reproduces the float64 oracle's choice.
__device__ __forceinline__ uint64_t select_key(float v, int e) {
  const u32 u = f32_as_u32(v + 0.f);
  const u32 o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - (u32)e);
}

constexpr int kTopkMaxE = 256;

// The selection and weights of one token by one wave: lane l's experts l + 64 i with pick[i] have rank[i] < KU
// (pick rank[i] of the token) and weight wo[i]. keys: the wave's table of 64 NS selection keys in LDS.
template <int NS>
__device__ __forceinline__ void topk_select(const float *__restrict__ lg, int E, int KU, int gating, int norm,
                                            float scale, const float *__restrict__ bias, uint64_t *keys,
                                            int (&rank)[NS], float (&wo)[NS], bool (&pick)[NS]) {
  const int lane = threadIdx.x & 63;
  float l[NS], bv[NS];
  bool in[NS];
  const float NEG = -3.0e38f;
  // every logit and bias load is issued before any is used (a lane past E reloads expert E - 1 and ignores it)
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int e = lane + 64 * i;
    in[i] = e < E;
    l[i] = lg[in[i] ? e : E - 1];
    bv[i] = bias ? bias[in[i] ? e : E - 1] : 0.f;
  }
  uint64_t key[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int e = lane + 64 * i;
    l[i] = in[i] ? l[i] : NEG;
    const float b = in[i] ? bv[i] : 0.f;
    if (gating == 3) l[i] = in[i] ? l[i] + b : NEG;   // the router bias is part of the logit (gating 3)
    float sv = l[i];
    if (gating == 2 && bias) sv = in[i] ? 1.f / (1.f + expf(-l[i])) + b : NEG;
    key[i] = in[i] ? select_key(sv, e) : 0ull;   // experts past E rank below every real one
    keys[e] = key[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < NS; ++i) rank[i] = 0;
  // every slot of the table is ranked against (those past E hold key 0 and beat nothing): a static trip count, so
  // the LDS reads are issued ahead of their use
#pragma unroll 16
  for (int e2 = 0; e2 < 64 * NS; e2 += 2) {
    typedef __attribute__((ext_vector_type(2))) uint64_t u64x2;
    const u64x2 q = *reinterpret_cast<const u64x2 *>(&keys[e2]);
#pragma unroll
    for (int i = 0; i < NS; ++i) rank[i] += (q.x > key[i] ? 1 : 0) + (q.y > key[i] ? 1 : 0);
  }
  // the weights: probabilities over all experts (gating 1), sigmoids (gating 2) or a softmax over the picks (3)
  float lmax = l[0];
#pragma unroll
  for (int i = 1; i < NS; ++i) lmax = fmaxf(lmax, l[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, off, 64));
  float w[NS], ws = 0.f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    pick[i] = in[i] && rank[i] < KU;
    const float ex = in[i] ? expf(l[i] - lmax) : 0.f;
    w[i] = gating == 2 ? 1.f / (1.f + expf(-l[i])) : ex;
    ws += gating == 1 ? ex : (pick[i] ? w[i] : 0.f);
  }
  float den = wave_sum(ws);                // gating 1: the softmax denominator; 3: the picks' sum; 2: the sum
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (gating != 2) w[i] = w[i] / den;
    sum += pick[i] ? w[i] : 0.f;
  }
  const float nden = norm ? fmaxf(gating == 2 ? den : wave_sum(sum), kNormFloor) : 1.f;
#pragma unroll
  for (int i = 0; i < NS; ++i) wo[i] = (norm ? w[i] / nden : w[i]) * scale;
}

// The selection and weights of token t by one wave, written to ids / wts [tokens, KU] in rank order.
template <int NS>
__device__ __forceinline__ void topk_token(const float *__restrict__ lg, int64_t t, int E, int KU, int gating,
                                           int norm, float scale, const float *__restrict__ bias, uint64_t *keys,
                                           int32_t *__restrict__ ids, float *__restrict__ wts) {
  const int lane = threadIdx.x & 63;
  int rank[NS];
  float wo[NS];
  bool pick[NS];
  topk_select<NS>(lg, E, KU, gating, norm, scale, bias, keys, rank, wo, pick);
#pragma unroll
  for (int i = 0; i < NS; ++i)
    if (pick[i]) {
      ids[t * KU + rank[i]] = lane + 64 * i;
      wts[t * KU + rank[i]] = wo[i];
    }
}

// Pick j of the token selected by topk_select, as wave-uniform values: its expert and weight.
template <int NS>
__device__ __forceinline__ void topk_pick(const int (&rank)[NS], const float (&wo)[NS], const bool (&pick)[NS], int j,
                                          int &expert, float &weight) {
  const int lane = threadIdx.x & 63;
  int e = 0;
  float w = 0.f;
  bool mine = false;
#pragma unroll
  for (int i = 0; i < NS; ++i)
    if (pick[i] && rank[i] == j) { e = lane + 64 * i; w = wo[i]; mine = true; }
  const uint64_t m = __ballot(mine);
  const int src = m ? __builtin_ctzll(m) : 0;
  expert = __builtin_amdgcn_readlane(e, src);
  weight = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), src));
}

// The routing of a gate/up matvec that selects its own experts: every wave ranks its token's logits (topk_select, the
// routing kernels' arithmetic) and takes pick a % KU; one wave of the assignment's first workgroup writes ids / wts.
struct RouteArgs {
  const float *logits;   // [tokens, E]
  int gating, norm;
  float scale;
  const float *bias;     // router bias [E] or NULL
  int32_t *ids;          // out: [tokens, KU]
  float *wts;            // out: [tokens, KU]
};

}  // namespace qmm
