// Transposed butterfly reductions of several values per lane over groups of 32 or 64 lanes (wave64), shared by
// the decode matvecs: every value goes through the same tree of lane pairs whatever their number, so results do
// not depend on how many tokens or rows a call carries.
#pragma once
#include "common.hpp"

namespace qmm {

// v from the butterfly partner at distance D: DPP quad permutes for 1 and 2, half-row / row mirrors for 4 and 8
// (they pair lanes that differ in that bit, which is all a butterfly needs), ds_swizzle for 16, ds_bpermute for 32.
template <int D>
__device__ __forceinline__ float xshfl(float v) {
  const int i = __builtin_bit_cast(int, v);
  int r;
  if constexpr (D == 1) r = __builtin_amdgcn_update_dpp(0, i, 0xB1, 0xF, 0xF, false);
  else if constexpr (D == 2) r = __builtin_amdgcn_update_dpp(0, i, 0x4E, 0xF, 0xF, false);
  else if constexpr (D == 4) r = __builtin_amdgcn_update_dpp(0, i, 0x141, 0xF, 0xF, false);
  else if constexpr (D == 8) r = __builtin_amdgcn_update_dpp(0, i, 0x140, 0xF, 0xF, false);
  else if constexpr (D == 16) r = __builtin_amdgcn_ds_swizzle(i, 0x401F);
  else r = __builtin_amdgcn_ds_bpermute((int)((threadIdx.x ^ 32u) << 2), i);
  return __builtin_bit_cast(float, r);
}

// One butterfly step at distance D. While more than one value is left (cnt > 1) the step halves them: a lane
// whose D bit is set keeps the upper half and adds its partner's copy of it. Afterwards it reduces fully.
template <int NV, int D>
__device__ __forceinline__ void bfly_step(float (&v)[NV], int &cnt, int &base, int lane) {
  const bool up = (lane & D) != 0;
  if (cnt > 1) {
    const int half = cnt >> 1;
#pragma unroll
    for (int i = 0; i < NV / 2; ++i) {
      if (i < half) {
        const float send = up ? v[i] : v[half + i];
        const float keep = up ? v[half + i] : v[i];
        v[i] = keep + xshfl<D>(send);
      }
    }
    if (up) base += half;
    cnt = half;
  } else {
    v[0] += xshfl<D>(v[0]);
  }
}

// Sums NV values per lane over groups of L lanes (L = 32 or 64). Every value goes through the same tree of
// lane pairs whatever NV is. Returns the lane's owned value; its index is `owned`.
template <int NV, int L>
__device__ __forceinline__ float group_reduce(float (&v)[NV], int lane, int &owned) {
  static_assert((NV & (NV - 1)) == 0 && NV <= L, "values per lane must be a power of two");
  int cnt = NV, base = 0;
  if constexpr (L == 64) bfly_step<NV, 32>(v, cnt, base, lane);
  bfly_step<NV, 16>(v, cnt, base, lane);
  bfly_step<NV, 8>(v, cnt, base, lane);
  bfly_step<NV, 4>(v, cnt, base, lane);
  bfly_step<NV, 2>(v, cnt, base, lane);
  bfly_step<NV, 1>(v, cnt, base, lane);
  owned = base;
  return v[0];
}

constexpr int log2i(int v) { return v <= 1 ? 0 : 1 + log2i(v / 2); }

}  // namespace qmm
