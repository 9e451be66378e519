// Canonical-order reductions held by one wavefront, shared by the block forest (forest.hip) and the LaneTree
// (lanetree.hip).  Each gives the value the CPU oracle's canonical mode computes, bit for bit, provided the
// including file turns floating-point contraction off.
#pragma once

#include "common.hpp"

namespace ta {

// canon_dot's value for two D-vectors held by one lane (fa(i), fb(i) give element i): groups of D/16 (at least
// 1) consecutive products reduced by the halving tree, then the halving tree over the (at most 16) groups.
template <int D, typename FA, typename FB>
__device__ __forceinline__ float lane_dot(FA fa, FB fb) {
  constexpr int G = D < 16 ? D : 16, R = D / G;
  float g[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float p[R];
#pragma unroll
    for (int i = 0; i < R; ++i) p[i] = fa(R * j + i) * fb(R * j + i);
#pragma unroll
    for (int n = R / 2; n >= 1; n /= 2)
#pragma unroll
      for (int i = 0; i < n; ++i) p[i] = p[i] + p[i + n];
    g[j] = p[0];
  }
#pragma unroll
  for (int n = G / 2; n >= 1; n /= 2)
#pragma unroll
    for (int i = 0; i < n; ++i) g[i] = g[i] + g[i + n];
  return g[0];
}

// The 32-bit value of lane (this lane ^ H), without the LDS crossbar: xor 1 and 2 by DPP quad permutes, xor 4 by
// a 16-lane row rotate by 4 or 12 (the one that lands on the partner), xor 8 by a row rotate by 8, xor 16 and 32
// by the gfx950 lane swaps (v_permlane16_swap / v_permlane32_swap of the value with itself; the swapped copy
// holds the partner's value in this lane).
template <int H>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v) {
  const int x = (int)v;
  if constexpr (H == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
  } else if constexpr (H == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
  } else if constexpr (H == 4) {
    const uint32_t r4 = (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false);
    const uint32_t r12 = (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x12C, 0xF, 0xF, false);
    return (threadIdx.x & 4) ? r4 : r12;
  } else if constexpr (H == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
  } else if constexpr (H == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? s[0] : s[1];
  } else {
    static_assert(H == 32, "xor distance 1..32");
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? s[0] : s[1];
  }
}
template <int H>
__device__ __forceinline__ float xor_lane(float v) { return __uint_as_float(xor_lane_u32<H>(__float_as_uint(v))); }
template <int H>
__device__ __forceinline__ int xor_lane(int v) { return (int)xor_lane_u32<H>((uint32_t)v); }

// Sum over the aligned S-lane segment holding this lane, by the halving tree over the segment's lanes in order
// (every lane returns the same value: each step adds the lane at distance h, and float addition commutes).
__device__ __forceinline__ float seg_sum(float v, int S) {
  if (S > 32) v = v + xor_lane<32>(v);
  if (S > 16) v = v + xor_lane<16>(v);
  if (S > 8) v = v + xor_lane<8>(v);
  if (S > 4) v = v + xor_lane<4>(v);
  if (S > 2) v = v + xor_lane<2>(v);
  if (S > 1) v = v + xor_lane<1>(v);
  return v;
}
__device__ __forceinline__ float seg_max(float v, int S) {
  if (S > 32) v = fmaxf(v, xor_lane<32>(v));
  if (S > 16) v = fmaxf(v, xor_lane<16>(v));
  if (S > 8) v = fmaxf(v, xor_lane<8>(v));
  if (S > 4) v = fmaxf(v, xor_lane<4>(v));
  if (S > 2) v = fmaxf(v, xor_lane<2>(v));
  if (S > 1) v = fmaxf(v, xor_lane<1>(v));
  return v;
}
// The first lane of the segment [gb, gb + S) whose v equals the segment's maximum.
__device__ __forceinline__ int seg_argmax_first(float v, int gb, int S) {
  const float mx = seg_max(v, S);
  const uint64_t seg = S >= 64 ? ~0ull : (((1ull << S) - 1) << gb);
  return __ffsll((unsigned long long)(__ballot(v == mx) & seg)) - 1;
}

}  // namespace ta
