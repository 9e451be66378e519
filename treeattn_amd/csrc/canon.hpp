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

// Sum over the aligned S-lane segment holding this lane, by the halving tree over the segment's lanes in order
// (every lane returns the same value: each step adds the lane at distance h, and float addition commutes).
__device__ __forceinline__ float seg_sum(float v, int S) {
  for (int h = S >> 1; h >= 1; h >>= 1) v = v + __shfl_xor(v, h, kWave);
  return v;
}
__device__ __forceinline__ float seg_max(float v, int S) {
  for (int h = S >> 1; h >= 1; h >>= 1) v = fmaxf(v, __shfl_xor(v, h, kWave));
  return v;
}
// The first lane of the segment [gb, gb + S) whose v equals the segment's maximum.
__device__ __forceinline__ int seg_argmax_first(float v, int gb, int S) {
  const float mx = seg_max(v, S);
  const uint64_t seg = S >= 64 ? ~0ull : (((1ull << S) - 1) << gb);
  return __ffsll((unsigned long long)(__ballot(v == mx) & seg)) - 1;
}

}  // namespace ta
