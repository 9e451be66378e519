// Decode-cache append (replaces SegState.add, engine.py:41-55), shared by the standalone append kernel and
// the fused descent + append kernel.
#pragma once

#include "common.hpp"

namespace ta {

// The new rows of a decode step and the caches they go to (element strides).
struct AppendIn {
  const void* kn;
  const void* vn;
  int64_t nsb, nsh, vnsb, vnsh;
  void* Kc;
  void* Vc;
  int64_t csb, csh, cst;
  int Tcap;
};

// Dimension d of one (sequence, head): writes row t of the K and V caches, then forms the nodes whose last
// position is t -- the leaf block from its keys (position 0 counted as 0), each higher node from its
// children -- as adjacent-pair float32 sums with a carry stack (stk: 16 entries per dimension, stride D).
// krow/vrow point at row 0 of this (sequence, head) in the caches, row stride cst.  level(j) returns tree
// level j's node rows (D floats each) for this (sequence, head); tree level j has binary level
// leaf_log2 + j * arity_log2.
template <typename T, typename LevelFn>
__device__ __forceinline__ void append_dim(int d, int D, int t, const T* __restrict__ kn, const T* __restrict__ vn,
                                           T* krow, T* vrow, int64_t cst, int n_levels, int leaf_log2,
                                           int arity_log2, float* stk, LevelFn level) {
  const T kx = kn[d];
  krow[(int64_t)t * cst + d] = kx;
  vrow[(int64_t)t * cst + d] = vn[d];
  if (n_levels == 0) return;
  const int leaf = 1 << leaf_log2;
  if (((t + 1) & (leaf - 1)) != 0) return;
  // leaf block [t + 1 - leaf, t]; its keys are read 8 at a time with every load in flight before the sums
  const int p0 = t + 1 - leaf;
  float x = 0.0f;
  for (int i0 = 0; i0 < leaf; i0 += 8) {
    float kv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int pp = p0 + i0 + u;
      kv[u] = i0 + u < leaf && pp < t ? to_f32(krow[(int64_t)pp * cst + d]) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u;
      if (i >= leaf) break;
      const int pp = p0 + i;
      x = pp == 0 ? 0.0f : (pp == t ? to_f32(kx) : kv[u]);
      int lvl = 0;
      while ((i >> lvl) & 1) {
        x = __fadd_rn(stk[lvl * D + d], x);
        ++lvl;
      }
      stk[lvl * D + d] = x;
    }
  }
  level(0)[(int64_t)(t >> leaf_log2) * D + d] = x;
  const int arity = 1 << arity_log2;
  for (int j = 1; j < n_levels; ++j) {
    const int lj = leaf_log2 + j * arity_log2;
    if (((t + 1) & ((1 << lj) - 1)) != 0) break;
    const int64_t node = t >> lj;
    const float* child = level(j - 1) + node * arity * D + d;
    for (int c = 0; c < arity; ++c) {
      x = child[(int64_t)c * D];
      int lvl = 0;
      while ((c >> lvl) & 1) {
        x = __fadd_rn(stk[lvl * D + d], x);
        ++lvl;
      }
      stk[lvl * D + d] = x;
    }
    level(j)[node * D + d] = x;
  }
}

}  // namespace ta
