// Decode-cache append (replaces SegState.add, engine.py:41-55), shared by the standalone append kernel and
// the fused descent + append kernel.
#pragma once

#include "common.hpp"

namespace ta {

// The new rows of a decode step and the caches they go to (element strides).  Paged caches (ptab != null):
// leaf block j of (b, h) is page ptab[b * pt_sb + h * pt_sh + j] (valid when in [0, npages)), its row r at
// Kc + page * pstride + r * cst (Vc likewise); csb and csh are unused.
struct AppendIn {
  const void* kn;
  const void* vn;
  int64_t nsb, nsh, vnsb, vnsh;
  void* Kc;
  void* Vc;
  int64_t csb, csh, cst;
  int Tcap;
  const int32_t* ptab;
  int64_t pt_sb, pt_sh, pstride, npages;
};

// Where the rows of one (sequence, head) of a decode cache are.  Dense: row pos at base + pos * cst.  Paged:
// leaf block pos >> blog2 is page table[pos >> blog2], row pos at base + page * pstride + (pos mod 2^blog2) * cst;
// a position whose page is outside [0, npages) has no row (off returns -1).
struct KvRows {
  const int32_t* table;   // this (sequence, head)'s page ids (null: dense)
  int64_t cst, pstride, npages;
  int blog2;
  __device__ __forceinline__ int64_t off(int pos) const {
    if (table == nullptr) return (int64_t)pos * cst;
    const int pg = table[pos >> blog2];
    if (pg < 0 || pg >= npages) return -1;
    return (int64_t)pg * pstride + (int64_t)(pos & ((1 << blog2) - 1)) * cst;
  }
};

// The rows and bases of (b, h) in the caches of ap (leaf blocks of 2^leaf_log2 rows).
template <typename T>
__device__ __forceinline__ KvRows append_rows(const AppendIn& ap, int b, int h, int leaf_log2, T*& kbase, T*& vbase) {
  KvRows r{};
  r.cst = ap.cst;
  r.blog2 = leaf_log2;
  if (ap.ptab) {
    r.table = ap.ptab + b * ap.pt_sb + h * ap.pt_sh;
    r.pstride = ap.pstride;
    r.npages = ap.npages;
    kbase = reinterpret_cast<T*>(ap.Kc);
    vbase = reinterpret_cast<T*>(ap.Vc);
  } else {
    kbase = reinterpret_cast<T*>(ap.Kc) + b * ap.csb + h * ap.csh;
    vbase = reinterpret_cast<T*>(ap.Vc) + b * ap.csb + h * ap.csh;
  }
  return r;
}

// Dimension d of one (sequence, head): writes row t of the K and V caches, then forms the nodes whose last
// position is t -- the leaf block from its keys (position 0 counted as 0), each higher node from its
// children -- as adjacent-pair float32 sums with a carry stack (stk: 16 entries per dimension, stride D).
// kbase/vbase and rows locate the rows of this (sequence, head) in the caches (rows.blog2 = leaf_log2); a
// row without a page is not written.  level(j) returns tree level j's node rows (D floats each) for this
// (sequence, head); tree level j has binary level leaf_log2 + j * arity_log2.
// The loads append_dim starts with (dimension d of the new K and V rows, row t's offset in the caches), split
// off so that a caller can issue them early and store later (append_dim_with).
template <typename T>
struct AppendPre {
  T kx, vx;
  int64_t ot;
};
template <typename T>
__device__ __forceinline__ AppendPre<T> append_prefetch(int d, int t, const T* __restrict__ kn,
                                                        const T* __restrict__ vn, const KvRows& rows) {
  return AppendPre<T>{kn[d], vn[d], rows.off(t)};
}

template <typename T, typename LevelFn>
__device__ __forceinline__ void append_dim_with(int d, int D, int t, const AppendPre<T>& pre, T* kbase, T* vbase,
                                                const KvRows& rows, int n_levels, int leaf_log2, int arity_log2,
                                                float* stk, LevelFn level) {
  const T kx = pre.kx;
  const int64_t ot = pre.ot;
  if (ot < 0) return;   // no page for row t: nothing stored, no node formed
  kbase[ot + d] = kx;
  vbase[ot + d] = pre.vx;
  if (n_levels == 0) return;
  const int leaf = 1 << leaf_log2;
  if (((t + 1) & (leaf - 1)) != 0) return;
  // leaf block [t + 1 - leaf, t] (one page); its keys are read 8 at a time with every load in flight before
  // the sums
  const int p0 = t + 1 - leaf;
  const int64_t ob = ot - (int64_t)(leaf - 1) * rows.cst;   // row p0 of the block's page
  float x = 0.0f;
  for (int i0 = 0; i0 < leaf; i0 += 8) {
    float kv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int pp = p0 + i0 + u;
      kv[u] = i0 + u < leaf && pp < t ? to_f32(kbase[ob + (int64_t)(i0 + u) * rows.cst + d]) : 0.0f;
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

template <typename T, typename LevelFn>
__device__ __forceinline__ void append_dim(int d, int D, int t, const T* __restrict__ kn, const T* __restrict__ vn,
                                           T* kbase, T* vbase, const KvRows& rows, int n_levels, int leaf_log2,
                                           int arity_log2, float* stk, LevelFn level) {
  append_dim_with<T>(d, D, t, append_prefetch<T>(d, t, kn, vn, rows), kbase, vbase, rows, n_levels, leaf_log2,
                     arity_log2, stk, level);
}

}  // namespace ta
