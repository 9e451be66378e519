// The mean-log gate's per-node work shared by its kernels and the fused decode descent: the gate of one node
// (gate_node_wave) and the decode append's log sums and gated vectors of the nodes ending at a position
// (gate_append_wave).  Every float operation here is rounded on its own (no contraction), as the gate's
// CPU restatement computes it.
#pragma once

#include "append.hpp"
#include "common.hpp"

namespace ta {

__device__ __forceinline__ float index_log(float x) {
#pragma clang fp contract(off)
  return (float)log((double)(fabsf(x) + 1e-6f)); }

// Gate of one node held by one wavefront: dimension d = lane + 64 i (i < EPL) in raw[i], lg[i] (lanes past D
// hold nothing).  lo / w: the quantile's lower order statistic and interpolation weight.  Returns the gated
// values in g[i].
template <int D>
__device__ __forceinline__ void gate_node_wave(const float (&raw)[(D + 63) / 64], const float (&lg)[(D + 63) / 64],
                                               float inv_size, int lo, float w, float (&g)[(D + 63) / 64]) {
#pragma clang fp contract(off)
  constexpr int EPL = (D + 63) / 64;
  const int lane = lane_id();
  float ml[EPL];
  int rank[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    ml[i] = lg[i] * inv_size;   // size is a power of two: the division is exact
    rank[i] = 0;
  }
  // rank of each value among the D (ties broken by dimension): the sorted order's position
#pragma unroll
  for (int i2 = 0; i2 < EPL; ++i2) {
    for (int e = 0; e < 64; ++e) {
      const int d2 = e + 64 * i2;
      const float o = __shfl(ml[i2], e, kWave);
      if (d2 < D) {
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const int d = lane + 64 * i;
          rank[i] += (o < ml[i] || (o == ml[i] && d2 < d)) ? 1 : 0;
        }
      }
    }
  }
  const int hi = w > 0.0f ? lo + 1 : lo;
  float vlo = 0.0f, vhi = 0.0f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const bool in = lane + 64 * i < D;
    const uint64_t blo = __ballot(in && rank[i] == lo), bhi = __ballot(in && rank[i] == hi);
    if (blo) vlo = __shfl(ml[i], __ffsll((unsigned long long)blo) - 1, kWave);
    if (bhi) vhi = __shfl(ml[i], __ffsll((unsigned long long)bhi) - 1, kWave);
  }
  const float thr = w < 0.5f ? vlo + w * (vhi - vlo) : vhi - (vhi - vlo) * (1.0f - w);
  int kept = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) kept += __popcll(__ballot(lane + 64 * i < D && ml[i] >= thr));
  const float scale = (float)D / (float)(kept > 1 ? kept : 1);
#pragma unroll
  for (int i = 0; i < EPL; ++i) g[i] = (raw[i] * (ml[i] >= thr ? 1.0f : 0.0f)) * scale;
}

struct GateLevels {
  const float* raw[kMaxLevels];
  const float* lg[kMaxLevels];
  float* out[kMaxLevels];   // null: the level is not gated
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
  int64_t n_nodes[kMaxLevels];
  int blevel[kMaxLevels];
};

// quantile position of gate_q over D values as torch.quantile computes it in float32 (lo, interpolation weight w)
void gate_rank(float gate_q, int D, int& lo, float& w);

// The levels a gate append works on, as GateLevels holds them.
struct GateLevelsView {
  const GateLevels& g;
  __device__ __forceinline__ const float* raw(int j) const { return g.raw[j]; }
  __device__ __forceinline__ float* lg(int j) const { return const_cast<float*>(g.lg[j]); }
  __device__ __forceinline__ float* out(int j) const { return g.out[j]; }
  __device__ __forceinline__ int64_t sb(int j) const { return g.sb[j]; }
  __device__ __forceinline__ int64_t sh(int j) const { return g.sh[j]; }
  __device__ __forceinline__ int blevel(int j) const { return g.blevel[j]; }
};

// Decode append of the gate, by one wavefront for (sequence b, head h) at position t, after the cache append of
// row t (raw nodes ending at t already formed): the log sums of the nodes ending at t (the leaf block's keys read
// back from the cache), then the gated vectors of those nodes on gated levels.  Lane d (and d + 64) keeps
// dimension d's carry stack in registers: at most 2 + log2(arity) entries per level are live, so a fixed
// 20-entry stack covers leaf blocks up to 2^14 and any arity.  LV: raw / lg / out / sb / sh / blevel per level.
template <typename T, int D, typename LV>
__device__ __forceinline__ void gate_append_wave(const AppendIn& ap, const LV& gl, int n_levels, int arity_log2,
                                                 int b, int h, int t, int lo, float w) {
#pragma clang fp contract(off)
  constexpr int EPL = (D + 63) / 64;
  if (t < 0 || t >= ap.Tcap || n_levels == 0) return;
  const int leaf_log2 = gl.blevel(0);
  const int leaf = 1 << leaf_log2;
  if (((t + 1) & (leaf - 1)) != 0) return;   // no node ends at t
  const int lane = lane_id();
  T *kbase, *vbase;
  const KvRows rows = append_rows<T>(ap, b, h, leaf_log2, kbase, vbase);
  const int64_t ot = rows.off(t);
  if (ot < 0) return;
  const int64_t ob = ot - (int64_t)(leaf - 1) * rows.cst;   // row t + 1 - leaf of the block's page
  const int p0 = t + 1 - leaf;
  float stk[EPL][20];
  float y[EPL];
  // leaf block: log-magnitudes of its index keys (position 0 counted as 0), adjacent pairs with a carry stack
  for (int i = 0; i < leaf; ++i) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int d = lane + 64 * e;
      const float kv = d < D && p0 + i > 0 ? to_f32(kbase[ob + (int64_t)i * rows.cst + d]) : 0.0f;
      float x = index_log(kv);
      int lvl = 0;
      while ((i >> lvl) & 1) {
        x = __fadd_rn(stk[e][lvl], x);
        ++lvl;
      }
      stk[e][lvl] = x;
      y[e] = x;
    }
  }
  auto emit = [&](int j, int64_t node) {
    const int64_t o = b * gl.sb(j) + h * gl.sh(j) + node * D;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (lane + 64 * e < D) gl.lg(j)[o + lane + 64 * e] = y[e];
    if (gl.out(j) != nullptr) {
      float raw[EPL], g[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) raw[e] = lane + 64 * e < D ? gl.raw(j)[o + lane + 64 * e] : 0.0f;
      gate_node_wave<D>(raw, y, 1.0f / (float)(1ll << gl.blevel(j)), lo, w, g);
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        if (lane + 64 * e < D) gl.out(j)[o + lane + 64 * e] = g[e];
    }
  };
  emit(0, t >> leaf_log2);
  const int arity = 1 << arity_log2;
  for (int j = 1; j < n_levels; ++j) {
    const int lj = gl.blevel(j);
    if (((t + 1) & ((1 << lj) - 1)) != 0) break;
    const int64_t node = t >> lj;
    const float* child = gl.lg(j - 1) + b * gl.sb(j - 1) + h * gl.sh(j - 1) + node * arity * D;
    for (int c = 0; c < arity; ++c) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e;
        float x = d < D ? child[(int64_t)c * D + d] : 0.0f;
        int lvl = 0;
        while ((c >> lvl) & 1) {
          x = __fadd_rn(stk[e][lvl], x);
          ++lvl;
        }
        stk[e][lvl] = x;
        y[e] = x;
      }
    }
    emit(j, node);
  }
}

}  // namespace ta
