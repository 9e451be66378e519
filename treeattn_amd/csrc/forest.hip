// Block forest: one content-sorted binary tree per block of `block` keys, and a beam descent over the trees of
// the blocks before the query's own (the reference's default attention, attn='block').
//
// Reference functions replaced: forest.py:12-33 two_means_order, forest.py:36-44 soft_gate, forest.py:47-75
// build_forest, and attention.py:88-148 (the descent over the block trees, the budget's cut, leaves to key
// positions, the static keys and their duplicates).  The attention over the candidate list this produces is
// ta_sparse_attn_fwd / ta_sparse_attn_bwd.
//
// Arithmetic order (the CPU oracle's canonical mode computes the same, bit for bit):
//  * a 2-means mean or centroid over the S members of a group: the halving tree over the members in group order
//    (member i + member i + S/2, then + S/4, ...), then the division by the member count;
//  * node sums and the gate's log-magnitude sums: adjacent pairs, ((x0 + x1) + (x2 + x3)) + ...;
//  * dot products and squared distances: per-dimension float32 products in canon_dot's order;
//    dist = (|x|^2 - 2 x.c) + |c|^2;
//  * argmax / argmin: the first index; the member order: stable ascending sort of the projections;
//  * soft gate: the float32 rounding of the double-precision log and logistic, the threshold as
//    torch.quantile's linear interpolation in float32, the kept mass by the halving tree over dimensions;
//  * descent ranking: valid first, score descending, node id ascending (invalid candidates by slot).
// Node sums are float32 whatever the key type.
#pragma clang fp contract(off)

#include "canon.hpp"
#include "descend.hpp"

namespace ta {

constexpr int kForestMaxRoots = 1024;   // blocks per sequence the descent ranks at its first level
constexpr int kForestMaxW = 64;         // wmax

__device__ __forceinline__ float forest_log(float x) { return (float)log((double)(fabsf(x) + 1e-6f)); }

// seg_sum of every element of v (the same butterfly per element), step-major so the shuffles of all D
// elements are in flight together.
template <int H, int D>
__device__ __forceinline__ void seg_sum_rows_step(float (&v)[D]) {
#pragma unroll
  for (int d = 0; d < D; ++d) v[d] = v[d] + xor_lane<H>(v[d]);
}
template <int D>
__device__ __forceinline__ void seg_sum_rows(float (&v)[D], int S) {
  if (S > 32) seg_sum_rows_step<32>(v);
  if (S > 16) seg_sum_rows_step<16>(v);
  if (S > 8) seg_sum_rows_step<8>(v);
  if (S > 4) seg_sum_rows_step<4>(v);
  if (S > 2) seg_sum_rows_step<2>(v);
  if (S > 1) seg_sum_rows_step<1>(v);
}

struct ForestLevels {
  float* sums[kMaxLevels];   // level l: (B, H, nb << l, D) float32, node rows contiguous
  float* lg[kMaxLevels];     // the gate's log-magnitude sums (null without the gate)
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
};

// One wavefront per (sequence, head, block); lane i holds the key at rank i of the block's current order.
// Every level splits each group of S = block >> lvl consecutive ranks by a 2-means projection (forest.py:12-33):
// the members are re-ranked inside the group, so the next level's groups are the halves.  Then the node sums
// of every level by adjacent pairs (and, with the gate, the log-magnitude sums the same way).
template <typename T, int D>
__global__ __launch_bounds__(kWave) void forest_build_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                                             int64_t kst, int H, int nb, int Bk, int depth,
                                                             int iters, int gate, int32_t* __restrict__ perm,
                                                             ForestLevels lv) {
  constexpr int DP = D + 1;   // LDS row stride of the reorder buffer
  __shared__ float s_x[kWave * DP];
  __shared__ int s_p[kWave];
  __shared__ __align__(16) float s_pr[kWave];   // the level's projections
  const int lane = lane_id();
  const int pb = blockIdx.x, blk = pb % nb, bh = pb / nb, b = bh / H, h = bh % H;
  const bool live = lane < Bk;
  const int64_t pos = (int64_t)blk * Bk + (live ? lane : 0);
  float x[D];
  load_row_g<T, D>(k + b * ksb + h * ksh + pos * kst, x);
#pragma unroll
  for (int d = 0; d < D; ++d) x[d] = live ? (pos == 0 ? x[d] * 0.0f : x[d]) : 0.0f;   // the sink: k * 0
  int p = lane;

  float c0[D], c1[D], t[D];
  for (int lvl = 0; lvl < depth; ++lvl) {
    const int S = Bk >> lvl, gb = lane & ~(S - 1), li = lane - gb;
    // the group mean, then the member farthest from it (a) and the member farthest from a (b)
#pragma unroll
    for (int d = 0; d < D; ++d) c0[d] = x[d];
    seg_sum_rows<D>(c0, S);
#pragma unroll
    for (int d = 0; d < D; ++d) c0[d] = c0[d] / (float)S;
    const float d2 = lane_dot<D>([&](int i) { return x[i] - c0[i]; }, [&](int i) { return x[i] - c0[i]; });
    const int la = seg_argmax_first(d2, gb, S);
#pragma unroll
    for (int d = 0; d < D; ++d) c0[d] = __shfl(x[d], la, kWave);
    const float d2b = lane_dot<D>([&](int i) { return x[i] - c0[i]; }, [&](int i) { return x[i] - c0[i]; });
    const int lb = seg_argmax_first(d2b, gb, S);
#pragma unroll
    for (int d = 0; d < D; ++d) c1[d] = __shfl(x[d], lb, kWave);
    const float xx = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return x[i]; });
    for (int it = 0; it < iters; ++it) {
      const float cc0 = lane_dot<D>([&](int i) { return c0[i]; }, [&](int i) { return c0[i]; });
      const float cc1 = lane_dot<D>([&](int i) { return c1[i]; }, [&](int i) { return c1[i]; });
      const float xc0 = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c0[i]; });
      const float xc1 = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c1[i]; });
      const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
      const bool lab1 = dist1 < dist0;   // argmin over the two centroids, the first on ties
      const float m0 = lab1 ? 0.0f : 1.0f, m1 = lab1 ? 1.0f : 0.0f;
      const float cnt0 = seg_sum(m0, S), cnt1 = seg_sum(m1, S);
      const float den0 = fmaxf(cnt0, 1.0f), den1 = fmaxf(cnt1, 1.0f);
#pragma unroll
      for (int d = 0; d < D; ++d) t[d] = x[d] * m0;
      seg_sum_rows<D>(t, S);
#pragma unroll
      for (int d = 0; d < D; ++d) c0[d] = cnt0 > 0.0f ? t[d] / den0 : c0[d];
#pragma unroll
      for (int d = 0; d < D; ++d) t[d] = x[d] * m1;
      seg_sum_rows<D>(t, S);
#pragma unroll
      for (int d = 0; d < D; ++d) c1[d] = cnt1 > 0.0f ? t[d] / den1 : c1[d];
    }
    const float proj = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c0[i] - c1[i]; });
    // stable ascending rank of the projection inside the group (read from LDS four at a time), then the
    // member moves to that rank
    s_pr[lane] = proj;
    wave_sync();
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < S; j += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(s_pr + gb + j);
      const float pj[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) rank += (pj[e] < proj || (pj[e] == proj && j + e < li)) ? 1 : 0;
    }
    const int slot = gb + rank;
#pragma unroll
    for (int d = 0; d < D; ++d) s_x[slot * DP + d] = x[d];
    s_p[slot] = p;
    wave_sync();
#pragma unroll
    for (int d = 0; d < D; ++d) x[d] = s_x[lane * DP + d];
    p = s_p[lane];
    wave_sync();
  }
  if (live) perm[(int64_t)bh * nb * Bk + (int64_t)blk * Bk + lane] = p;

  // node sums by adjacent pairs: level depth holds pairs of ranks, level 0 the whole block
  auto pyramid = [&](float (&y)[D], float* const* out) {
    for (int l = depth; l >= 0; --l) {
      const int sz = Bk >> l;   // keys per node at level l
      switch (sz >> 1) {   // adjacent pairs of the level below: partner at distance sz / 2
        case 1: seg_sum_rows_step<1>(y); break;
        case 2: seg_sum_rows_step<2>(y); break;
        case 4: seg_sum_rows_step<4>(y); break;
        case 8: seg_sum_rows_step<8>(y); break;
        case 16: seg_sum_rows_step<16>(y); break;
        default: seg_sum_rows_step<32>(y); break;
      }
      if (live && (lane & (sz - 1)) == 0) {
        float* row = out[l] + b * lv.sb[l] + h * lv.sh[l] + ((int64_t)blk * (Bk / sz) + lane / sz) * D;
#pragma unroll
        for (int d = 0; d < D; ++d) row[d] = y[d];
      }
    }
  };
  float y[D];
#pragma unroll
  for (int d = 0; d < D; ++d) y[d] = x[d];
  pyramid(y, lv.sums);
  if (gate) {
#pragma unroll
    for (int d = 0; d < D; ++d) y[d] = forest_log(x[d]);
    pyramid(y, lv.lg);
  }
}

// The same build with a workgroup of Q = D / 16 wavefronts per block, key i held 16 dimensions per lane by lanes
// [Q i, Q i + Q): the build for head sizes 32, 64 and 128 (forest_build_kernel, one wavefront per block with a
// whole key per lane, would hold five D-vectors per lane at 128, and at 64 and 32 its 64 or 32 sequential
// per-dimension sums per group are a longer chain than Q lanes' 16: 0.161 -> 0.111 ms for bench_speed's layer).  The member sums
// are the same halving trees (member i + member i + S/2 first, ...) and the node sums the same adjacent pairs:
// a step whose partner lies in another wavefront goes through LDS, the others are xor exchanges; dot products
// are canon_dot's value finished across the Q lanes of a key.  The results equal the one-wavefront kernel's
// arithmetic, so the canonical oracle's, bit for bit.
template <int Q>
__device__ __forceinline__ void fw_step(float (&v)[16], int lh, float* xb, int tid) {
  if (lh >= kWave) {   // the partner in another wavefront: every lane's 16 values through LDS
    __syncthreads();
#pragma unroll
    for (int d = 0; d < 16; d += 4)
      *reinterpret_cast<float4*>(xb + tid * 16 + d) = make_float4(v[d], v[d + 1], v[d + 2], v[d + 3]);
    __syncthreads();
    const float* o = xb + (tid ^ lh) * 16;
#pragma unroll
    for (int d = 0; d < 16; d += 4) {
      const float4 u = *reinterpret_cast<const float4*>(o + d);
      v[d] = v[d] + u.x;
      v[d + 1] = v[d + 1] + u.y;
      v[d + 2] = v[d + 2] + u.z;
      v[d + 3] = v[d + 3] + u.w;
    }
    return;
  }
  switch (lh) {
    case 32: seg_sum_rows_step<32>(v); break;
    case 16: seg_sum_rows_step<16>(v); break;
    case 8: seg_sum_rows_step<8>(v); break;
    case 4: seg_sum_rows_step<4>(v); break;
    case 2: seg_sum_rows_step<2>(v); break;
    default: seg_sum_rows_step<1>(v); break;
  }
}
// A scalar of every member summed over the group by the same halving tree (the counts: integers, any order).
template <int Q>
__device__ __forceinline__ float fw_sum(float v, int S, float* xs, int tid) {
  for (int h = S / 2; h >= 1; h >>= 1) {
    const int lh = h * Q;
    if (lh >= kWave) {
      __syncthreads();
      xs[tid] = v;
      __syncthreads();
      v = v + xs[tid ^ lh];
    } else {
      v = v + __shfl_xor(v, lh, kWave);
    }
  }
  return v;
}
// The first member (smallest index) of the group whose value is the group's largest.
template <int Q>
__device__ __forceinline__ int fw_argmax_first(float v, int m, int S, float* xs, int* xi, int tid) {
  int i = m;
  for (int h = S / 2; h >= 1; h >>= 1) {
    const int lh = h * Q;
    float ov;
    int oi;
    if (lh >= kWave) {
      __syncthreads();
      xs[tid] = v;
      xi[tid] = i;
      __syncthreads();
      ov = xs[tid ^ lh];
      oi = xi[tid ^ lh];
    } else {
      ov = __shfl_xor(v, lh, kWave);
      oi = __shfl_xor(i, lh, kWave);
    }
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  return i;
}
// canon_dot's value for two D-vectors held 16 dimensions per lane by the Q lanes of a key (lane q: dimensions
// [16 q, 16 q + 16)): each lane reduces its 16 / Q whole groups of D / 16, then the halving tree over the 16
// groups crosses lanes where a step pairs groups held by different lanes.
template <int D, int Q, typename FA, typename FB>
__device__ __forceinline__ float fw_dot(FA fa, FB fb) {
  constexpr int R = D / 16, GQ = 16 / Q;
  float g[GQ];
#pragma unroll
  for (int j = 0; j < GQ; ++j) {
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
  for (int n = 8; n >= 1; n /= 2) {
    if (n >= GQ) {
#pragma unroll
      for (int i = 0; i < GQ; ++i) g[i] = g[i] + __shfl_xor(g[i], n / GQ, kWave);
    } else {
#pragma unroll
      for (int i = 0; i < n; ++i) g[i] = g[i] + g[i + n];
    }
  }
  return g[0];
}

template <typename T, int D>
__global__ __launch_bounds__(kWave * (D / 16)) void forest_build_wide_kernel(const T* __restrict__ k, int64_t ksb,
                                                                            int64_t ksh, int64_t kst, int H, int nb,
                                                                            int Bk, int depth, int iters, int gate,
                                                                            int32_t* __restrict__ perm,
                                                                            ForestLevels lv) {
  constexpr int Q = D / 16, DQ = 16, NT = kWave * Q, RS = D + 4;
  __shared__ __align__(16) float s_x[kWave * RS];   // the members' rows (the reorder buffer too)
  __shared__ __align__(16) float s_xb[NT * DQ];     // cross-wavefront exchange of 16 values per lane
  __shared__ float s_xs[NT];
  __shared__ int s_xi[NT];
  __shared__ int s_p[kWave];
  __shared__ __align__(16) float s_pr[kWave];       // the level's projections
  const int tid = threadIdx.x, m = tid / Q, q = tid % Q, d0 = q * DQ;
  const int pb = blockIdx.x, blk = pb % nb, bh = pb / nb, b = bh / H, h = bh % H;
  const bool live = m < Bk;
  const int64_t pos = (int64_t)blk * Bk + (live ? m : 0);
  float x[DQ];
  load_row_g<T, DQ>(k + b * ksb + h * ksh + pos * kst + d0, x);
#pragma unroll
  for (int d = 0; d < DQ; ++d) x[d] = live ? (pos == 0 ? x[d] * 0.0f : x[d]) : 0.0f;   // the sink: k * 0
  int p = m;
  float c0[DQ], c1[DQ], t[DQ];
  auto bfly = [&](float (&v)[DQ], int S) {
    for (int hh = S / 2; hh >= 1; hh >>= 1) fw_step<Q>(v, hh * Q, s_xb, tid);
  };
  for (int lvl = 0; lvl < depth; ++lvl) {
    const int S = Bk >> lvl, gb = m & ~(S - 1), li = m - gb;
    // the members' rows in LDS, for the two farthest members' rows
#pragma unroll
    for (int d = 0; d < DQ; d += 4)
      *reinterpret_cast<float4*>(s_x + m * RS + d0 + d) = make_float4(x[d], x[d + 1], x[d + 2], x[d + 3]);
    // the group mean, then the member farthest from it (a) and the member farthest from a (b)
#pragma unroll
    for (int d = 0; d < DQ; ++d) c0[d] = x[d];
    bfly(c0, S);
#pragma unroll
    for (int d = 0; d < DQ; ++d) c0[d] = c0[d] / (float)S;
    const float d2 = fw_dot<D, Q>([&](int i) { return x[i] - c0[i]; }, [&](int i) { return x[i] - c0[i]; });
    const int la = fw_argmax_first<Q>(d2, m, S, s_xs, s_xi, tid);
    __syncthreads();   // the rows in s_x
#pragma unroll
    for (int d = 0; d < DQ; ++d) c0[d] = s_x[la * RS + d0 + d];
    const float d2b = fw_dot<D, Q>([&](int i) { return x[i] - c0[i]; }, [&](int i) { return x[i] - c0[i]; });
    const int lb = fw_argmax_first<Q>(d2b, m, S, s_xs, s_xi, tid);
#pragma unroll
    for (int d = 0; d < DQ; ++d) c1[d] = s_x[lb * RS + d0 + d];
    const float xx = fw_dot<D, Q>([&](int i) { return x[i]; }, [&](int i) { return x[i]; });
    for (int it = 0; it < iters; ++it) {
      const float cc0 = fw_dot<D, Q>([&](int i) { return c0[i]; }, [&](int i) { return c0[i]; });
      const float cc1 = fw_dot<D, Q>([&](int i) { return c1[i]; }, [&](int i) { return c1[i]; });
      const float xc0 = fw_dot<D, Q>([&](int i) { return x[i]; }, [&](int i) { return c0[i]; });
      const float xc1 = fw_dot<D, Q>([&](int i) { return x[i]; }, [&](int i) { return c1[i]; });
      const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
      const bool lab1 = dist1 < dist0;   // argmin over the two centroids, the first on ties
      const float m0 = lab1 ? 0.0f : 1.0f, m1 = lab1 ? 1.0f : 0.0f;
      const float cnt0 = fw_sum<Q>(m0, S, s_xs, tid), cnt1 = fw_sum<Q>(m1, S, s_xs, tid);
      const float den0 = fmaxf(cnt0, 1.0f), den1 = fmaxf(cnt1, 1.0f);
#pragma unroll
      for (int d = 0; d < DQ; ++d) t[d] = x[d] * m0;
      bfly(t, S);
#pragma unroll
      for (int d = 0; d < DQ; ++d) c0[d] = cnt0 > 0.0f ? t[d] / den0 : c0[d];
#pragma unroll
      for (int d = 0; d < DQ; ++d) t[d] = x[d] * m1;
      bfly(t, S);
#pragma unroll
      for (int d = 0; d < DQ; ++d) c1[d] = cnt1 > 0.0f ? t[d] / den1 : c1[d];
    }
    const float proj = fw_dot<D, Q>([&](int i) { return x[i]; }, [&](int i) { return c0[i] - c1[i]; });
    // stable ascending rank of the projection inside the group, then the member moves to that rank
    __syncthreads();   // every read of s_x above is done
    if (q == 0) s_pr[m] = proj;
    __syncthreads();
    int rank = 0;
    for (int j = 0; j < S; ++j) {
      const float pj = s_pr[gb + j];
      rank += (pj < proj || (pj == proj && j < li)) ? 1 : 0;
    }
    const int slot = gb + rank;
#pragma unroll
    for (int d = 0; d < DQ; d += 4)
      *reinterpret_cast<float4*>(s_x + slot * RS + d0 + d) = make_float4(x[d], x[d + 1], x[d + 2], x[d + 3]);
    if (q == 0) s_p[slot] = p;
    __syncthreads();
#pragma unroll
    for (int d = 0; d < DQ; ++d) x[d] = s_x[m * RS + d0 + d];
    p = s_p[m];
    __syncthreads();
  }
  if (live && q == 0) perm[(int64_t)bh * nb * Bk + (int64_t)blk * Bk + m] = p;

  // node sums by adjacent pairs: level depth holds pairs of ranks, level 0 the whole block
  auto pyramid = [&](float (&y)[DQ], float* const* out) {
    for (int l = depth; l >= 0; --l) {
      const int sz = Bk >> l;   // keys per node at level l
      fw_step<Q>(y, (sz >> 1) * Q, s_xb, tid);
      if (live && (m & (sz - 1)) == 0) {
        float* row = out[l] + b * lv.sb[l] + h * lv.sh[l] + ((int64_t)blk * (Bk / sz) + m / sz) * D + d0;
#pragma unroll
        for (int d = 0; d < DQ; d += 4) *reinterpret_cast<float4*>(row + d) = make_float4(y[d], y[d + 1], y[d + 2], y[d + 3]);
      }
    }
  };
  float y[DQ];
#pragma unroll
  for (int d = 0; d < DQ; ++d) y[d] = x[d];
  pyramid(y, lv.sums);
  if (gate) {
#pragma unroll
    for (int d = 0; d < DQ; ++d) y[d] = forest_log(x[d]);
    pyramid(y, lv.lg);
  }
}

// The soft gate of every node (forest.py:36-44), one wavefront per node, lane = dimension: mean log-magnitude
// ml = lg / keys, thr = the gate_q quantile of ml over the dimensions, g = logistic((ml - thr) / temp), the node
// sum becomes (sum * g) * (D / max(sum of g, 1)).  In place.
template <int D>
__global__ __launch_bounds__(256) void forest_gate_kernel(ForestLevels lv, int H, int nb, int Bk, int depth, int lo,
                                                          float w, float temp) {
  const int lane = lane_id();
  const int64_t idx = (int64_t)blockIdx.x * 4 + wave_id();   // node index over all levels of one (b, h)
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  // level l holds nb << l nodes; they follow each other in level order
  int l = 0;
  int64_t n = idx, cnt = nb;
  while (l <= depth && n >= cnt) {
    n -= cnt;
    cnt <<= 1;
    ++l;
  }
  if (l > depth) return;
  const bool in = lane < D;
  float* row = lv.sums[l] + b * lv.sb[l] + h * lv.sh[l] + n * D;
  const float* lrow = lv.lg[l] + b * lv.sb[l] + h * lv.sh[l] + n * D;
  const float raw = in ? row[lane] : 0.0f;
  const float ml = (in ? lrow[lane] : 0.0f) / (float)(Bk >> l);
  int rank = 0;
  for (int e = 0; e < D; ++e) {
    const float o = __shfl(ml, e, kWave);
    rank += (o < ml || (o == ml && e < lane)) ? 1 : 0;
  }
  const int hi = w > 0.0f ? lo + 1 : lo;
  const uint64_t blo = __ballot(in && rank == lo), bhi = __ballot(in && rank == hi);
  const float vlo = __shfl(ml, __ffsll((unsigned long long)blo) - 1, kWave);
  const float vhi = __shfl(ml, __ffsll((unsigned long long)bhi) - 1, kWave);
  const float dd = vhi - vlo;
  const float thr = w < 0.5f ? vlo + w * dd : vhi - dd * (1.0f - w);
  const float z = (ml - thr) / temp;
  const float g = in ? (float)(1.0 / (1.0 + exp(-(double)z))) : 0.0f;
  const float kept = fmaxf(seg_sum(g, D), 1.0f);
  const float scale = (float)D / kept;
  if (in) row[lane] = (raw * g) * scale;
}

// forest_gate_kernel for a head size above 64: lane i holds dimensions i + 64 e (e < D / 64).  The rank of a
// mean log-magnitude among the D is the same stable count, the quantile the same interpolation, and the kept mass
// the same halving tree over dimensions (dimension d + dimension d + D/2 first: the lane's own values when
// D = 128, then the butterfly over the 64 lanes).
template <int D>
__global__ __launch_bounds__(256) void forest_gate_wide_kernel(ForestLevels lv, int H, int nb, int Bk, int depth,
                                                               int lo, float w, float temp) {
  static_assert(D == 128, "two dimensions per lane");
  constexpr int DL = D / kWave;
  const int lane = lane_id();
  const int64_t idx = (int64_t)blockIdx.x * 4 + wave_id();
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  int l = 0;
  int64_t n = idx, cnt = nb;
  while (l <= depth && n >= cnt) {
    n -= cnt;
    cnt <<= 1;
    ++l;
  }
  if (l > depth) return;
  float* row = lv.sums[l] + b * lv.sb[l] + h * lv.sh[l] + n * D;
  const float* lrow = lv.lg[l] + b * lv.sb[l] + h * lv.sh[l] + n * D;
  float raw[DL], ml[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) {
    raw[e] = row[lane + kWave * e];
    ml[e] = lrow[lane + kWave * e] / (float)(Bk >> l);
  }
  int rank[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) rank[e] = 0;
#pragma unroll
  for (int e2 = 0; e2 < DL; ++e2) {
    for (int src = 0; src < kWave; ++src) {
      const float o = __shfl(ml[e2], src, kWave);
      const int d2 = src + kWave * e2;
#pragma unroll
      for (int e = 0; e < DL; ++e) {
        const int d = lane + kWave * e;
        rank[e] += (o < ml[e] || (o == ml[e] && d2 < d)) ? 1 : 0;
      }
    }
  }
  const int hi = w > 0.0f ? lo + 1 : lo;
  // the values at ranks lo and hi (each rank held by exactly one dimension)
  float vlo = 0.0f, vhi = 0.0f;
#pragma unroll
  for (int e = 0; e < DL; ++e) {
    const uint64_t blo = __ballot(rank[e] == lo), bhi = __ballot(rank[e] == hi);
    if (blo) vlo = __shfl(ml[e], __ffsll((unsigned long long)blo) - 1, kWave);
    if (bhi) vhi = __shfl(ml[e], __ffsll((unsigned long long)bhi) - 1, kWave);
  }
  const float dd = vhi - vlo;
  const float thr = w < 0.5f ? vlo + w * dd : vhi - dd * (1.0f - w);
  float g[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) {
    const float z = (ml[e] - thr) / temp;
    g[e] = (float)(1.0 / (1.0 + exp(-(double)z)));
  }
  const float kept = fmaxf(seg_sum(g[0] + g[1], kWave), 1.0f);
  const float scale = (float)D / kept;
#pragma unroll
  for (int e = 0; e < DL; ++e) row[lane + kWave * e] = (raw[e] * g[e]) * scale;
}

struct ForestDesc {
  const void* q;
  int64_t qsb, qsh, qst;
  int H, T, nb, Bk, depth, wmax, bq_desc, wl, Kc;
  const float* sums[kMaxLevels];
  int64_t sb[kMaxLevels], sh[kMaxLevels];
  const int32_t* perm;      // (B, H, nb * Bk)
  const int32_t* bq_use;    // (B, H, T) leaves the attention uses, or null (all the valid ones)
  int32_t* leaf;            // (B, H, T, wl)
  uint8_t* leafv;
  int32_t* cand;            // (B, H, T, Kc): own block, static keys, tree keys; -1 where unused
  int32_t* lv_cur;          // (depth + 1, B, H, T, lv_stride) candidates of every level, or null
  uint8_t* lv_cv;
  int lv_stride;
  int32_t* counts;          // (B, H, T, 2): the row's valid static keys and tree keys, or null
};

// One wavefront per query (attention.py:93-148): score the roots of all blocks (valid: the blocks before the
// query's own), keep the best min(wmax, C) (valid while their rank is below bq_desc), expand every kept node to
// its two children (all left children, then all right ones), ... down to the pairs; then the candidate list.
template <typename T, int D>
__global__ __launch_bounds__(256) void forest_descend_kernel(ForestDesc p) {
  constexpr int R = D / 16;
  __shared__ __align__(16) float s_sc[4][kForestMaxRoots];
  __shared__ __align__(16) int32_t s_id[4][kForestMaxRoots];
  __shared__ __align__(16) uint8_t s_v[4][kForestMaxRoots];
  __shared__ int32_t s_kid[4][kForestMaxW];
  __shared__ uint8_t s_kv[4][kForestMaxW];
  const int wv = wave_id(), lane = lane_id();
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;   // grid: (positions / 4, B * H)
  const int t = blockIdx.x * 4 + wv;
  if (t >= p.T) return;
  const int blk = t / p.Bk;
  float* sc = s_sc[wv];
  int32_t* id = s_id[wv];
  uint8_t* vv = s_v[wv];
  const int g = lane >> 4, j16 = lane & 15;
  float qr[R];
  load_row<T, R>(reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)t * p.qst + R * j16, qr);
  const int64_t qflat = (int64_t)bh * p.T + t;

  int C = p.nb;
  for (int c = lane; c < C; c += kWave) {
    id[c] = c;
    vv[c] = c < blk ? 1 : 0;
  }
  wave_sync();
  int w = 0;
  for (int l = 0; l <= p.depth; ++l) {
    const float* base = p.sums[l] + b * p.sb[l] + h * p.sh[l] + R * j16;
    // four candidates at a time (a 16-lane group each), the rows of eight such steps requested before the
    // first is scored
    constexpr int U = 8;
    for (int c0 = 0; c0 < C; c0 += 4 * U) {
      float rows[U][R];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + 4 * u + g;
        load_row_g<float, R>(base + (int64_t)id[c < C ? c : 0] * D, rows[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + 4 * u + g;
        const float s = canon_dot<R>(qr, rows[u]);
        if (c < C && j16 == 0) sc[c] = vv[c] ? s : -INFINITY;
      }
    }
    if (p.lv_cur != nullptr) {
      const int64_t o = ((int64_t)l * gridDim.y * p.T + qflat) * p.lv_stride;
      for (int c = lane; c < p.lv_stride; c += kWave) {
        p.lv_cur[o + c] = c < C ? id[c] : -1;
        p.lv_cv[o + c] = c < C ? vv[c] : 0;
      }
    }
    wave_sync();
    w = C < p.wmax ? C : p.wmax;
    for (int c = lane; c < C; c += kWave) {
      const float si = sc[c];
      const int ii = id[c];
      const bool vi = vv[c] != 0;
      int rank = 0;
      for (int e0 = 0; e0 < C; e0 += 4) {   // four entries per LDS read (the arrays hold kForestMaxRoots)
        const float4 s4 = *reinterpret_cast<const float4*>(sc + e0);
        const int4 i4 = *reinterpret_cast<const int4*>(id + e0);
        const uint32_t v4 = *reinterpret_cast<const uint32_t*>(vv + e0);
        const float se[4] = {s4.x, s4.y, s4.z, s4.w};
        const int ie[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int e = e0 + k;
          const bool ve = ((v4 >> (8 * k)) & 0xffu) != 0;
          bool better;
          if (ve != vi) better = ve;
          else if (vi) better = se[k] > si || (se[k] == si && ie[k] < ii);
          else better = e < c;
          rank += (better && e < C) ? 1 : 0;
        }
      }
      if (rank < w) {
        s_kid[wv][rank] = ii;
        s_kv[wv][rank] = (vi && rank < p.bq_desc) ? 1 : 0;
      }
    }
    wave_sync();
    if (l == p.depth) break;
    C = 2 * w;
    for (int c = lane; c < C; c += kWave) {
      const int k0 = c < w ? c : c - w;
      id[c] = 2 * s_kid[wv][k0] + (c < w ? 0 : 1);
      vv[c] = s_kv[wv][k0];
    }
    wave_sync();
  }

  // outputs: the leaves, and the candidate list [own block | 0, t-1, t-2 | left keys | right keys]
  const int wl = p.wl;
  for (int i = lane; i < wl; i += kWave) {
    p.leaf[qflat * wl + i] = i < w ? s_kid[wv][i] : -1;
    p.leafv[qflat * wl + i] = i < w ? s_kv[wv][i] : 0;
  }
  int32_t* cr = p.cand + qflat * p.Kc;
  const int own0 = blk * p.Bk;
  for (int j = lane; j < p.Bk; j += kWave) cr[j] = own0 + j <= t ? own0 + j : -1;
  const int s0 = 0, s1 = t - 1, s2 = t - 2;
  const bool v0 = s0 < own0, v1 = s1 >= 0 && s1 < own0, v2 = s2 >= 0 && s2 < own0;
  if (lane == 0) {
    cr[p.Bk] = v0 ? s0 : -1;
    cr[p.Bk + 1] = v1 ? s1 : -1;
    cr[p.Bk + 2] = v2 ? s2 : -1;
  }
  const int use = p.bq_use != nullptr ? p.bq_use[qflat] : wl;
  const int32_t* pr = p.perm + (int64_t)bh * p.nb * p.Bk;
  int ntree = 0;
  for (int c = lane; c < 2 * wl; c += kWave) {
    const int i = c < wl ? c : c - wl;
    int key = -1;
    if (i < w && s_kv[wv][i] && i < use) {
      const int pf = 2 * s_kid[wv][i] + (c < wl ? 0 : 1);
      const int kk = (pf / p.Bk) * p.Bk + pr[pf];
      const bool dup = (v0 && kk == s0) || (v1 && kk == s1) || (v2 && kk == s2);
      key = dup ? -1 : kk;
    }
    cr[p.Bk + 3 + c] = key;
    ntree += key >= 0 ? 1 : 0;
  }
  if (p.counts != nullptr) {
    for (int o = 32; o >= 1; o >>= 1) ntree += __shfl_xor(ntree, o, kWave);
    if (lane == 0) {
      p.counts[qflat * 2] = (int)v0 + (int)v1 + (int)v2;
      p.counts[qflat * 2 + 1] = ntree;
    }
  }
}

}  // namespace ta

using namespace ta;

namespace {
bool forest_dim_ok(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }
}  // namespace

extern "C" int ta_forest_build(const void* k, int dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int T,
                               int D, int block, int kmeans_iters, int gate, float gate_q, float gate_temp,
                               int32_t* perm, float* const* sums, float* const* lg, const int64_t* sb,
                               const int64_t* sh, void* stream) {
  if (B <= 0 || H <= 0 || T <= 0 || block < 4 || block > kWave || (block & (block - 1)) || T % block ||
      !forest_dim_ok(D) || kmeans_iters < 0 || perm == nullptr || sums == nullptr || sb == nullptr ||
      sh == nullptr || (gate && (lg == nullptr || !(gate_q >= 0.0f && gate_q <= 1.0f) || !(gate_temp > 0.0f)))) {
    set_error("ta_forest_build: bad arguments (block a power of two in [4, 64] dividing T; D 16, 32, 64 or 128)");
    return TA_ERR_ARG;
  }
  const int es = dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)k % 16) || (ksb * es) % 16 || (ksh * es) % 16 || (kst * es) % 16) {
    set_error("ta_forest_build: key rows 16-byte aligned");
    return TA_ERR_ARG;
  }
  const int nb = T / block;
  int depth = 0;
  while ((2 << depth) < block) ++depth;   // block / 2 = 2^depth
  ForestLevels lv{};
  for (int l = 0; l <= depth; ++l) {
    if (sums[l] == nullptr || (gate && lg[l] == nullptr)) {
      set_error("ta_forest_build: a level pointer is null");
      return TA_ERR_ARG;
    }
    lv.sums[l] = sums[l];
    lv.lg[l] = gate ? lg[l] : nullptr;
    lv.sb[l] = sb[l];
    lv.sh[l] = sh[l];
  }
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((int64_t)B * H * nb));
#define TA_FB(TT, DD)                                                                                           \
  hipLaunchKernelGGL((forest_build_kernel<TT, DD>), grid, dim3(kWave), 0, st, (const TT*)k, ksb, ksh, kst, H, \
                     nb, block, depth, kmeans_iters, gate, perm, lv)
#define TA_FB_D(TT)                                                                                          \
  switch (D) {                                                                                               \
    case 16: TA_FB(TT, 16); break;                                                                           \
    case 32:                                                                                                 \
      hipLaunchKernelGGL((forest_build_wide_kernel<TT, 32>), grid, dim3(2 * kWave), 0, st, (const TT*)k, ksb,  \
                         ksh, kst, H, nb, block, depth, kmeans_iters, gate, perm, lv);                       \
      break;                                                                                                 \
    case 64:                                                                                                 \
      hipLaunchKernelGGL((forest_build_wide_kernel<TT, 64>), grid, dim3(4 * kWave), 0, st, (const TT*)k, ksb,  \
                         ksh, kst, H, nb, block, depth, kmeans_iters, gate, perm, lv);                       \
      break;                                                                                                 \
    default:                                                                                                 \
      hipLaunchKernelGGL((forest_build_wide_kernel<TT, 128>), grid, dim3(8 * kWave), 0, st, (const TT*)k, ksb, \
                         ksh, kst, H, nb, block, depth, kmeans_iters, gate, perm, lv);                       \
      break;                                                                                                 \
  }
  switch (dtype) {
    case TA_F32: TA_FB_D(float); break;
    case TA_F16: TA_FB_D(f16_t); break;
    case TA_BF16: TA_FB_D(bf16_t); break;
    default: set_error("ta_forest_build: unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_FB_D
#undef TA_FB
  int rc = check_launch("forest_build_kernel");
  if (rc != TA_OK || !gate) return rc;
  const float r = gate_q * (float)(D - 1);
  const int lo = (int)floorf(r);
  const float w = r - (float)lo;
  // nodes per (b, h): nb * (1 + 2 + ... + 2^depth) = nb * (block - 1), four per workgroup
  const dim3 ggrid((unsigned)((nb * (int64_t)(block - 1) + 3) / 4), B * H);
  switch (D) {
    case 16: hipLaunchKernelGGL((forest_gate_kernel<16>), ggrid, dim3(256), 0, st, lv, H, nb, block, depth, lo, w, gate_temp); break;
    case 32: hipLaunchKernelGGL((forest_gate_kernel<32>), ggrid, dim3(256), 0, st, lv, H, nb, block, depth, lo, w, gate_temp); break;
    case 64: hipLaunchKernelGGL((forest_gate_kernel<64>), ggrid, dim3(256), 0, st, lv, H, nb, block, depth, lo, w, gate_temp); break;
    default: hipLaunchKernelGGL((forest_gate_wide_kernel<128>), ggrid, dim3(256), 0, st, lv, H, nb, block, depth, lo, w, gate_temp); break;
  }
  return check_launch("forest_gate_kernel");
}

extern "C" int ta_forest_descend(const void* q, int dtype, int64_t qsb, int64_t qsh, int64_t qst, int B, int H, int T,
                                 int D, int block, const float* const* sums, const int64_t* sb, const int64_t* sh,
                                 const int32_t* perm, int wmax, int bq_desc, const int32_t* bq_use, int32_t* leaf,
                                 uint8_t* leafv, int32_t* cand, int32_t* lv_cur, uint8_t* lv_cv, int lv_stride,
                                 int32_t* counts, void* stream) {
  if (B <= 0 || H <= 0 || T <= 0 || block < 4 || block > kWave || (block & (block - 1)) || T % block ||
      !forest_dim_ok(D) || wmax < 1 || wmax > kForestMaxW || T / block > kForestMaxRoots || q == nullptr ||
      sums == nullptr || perm == nullptr || leaf == nullptr || leafv == nullptr || cand == nullptr ||
      (lv_cur != nullptr && lv_cv == nullptr)) {
    set_error("ta_forest_descend: bad arguments (block a power of two in [4, 64] dividing T, at most 1024 blocks; "
              "D 16, 32, 64 or 128; 1 <= wmax <= 64)");
    return TA_ERR_ARG;
  }
  const int R = D / 16, es = dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)q % (R * es)) || (qsb % R) || (qsh % R) || (qst % R)) {
    set_error("ta_forest_descend: query rows aligned to D / 16 elements");
    return TA_ERR_ARG;
  }
  ForestDesc p{};
  p.q = q; p.qsb = qsb; p.qsh = qsh; p.qst = qst;
  p.H = H; p.T = T; p.nb = T / block; p.Bk = block;
  int depth = 0;
  while ((2 << depth) < block) ++depth;
  p.depth = depth;
  p.wmax = wmax;
  p.bq_desc = bq_desc;
  int w = p.nb < wmax ? p.nb : wmax, wide = p.nb;
  for (int l = 1; l <= depth; ++l) {
    wide = wide > 2 * w ? wide : 2 * w;
    w = 2 * w < wmax ? 2 * w : wmax;
  }
  p.wl = w;
  p.Kc = block + 3 + 2 * w;
  if (lv_cur != nullptr && lv_stride < wide) {
    set_error("ta_forest_descend: lv_stride below the widest level");
    return TA_ERR_ARG;
  }
  for (int l = 0; l <= depth; ++l) {
    if (sums[l] == nullptr) {
      set_error("ta_forest_descend: a level pointer is null");
      return TA_ERR_ARG;
    }
    p.sums[l] = sums[l];
    p.sb[l] = sb[l];
    p.sh[l] = sh[l];
  }
  p.perm = perm; p.bq_use = bq_use; p.leaf = leaf; p.leafv = leafv; p.cand = cand;
  p.lv_cur = lv_cur; p.lv_cv = lv_cv; p.lv_stride = lv_stride; p.counts = counts;
  const dim3 grid((unsigned)((T + 3) / 4), B * H);
  hipStream_t st = (hipStream_t)stream;
#define TA_FD(TT, DD) hipLaunchKernelGGL((forest_descend_kernel<TT, DD>), grid, dim3(256), 0, st, p)
#define TA_FD_D(TT)                  \
  switch (D) {                       \
    case 16: TA_FD(TT, 16); break;   \
    case 32: TA_FD(TT, 32); break;   \
    case 64: TA_FD(TT, 64); break;   \
    default: TA_FD(TT, 128); break;  \
  }
  switch (dtype) {
    case TA_F32: TA_FD_D(float); break;
    case TA_F16: TA_FD_D(f16_t); break;
    case TA_BF16: TA_FD_D(bf16_t); break;
    default: set_error("ta_forest_descend: unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_FD_D
#undef TA_FD
  return check_launch("forest_descend_kernel");
}

// Candidate-list width and leaf count of ta_forest_descend for T positions (for the caller's allocations).
extern "C" int ta_forest_shape(int T, int block, int wmax, int* wl, int* kc, int* widest) {
  if (T <= 0 || block < 4 || (block & (block - 1)) || T % block || wmax < 1) {
    set_error("ta_forest_shape: bad arguments");
    return TA_ERR_ARG;
  }
  const int nb = T / block;
  int depth = 0;
  while ((2 << depth) < block) ++depth;
  int w = nb < wmax ? nb : wmax, wide = nb;
  for (int l = 1; l <= depth; ++l) {
    wide = wide > 2 * w ? wide : 2 * w;
    w = 2 * w < wmax ? 2 * w : wmax;
  }
  *wl = w;
  *kc = block + 3 + 2 * w;
  *widest = wide;
  return TA_OK;
}
