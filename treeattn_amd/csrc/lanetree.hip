// LaneTree: the key selection of the reference's 'dyn' attention.  The sequence is cut into lanes of `chunk`
// positions; lane l owns one balanced binary tree of capacity T over the keys [1, l * chunk) (the tree a
// sequential decoder would hold when it reaches the lane), then walks through the lane's positions one at a time:
// neighbour search over the leaves the lane's previous positions stored, beam search over the tree, store,
// insertion of the position's key.  One wavefront per lane tree; the lane trees run in parallel.
//
// Reference functions replaced: dyntree.py:6-31 masked_two_means_order, dyntree.py:34-82 LaneTree.__init__,
// dyntree.py:84-106 insert, dyntree.py:108-127 search, dyntree.py:129-131 leaf_keys and dyntree.py:148-243
// select_keys.  The candidate list and the attention over it are the segment tree's (selection.assemble,
// ta_sparse_attn_fwd / ta_sparse_attn_bwd), as in attention_dyn.py:74-96.
//
// Arithmetic order (the CPU oracle's canonical mode computes the same, bit for bit):
//  * a mean or centroid over the S members of a group: L = min(S, 64) partial sums, partial j adding members
//    j, j + L, j + 2L, ... in that order, then the halving tree over the L partials (the xor butterfly over L
//    lanes); divided by the member count (at least 1);
//  * dot products: per-dimension float32 products in canon_dot's order; node score = dot / max(count, 1);
//    dist = (|x|^2 - 2 x.c) + |c|^2;
//  * argmax: the first index; member order: stable ascending sort of the projections, empty slots last;
//  * the initial node sums: adjacent pairs over the slots, empty slots contributing key * 0; later insertions
//    add the key in insertion order;
//  * search ranking: valid first, score descending, node id ascending (invalid candidates by slot).
#pragma clang fp contract(off)

#include "canon.hpp"

namespace ta {

constexpr int kLaneMaxT = 4096;    // tree capacity = sequence length
constexpr int kLaneMaxW = 32;      // wmax: the 2 * wmax children of a level are scored one per lane
constexpr int kLaneMaxNb = 64;     // nb_window * nb_store neighbour entries, one per lane

__device__ __forceinline__ int lt_log2(int x) { return 31 - __clz(x); }

// Node (level l, index i) of a lane tree lives at row (1 << l) - 1 + i of its (C, D) float32 sums and (C,)
// int32 counts; leaf i's two key positions at slot[2i], slot[2i + 1] (-1: empty).
struct LaneTree {
  float* sums;
  int32_t* cnt;
  int32_t* slot;
};

__device__ __forceinline__ LaneTree lane_tree(float* ws, int64_t P, int C, int D, int64_t p) {
  LaneTree t;
  t.sums = ws + p * C * D;
  int32_t* ints = reinterpret_cast<int32_t*>(ws + P * C * D);
  t.cnt = ints + p * C;
  t.slot = ints + P * C + p * C;
  return t;
}

// (value, index) argmax over an aligned L-lane segment: the largest value, the smallest index among equals.
template <int H>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  const float ov = xor_lane<H>(v);
  const int oi = xor_lane<H>(i);
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}
__device__ __forceinline__ int seg_argmax_idx(float v, int i, int L) {
  if (L > 32) argmax_step<32>(v, i);
  if (L > 16) argmax_step<16>(v, i);
  if (L > 8) argmax_step<8>(v, i);
  if (L > 4) argmax_step<4>(v, i);
  if (L > 2) argmax_step<2>(v, i);
  if (L > 1) argmax_step<1>(v, i);
  return i;
}

// Integer min / max over an aligned L-lane segment.
template <bool MAX>
__device__ __forceinline__ int seg_iext(int v, int L) {
  auto f = [](int a, int b) { return MAX ? max(a, b) : min(a, b); };
  if (L > 32) v = f(v, xor_lane<32>(v));
  if (L > 16) v = f(v, xor_lane<16>(v));
  if (L > 8) v = f(v, xor_lane<8>(v));
  if (L > 4) v = f(v, xor_lane<4>(v));
  if (L > 2) v = f(v, xor_lane<2>(v));
  if (L > 1) v = f(v, xor_lane<1>(v));
  return v;
}
__device__ __forceinline__ int seg_imax(int v, int L) { return seg_iext<true>(v, L); }
__device__ __forceinline__ int seg_imin(int v, int L) { return seg_iext<false>(v, L); }

// Sort key of a projection: ascending float order (-0 taken as +0, as the comparison does) above the member
// index, so that sorting the 64-bit words is the stable sort of the projections.
__device__ __forceinline__ uint64_t lt_sort_key(float p, int idx) {
  const uint32_t u = __float_as_uint(p + 0.0f);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint32_t)idx;
}

// Ascending bitonic sort of s[0, n2) (n2 a power of two) by one wavefront.
__device__ __forceinline__ void wave_bitonic_sort(uint64_t* s, int n2, int lane) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < (n2 >> 1); i += kWave) {
        const int a = ((i & ~(j - 1)) << 1) | (i & (j - 1)), b = a + j;
        const uint64_t x = s[a], y = s[b];
        if ((x > y) == ((a & k) == 0)) {
          s[a] = y;
          s[b] = x;
        }
      }
      wave_sync();
    }
  }
}

constexpr int kLtGroups = 16;   // groups side by side in a 64-slot window (the smallest group has 4 slots)

// The outputs of lt_group_reduce for groups of L lanes: every (group, dimension) this lane owns (D / L of them,
// at most one when L = 64), the halving tree over the group's L partials (LDS rows of stride D + 4), divided by
// max(count, 1).  All reads are issued before the first store.
template <int D, int L>
__device__ __forceinline__ void lt_group_outputs(const float* red, const float* cnt, bool always, float* dst,
                                                 int lane) {
  constexpr int RS = D + 4, nout = (kWave / L) * D, NU = nout >= kWave ? nout / kWave : 1;
  float p[NU][L], c[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int o = lane + kWave * u, g = o / D, d = o - g * D;
    const bool in = o < nout;
    const float* col = red + g * L * RS + d;
#pragma unroll
    for (int j = 0; j < L; ++j) p[u][j] = in ? col[j * RS] : 0.0f;
    c[u] = in ? cnt[g] : 0.0f;
  }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
#pragma unroll
    for (int n = L / 2; n >= 1; n >>= 1)
#pragma unroll
      for (int i = 0; i < n; ++i) p[u][i] = p[u][i] + p[u][i + n];
    p[u][0] = p[u][0] / fmaxf(c[u], 1.0f);
  }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int o = lane + kWave * u, g = o / D, d = o - g * D;
    if (o < nout && (always || c[u] > 0.0f)) dst[g * RS + d] = p[u][0];
  }
}

// Canonical sums of the groups of L consecutive lanes (64 / L groups, L in {4, ..., 64}), in two steps:
// lt_group_row puts this lane's partial (v, or zero when !take) into its LDS row; lt_group_reduce then reduces
// every (group, dimension) by the halving tree over the group's L partials in one lane, divides by
// max(count, 1) and writes dst (row stride D + 4) when the count is positive or `always`.
template <int D>
__device__ __forceinline__ void lt_group_row(const float (&v)[D], bool take, float* red, int lane) {
  float* row = red + lane * (D + 4);
#pragma unroll
  for (int d = 0; d < D; d += 4)
    *reinterpret_cast<float4*>(row + d) = take ? make_float4(v[d], v[d + 1], v[d + 2], v[d + 3])
                                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}
template <int D>
__device__ __forceinline__ void lt_group_reduce(const float* red, int L, const float* cnt, bool always, float* dst,
                                                int lane) {
  wave_sync();
  switch (L) {
    case 4: lt_group_outputs<D, 4>(red, cnt, always, dst, lane); break;
    case 8: lt_group_outputs<D, 8>(red, cnt, always, dst, lane); break;
    case 16: lt_group_outputs<D, 16>(red, cnt, always, dst, lane); break;
    case 32: lt_group_outputs<D, 32>(red, cnt, always, dst, lane); break;
    default: lt_group_outputs<D, 64>(red, cnt, always, dst, lane); break;
  }
  wave_sync();
}

// ---------------------------------------------------------------------------------------------------- build
// One wavefront per lane tree (dyntree.py:34-82).  Every level splits each group of S = C >> lvl slots by a
// masked 2-means projection; the group's real keys are then laid out half and half (the larger half first),
// empty slots after each half's keys, every empty slot holding the position of the group's last empty slot
// (the one the stable sort ranks last).  Empty slots add key * 0 to the masked sums; they are skipped, which
// changes at most the sign of a zero.  A window of max(S, 64) slots is done at a time: lane j holds member j
// (and j + 64, j + 128, ... when S > 64: partial j of the canonical sums); groups of S < 64 slots sit side by
// side, L = min(S, 64) lanes each.  Means and centroids live in LDS.  The order: for S >= 64 a bitonic sort of
// (projection, index) over the span of the real keys, for smaller groups ranks by counting.
// LDS: permutation (4 C bytes), sort words / projections / reduction rows (max(8 C, 64 (D + 4) 4)),
// centroids (2 x 16 x (D + 4) floats), counts (2 x 16 floats), validity (C).
template <typename T, int D>
__global__ __launch_bounds__(kWave) void lanetree_build_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                                               int64_t kst, int H, int C, int nlane, int chunk,
                                                               int iters, float* __restrict__ ws, int64_t P) {
  constexpr int RS = D + 4;
  extern __shared__ __align__(16) unsigned char s_raw[];
  int32_t* s_perm = reinterpret_cast<int32_t*>(s_raw);
  uint64_t* s_sort = reinterpret_cast<uint64_t*>(s_perm + C);
  float* s_key = reinterpret_cast<float*>(s_sort);
  float* s_red = reinterpret_cast<float*>(s_sort);
  const int scratch = 8 * C > kWave * RS * 4 ? 8 * C : kWave * RS * 4;
  float* s_cen = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(s_sort) + scratch);   // [2][16][RS]
  float* s_cnt = s_cen + 2 * kLtGroups * RS;                                                       // [2][16]
  uint8_t* s_val = reinterpret_cast<uint8_t*>(s_cnt + 2 * kLtGroups);
  const int lane = lane_id();
  const int64_t pt = blockIdx.x;
  const int ln = (int)(pt % nlane);
  const int64_t bh = pt / nlane;
  const T* kb = k + (bh / H) * ksb + (bh % H) * ksh;
  const int n0 = ln * chunk;
  const LaneTree tr = lane_tree(ws, P, C, D, pt);
  const float kInf = __int_as_float(0x7f800000);
  for (int c = lane; c < C; c += kWave) {
    s_perm[c] = c;
    s_val[c] = (c >= 1 && c < n0) ? 1 : 0;
  }
  wave_sync();
  const int nlev = lt_log2(C) - 1;
  float x[D], acc0[D], acc1[D];
  for (int lvl = 0; lvl < nlev; ++lvl) {
    const int S = C >> lvl, half = S >> 1;
    const int L = S < kWave ? S : kWave, M = S < kWave ? 1 : S / kWave, Wz = S < kWave ? kWave : S;
    const int nwin = C > Wz ? C / Wz : 1;
    const int g = lane / L, gl = lane & (L - 1);
    float* c0 = s_cen + g * RS;
    float* c1 = s_cen + (kLtGroups + g) * RS;
    for (int win = 0; win < nwin; ++win) {
      const int gb = win * Wz + g * S;
      const bool live = win * Wz + lane < C;   // C < 64: lanes past the tree sit out
      // (1) counts and the masked mean
#pragma unroll
      for (int d = 0; d < D; ++d) acc0[d] = 0.0f;
      float cntp = 0.0f;
      int vlo = S, vhi = -1, lastinv = -1;
      const bool resident = M == 1;   // one member per lane: its row stays in x for every pass of the window
      for (int t = 0; t < M; ++t) {
        const int i = gl + L * t, s = gb + i;
        if (!live) continue;
        if (s_val[s]) {
          load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
          if (!resident) {
#pragma unroll
            for (int d = 0; d < D; ++d) acc0[d] = acc0[d] + x[d];
          }
          cntp = cntp + 1.0f;
          vlo = min(vlo, i);
          vhi = max(vhi, i);
        } else {
          lastinv = i;
        }
      }
      const float cnt = seg_sum(cntp, L);
      const int ng = (int)cnt;
      vlo = seg_imin(vlo, L);
      vhi = seg_imax(vhi, L);
      lastinv = seg_imax(lastinv, L);
      const bool work = __ballot(cntp > 0.0f) != 0;
      if (work) {
        if (gl == 0) s_cnt[g] = cnt;
        if (resident) lt_group_row<D>(x, cntp > 0.0f, s_red, lane);
        else lt_group_row<D>(acc0, true, s_red, lane);
        lt_group_reduce<D>(s_red, L, s_cnt, true, c0 - g * RS, lane);   // the means, into c0
        // a = the real key farthest from the mean, then b = the real key farthest from a
        for (int pass = 0; pass < 2; ++pass) {
          float bv = -1.0f;
          int bi = 0;
          for (int t = 0; t < M; ++t) {
            const int i = gl + L * t, s = gb + i;
            if (!live || !s_val[s]) continue;
            if (!resident) load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
            const float d2 = lane_dot<D>([&](int e) { return x[e] - c0[e]; }, [&](int e) { return x[e] - c0[e]; });
            if (d2 > bv) {
              bv = d2;
              bi = i;
            }
          }
          const int sel = seg_argmax_idx(bv, bi, L);
          if (live) load_row_g<T, D>(kb + (int64_t)s_perm[gb + sel] * kst, acc1);
          wave_sync();
          float* dst = pass == 0 ? c0 : c1;
          if (live) {
#pragma unroll
            for (int d = 0; d < D; d += 4)
              *reinterpret_cast<float4*>(dst + d) = make_float4(acc1[d], acc1[d + 1], acc1[d + 2], acc1[d + 3]);
          }
          wave_sync();
        }
        // Lloyd iterations: labels from the current centroids, then both masked sums, in one pass
        for (int it = 0; it < iters; ++it) {
          const float cc0 = lane_dot<D>([&](int e) { return c0[e]; }, [&](int e) { return c0[e]; });
          const float cc1 = lane_dot<D>([&](int e) { return c1[e]; }, [&](int e) { return c1[e]; });
#pragma unroll
          for (int d = 0; d < D; ++d) {
            acc0[d] = 0.0f;
            acc1[d] = 0.0f;
          }
          float cp0 = 0.0f, cp1 = 0.0f;
          for (int t = 0; t < M; ++t) {
            const int s = gb + gl + L * t;
            if (!live || !s_val[s]) continue;
            if (!resident) load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
            const float xx = lane_dot<D>([&](int e) { return x[e]; }, [&](int e) { return x[e]; });
            const float xc0 = lane_dot<D>([&](int e) { return x[e]; }, [&](int e) { return c0[e]; });
            const float xc1 = lane_dot<D>([&](int e) { return x[e]; }, [&](int e) { return c1[e]; });
            const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
            if (dist1 < dist0) {
              if (!resident) {
#pragma unroll
                for (int d = 0; d < D; ++d) acc1[d] = acc1[d] + x[d];
              }
              cp1 = cp1 + 1.0f;
            } else {
              if (!resident) {
#pragma unroll
                for (int d = 0; d < D; ++d) acc0[d] = acc0[d] + x[d];
              }
              cp0 = cp0 + 1.0f;
            }
          }
          const float cj0 = seg_sum(cp0, L), cj1 = seg_sum(cp1, L);
          if (gl == 0) {
            s_cnt[g] = cj0;
            s_cnt[kLtGroups + g] = cj1;
          }
          if (resident) lt_group_row<D>(x, cp0 > 0.0f, s_red, lane);
          else lt_group_row<D>(acc0, true, s_red, lane);
          lt_group_reduce<D>(s_red, L, s_cnt, false, c0 - g * RS, lane);
          if (resident) lt_group_row<D>(x, cp1 > 0.0f, s_red, lane);
          else lt_group_row<D>(acc1, true, s_red, lane);
          lt_group_reduce<D>(s_red, L, s_cnt + kLtGroups, false, c1 - g * RS, lane);
        }
      }
      const int nl = (ng + 1) / 2, nr = ng - nl;
      if (S >= kWave) {
        // one group: projections on c0 - c1 over the span of the real keys (empty slots inside it: +inf),
        // padded to a power of two with entries that sort last; bitonic sort
        if (ng > 0) {
          const int n = vhi - vlo + 1;
          int n2 = 1;
          while (n2 < n) n2 <<= 1;
          for (int t = 0; t < M; ++t) {
            const int i = lane + kWave * t, s = gb + i;
            if (i < vlo || i > vhi) continue;
            float pr = kInf;
            if (s_val[s]) {
              if (!resident) load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
              pr = lane_dot<D>([&](int e) { return x[e]; }, [&](int e) { return c0[e] - c1[e]; });
            }
            s_sort[i - vlo] = lt_sort_key(pr, i - vlo);
          }
          for (int r = n + lane; r < n2; r += kWave) s_sort[r] = lt_sort_key(kInf, r);
          wave_sync();
          wave_bitonic_sort(s_sort, n2, lane);
        }
        // layout: sorted ranks [0, nl) to the left half, [nl, ng) to the right half (phase A rewrites each
        // sort word as (position, key position) before phase B moves the permutation)
        for (int r = lane; r < ng; r += kWave) {
          const int m = vlo + (int)(uint32_t)s_sort[r];
          const int pos = r < nl ? r : half + r - nl;
          s_sort[r] = ((uint64_t)(uint32_t)pos << 32) | (uint32_t)s_perm[gb + m];
        }
        const int fillp = lastinv >= 0 ? s_perm[gb + lastinv] : 0;
        wave_sync();
        for (int r = lane; r < ng; r += kWave) {
          const uint64_t e = s_sort[r];
          s_perm[gb + (int)(e >> 32)] = (int32_t)(uint32_t)e;
        }
        for (int p = lane; p < S; p += kWave) {
          const bool filled = p < half ? p < nl : (p - half) < nr;
          if (!filled) s_perm[gb + p] = fillp;
          s_val[gb + p] = filled ? 1 : 0;
        }
        wave_sync();
      } else {
        // groups of S < 64 side by side, one member per lane: ranks by counting
        const int s = gb + gl;
        const bool v = live && s_val[s];
        float key = kInf;
        if (v) {
          key = lane_dot<D>([&](int e) { return x[e]; }, [&](int e) { return c0[e] - c1[e]; });
        }
        if (live) s_key[s] = key;
        wave_sync();
        int rank = 0;
        if (v) {
          for (int j = 0; j < S; ++j) {
            const float kj = s_key[gb + j];
            rank += (kj < key || (kj == key && j < gl)) ? 1 : 0;
          }
        }
        const int pm = live ? s_perm[s] : 0;
        const int fillp = live && lastinv >= 0 ? s_perm[gb + lastinv] : 0;
        wave_sync();
        if (v) s_perm[gb + (rank < nl ? rank : half + rank - nl)] = pm;
        if (live) {
          const bool filled = gl < half ? gl < nl : (gl - half) < nr;
          if (!filled) s_perm[s] = fillp;
          s_val[s] = filled ? 1 : 0;
        }
        wave_sync();
      }
    }
  }
  // leaf slots, then the node sums and counts by adjacent pairs from the slots up
  for (int c = lane; c < C; c += kWave) tr.slot[c] = s_val[c] ? s_perm[c] : -1;
  const int nleaf = C / 2;
  for (int i = lane; i < nleaf; i += kWave) {
    float y[D];
    load_row_g<T, D>(kb + (int64_t)s_perm[2 * i] * kst, x);
    load_row_g<T, D>(kb + (int64_t)s_perm[2 * i + 1] * kst, y);
    const float v0 = s_val[2 * i] ? 1.0f : 0.0f, v1 = s_val[2 * i + 1] ? 1.0f : 0.0f;
    float* row = tr.sums + (int64_t)(nleaf - 1 + i) * D;
#pragma unroll
    for (int d = 0; d < D; d += 4)
      *reinterpret_cast<float4*>(row + d) =
          make_float4(x[d] * v0 + y[d] * v1, x[d + 1] * v0 + y[d + 1] * v1, x[d + 2] * v0 + y[d + 2] * v1,
                      x[d + 3] * v0 + y[d + 3] * v1);
    tr.cnt[nleaf - 1 + i] = (int)s_val[2 * i] + (int)s_val[2 * i + 1];
  }
  for (int lv = nlev - 1; lv >= 0; --lv) {
    __threadfence_block();
    const int nn = 1 << lv, base = nn - 1, cb = 2 * nn - 1;
    for (int i = lane; i < nn; i += kWave) {
      const float* a = tr.sums + (int64_t)(cb + 2 * i) * D;
      float* row = tr.sums + (int64_t)(base + i) * D;
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 u = *reinterpret_cast<const float4*>(a + d);
        const float4 w = *reinterpret_cast<const float4*>(a + D + d);
        *reinterpret_cast<float4*>(row + d) = make_float4(u.x + w.x, u.y + w.y, u.z + w.z, u.w + w.w);
      }
      tr.cnt[base + i] = tr.cnt[cb + 2 * i] + tr.cnt[cb + 2 * i + 1];
    }
  }
}

// ----------------------------------------------------------------------------------------------------- walk
struct LaneWalk {
  const void* q;
  const void* k;
  int64_t qsb, qsh, qst, ksb, ksh, kst;
  const int32_t* lhat;   // (B, H, T) leaf budget per query
  float* ws;
  int64_t P;
  int H, T, C, nlev, nlane, chunk, wmax, wl, Wn, NS, probe, cap_min, neighbors;
  int ntop;   // nodes held in LDS during the walk
  float rho;
  int32_t* tree_pos;   // (B, H, T, 2 wl)
  uint8_t* leaf_ok;    // (B, H, T, wl)
  int32_t* nb_pos;     // (B, H, T, 2 Wn NS)
  int32_t* n_tree;     // (B, H, T)
  int32_t* nb_leaves;  // (B, H, T)
};

// The nodes of a lane tree during the walk: nodes [0, ntop) (its top levels) live in LDS for the whole walk
// (rows of stride D + 4 floats, and counts), deeper nodes in the workspace; the leaf slots (C entries) live in
// LDS too.  Every access below is uniform in which side it takes (one level at a time).
template <int D>
struct LaneNodes {
  LaneTree tr;
  float* top;
  int32_t* tcnt;
  int32_t* slot;   // LDS copy of the leaf slots
  int ntop, C;
  __device__ __forceinline__ int cnt(int n) const { return n < ntop ? tcnt[n] : tr.cnt[n]; }
  __device__ __forceinline__ void set_cnt(int n, int v) const {
    if (n < ntop) tcnt[n] = v;
    else tr.cnt[n] = v;
  }
  __device__ __forceinline__ float elem(int n, int d) const {
    return n < ntop ? top[n * (D + 4) + d] : tr.sums[(int64_t)n * D + d];
  }
  __device__ __forceinline__ void set_elem(int n, int d, float v) const {
    if (n < ntop) top[n * (D + 4) + d] = v;
    else tr.sums[(int64_t)n * D + d] = v;
  }
  __device__ __forceinline__ void row(int n, float (&r)[D]) const {
    if (n < ntop) {
      const float* src = top + n * (D + 4);
#pragma unroll
      for (int d = 0; d < D; d += 4) {
        const float4 v = *reinterpret_cast<const float4*>(src + d);
        r[d] = v.x;
        r[d + 1] = v.y;
        r[d + 2] = v.z;
        r[d + 3] = v.w;
      }
    } else {
      load_row_g<float, D>(tr.sums + (int64_t)n * D, r);
    }
  }
  // workspace -> LDS (to_lds) or back
  __device__ __forceinline__ void copy(bool to_lds, int lane) const {
    for (int i = lane; i < ntop * (D / 4); i += kWave) {
      const int n = i / (D / 4), d = (i - n * (D / 4)) * 4;
      float4* l = reinterpret_cast<float4*>(top + n * (D + 4) + d);
      float4* g = reinterpret_cast<float4*>(tr.sums + (int64_t)n * D + d);
      if (to_lds) *l = *g;
      else *g = *l;
    }
    for (int n = lane; n < ntop; n += kWave) {
      if (to_lds) tcnt[n] = tr.cnt[n];
      else tr.cnt[n] = tcnt[n];
    }
    for (int n = lane; n < C; n += kWave) {
      if (to_lds) slot[n] = tr.slot[n];
      else tr.slot[n] = slot[n];
    }
  }
};

// Canonical dot of two D-vectors held one element per lane (lane d < D holds a[d] * b[d] in `prod`, 0 past D):
// the halving tree inside groups of R = D/16 consecutive lanes, then over the 16 groups (lanes R apart), as
// an xor butterfly (every lane ends with the sum).
template <int D>
__device__ __forceinline__ float dims_dot(float prod) {
  constexpr int R = D < 16 ? 1 : D / 16;
  if constexpr (R >= 4) prod = prod + xor_lane<2>(prod);
  if constexpr (R >= 2) prod = prod + xor_lane<1>(prod);
  if constexpr (8 * R >= 32) prod = prod + xor_lane<32>(prod);
  if constexpr (8 * R >= 16 && R <= 16) prod = prod + xor_lane<16>(prod);
  if constexpr (R <= 8) prod = prod + xor_lane<8>(prod);
  if constexpr (R <= 4) prod = prod + xor_lane<4>(prod);
  if constexpr (R <= 2) prod = prod + xor_lane<2>(prod);
  if constexpr (R <= 1) prod = prod + xor_lane<1>(prod);
  return prod;
}

// Search ranking word: valid first, then score descending, node id ascending; invalid candidates by slot.
// Unique per candidate, so a candidate's rank is the number of smaller words.
__device__ __forceinline__ uint64_t lt_rank_word(bool valid, float sc, int id, int slot) {
  if (!valid) return (1ull << 63) | (uint32_t)slot;
  const uint32_t u = __float_as_uint(sc + 0.0f);
  const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)(~asc) << 31) | (uint32_t)id;
}

// One wavefront per lane tree, built by lanetree_build_kernel, walking the lane's positions in order
// (dyntree.py:148-243).  The tree state is read back by the same wavefront after its own stores; a
// workgroup-scope fence ends every position.
template <typename T, int D>
__global__ __launch_bounds__(kWave) void lanetree_walk_kernel(LaneWalk p) {
  __shared__ int32_t s_stl[kLaneMaxNb];   // stored leaves of the last Wn positions (ring), NS each
  __shared__ float s_sts[kLaneMaxNb];
  __shared__ uint8_t s_sto[kLaneMaxNb];
  __shared__ int32_t s_nid[kWave];
  __shared__ __align__(16) uint64_t s_rw[kWave];   // the level's children's ranking words
  __shared__ int32_t s_cur[kWave];   // the beam
  __shared__ float s_bsc[kWave];
  __shared__ uint8_t s_bok[kWave];
  const int lane = lane_id();
  const int64_t pt = blockIdx.x;
  const int ln = (int)(pt % p.nlane);
  const int64_t bh = pt / p.nlane;
  const int64_t b = bh / p.H, h = bh % p.H;
  const T* qb = static_cast<const T*>(p.q) + b * p.qsb + h * p.qsh;
  const T* kb = static_cast<const T*>(p.k) + b * p.ksb + h * p.ksh;
  const LaneTree tr = lane_tree(p.ws, p.P, p.C, D, pt);
  extern __shared__ __align__(16) unsigned char s_dyn[];
  LaneNodes<D> nd;
  nd.tr = tr;
  nd.top = reinterpret_cast<float*>(s_dyn);
  nd.tcnt = reinterpret_cast<int32_t*>(nd.top + p.ntop * (D + 4));
  nd.slot = nd.tcnt + p.ntop;
  nd.ntop = p.ntop;
  nd.C = p.C;
  nd.copy(true, lane);
  wave_sync();
  const int WN = p.Wn * p.NS, wl = p.wl, nlev = p.nlev;
  const float kInf = __int_as_float(0x7f800000);
  const int start = ln * p.chunk;
  float qn[D];   // the next position's query and key, requested while the current position runs
  load_row_g<T, D>(qb + (int64_t)start * p.qst, qn);
  float kn = lane < D ? to_f32(kb[(int64_t)start * p.kst + lane]) : 0.0f;
  for (int i = 0; i < p.chunk; ++i) {
    const int t = start + i;
    const int64_t orow = bh * p.T + t;
    float qv[D];
#pragma unroll
    for (int d = 0; d < D; ++d) qv[d] = qn[d];
    const float kd = kn;
    if (i + 1 < p.chunk) {
      load_row_g<T, D>(qb + (int64_t)(t + 1) * p.qst, qn);
      kn = lane < D ? to_f32(kb[(int64_t)(t + 1) * p.kst + lane]) : 0.0f;
    }
    // ---- neighbours: the leaves the last Wn positions of the lane stored, re-scored on the current tree
    int id = 0;
    bool ok0 = false, match = false;
    if (lane < WN) {
      const int back = lane / p.NS + 1, j = i - back;
      if (j >= 0) {
        const int rs = (j % p.Wn) * p.NS + lane % p.NS;
        ok0 = s_sto[rs] != 0;
        id = s_stl[rs];
        if (ok0) {
          const int node = (1 << nlev) - 1 + id;
          const int cn = nd.cnt(node);
          float row[D];
          nd.row(node, row);
          const float sc = lane_dot<D>([&](int e) { return qv[e]; }, [&](int e) { return row[e]; }) /
                           (float)(cn > 1 ? cn : 1);
          const float base = s_sts[rs];
          match = cn > 0 && sc >= base - p.rho * fabsf(base);
        }
      }
    }
    const bool inprobe = lane < p.probe;
    const int pm = __popcll(__ballot(match && inprobe)), po = __popcll(__ballot(ok0 && inprobe));
    const float rate = (float)pm / fmaxf((float)po, 1.0f);
    const int cap = p.cap_min + (int)rintf((float)(p.Wn - p.cap_min) * rate);
    match = match && (lane / p.NS + 1) <= cap && p.neighbors;
    s_nid[lane] = match ? id : -1;
    wave_sync();
    bool first = match;
    for (int e = 0; e < lane && first; ++e) first = s_nid[e] != id;
    const int nL = __popcll(__ballot(first));
    if (lane < WN) {
      const int s0 = nd.slot[2 * id], s1 = nd.slot[2 * id + 1];
      int32_t* o = p.nb_pos + orow * 2 * WN;
      o[lane] = match && s0 >= 0 ? s0 : -1;
      o[WN + lane] = match && s1 >= 0 ? s1 : -1;
    }
    // ---- budget (dyntree.py:218-222)
    const int Lq = p.lhat[orow];
    const int lo = (Lq + 1) >> 1, need = Lq - nL > 0 ? Lq - nL : 0, floor_b = nL < lo ? 2 : 1;
    int bt = nL >= Lq ? 0 : (need > floor_b ? need : floor_b);
    bt = bt < p.wmax ? bt : p.wmax;
    // ---- beam search from the root
    if (lane == 0) {
      s_cur[0] = 0;
      s_bok[0] = nd.cnt(0) > 0;
      s_bsc[0] = 0.0f;
    }
    wave_sync();
    int wp = 1;
    for (int lv = 1; lv <= nlev; ++lv) {
      const int nch = 2 * wp;
      int cid = 0;
      bool cv = false;
      float sc = -kInf;
      if (lane < nch) {
        const int par = lane < wp ? lane : lane - wp;
        cid = 2 * s_cur[par] + (lane < wp ? 0 : 1);
        if (s_bok[par]) {
          const int node = (1 << lv) - 1 + cid;
          const int cn = nd.cnt(node);
          float row[D];
          nd.row(node, row);
          cv = cn > 0;
          if (cv)
            sc = lane_dot<D>([&](int e) { return qv[e]; }, [&](int e) { return row[e]; }) / (float)(cn > 1 ? cn : 1);
        }
        s_rw[lane] = lt_rank_word(cv, sc, cid, lane);
      }
      wave_sync();
      const int w = nch < p.wmax ? nch : p.wmax;
      if (lane < nch) {
        const uint64_t mine = s_rw[lane];
        int rank = 0;
        for (int j0 = 0; j0 < nch; j0 += 8) {   // words read four pairs at a time
          uint64_t wv[8];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint4 two = *reinterpret_cast<const uint4*>(s_rw + j0 + 2 * h);
            wv[2 * h] = ((uint64_t)two.y << 32) | two.x;
            wv[2 * h + 1] = ((uint64_t)two.w << 32) | two.z;
          }
#pragma unroll
          for (int h = 0; h < 8; ++h) rank += (j0 + h < nch && wv[h] < mine) ? 1 : 0;
        }
        if (rank < w) {
          s_cur[rank] = cid;
          s_bsc[rank] = sc;
          s_bok[rank] = cv;
        }
      }
      wave_sync();
      wp = w;
    }
    // ---- outputs, and the stored leaves of this position
    if (lane < wl) {
      const int lid = s_cur[lane];
      const bool ok = s_bok[lane] != 0;
      const int s0 = nd.slot[2 * lid], s1 = nd.slot[2 * lid + 1];
      int32_t* o = p.tree_pos + orow * 2 * wl;
      o[lane] = ok && s0 >= 0 ? s0 : -1;
      o[wl + lane] = ok && s1 >= 0 ? s1 : -1;
      p.leaf_ok[orow * wl + lane] = ok ? 1 : 0;
    }
    if (lane == 0) {
      p.n_tree[orow] = bt;
      p.nb_leaves[orow] = nL;
    }
    if (lane < p.NS) {
      const int rs = (i % p.Wn) * p.NS + lane;
      s_stl[rs] = s_cur[lane];
      s_sts[rs] = s_bsc[lane];
      s_sto[rs] = s_bok[lane];
    }
    // ---- insertion of this position's key (dyntree.py:84-106), one dimension per lane
    const int act = t >= 1 ? 1 : 0;
    const float kva = kd * (act ? 1.0f : 0.0f);
    if (lane < D) nd.set_elem(0, lane, nd.elem(0, lane) + kva);
    if (lane == 0) nd.set_cnt(0, nd.cnt(0) + act);
    int node = 0;
    for (int lv = 0; lv < nlev; ++lv) {
      const int base = (2 << lv) - 1, lc = 2 * node, cap = p.C >> (lv + 1);
      const int cL = nd.cnt(base + lc), cR = nd.cnt(base + lc + 1);
      const float xL = lane < D ? nd.elem(base + lc, lane) : 0.0f;
      const float xR = lane < D ? nd.elem(base + lc + 1, lane) : 0.0f;
      const float dL = dims_dot<D>(kd * xL), dR = dims_dot<D>(kd * xR);
      float sL = cL == 0 ? -1e9f : dL / (float)(cL > 1 ? cL : 1);
      float sR = cR == 0 ? -1e9f : dR / (float)(cR > 1 ? cR : 1);
      if (cL >= cap) sL = -kInf;
      if (cR >= cap) sR = -kInf;
      const bool right = sR > sL;
      node = lc + (right ? 1 : 0);
      if (lane < D) nd.set_elem(base + node, lane, (right ? xR : xL) + kva);
      if (lane == 0) nd.set_cnt(base + node, (right ? cR : cL) + act);
    }
    if (lane == 0 && act) {
      const int s0 = nd.slot[2 * node];
      nd.slot[2 * node + (s0 >= 0 ? 1 : 0)] = t;
    }
    __threadfence_block();
    wave_sync();
  }
  nd.copy(false, lane);
}

bool lanetree_dim_ok(int D) { return D == 16 || D == 32 || D == 64; }

int lanetree_levels(int T) {
  int lg = 0;
  while ((1 << lg) < T) ++lg;
  return lg - 1;
}

}  // namespace ta

using namespace ta;

extern "C" int ta_lanetree_workspace_size(int B, int H, int T, int D, int chunk, int64_t* bytes) {
  if (B <= 0 || H <= 0 || T < 4 || T > kLaneMaxT || (T & (T - 1)) || chunk <= 0 || T % chunk ||
      !lanetree_dim_ok(D) || bytes == nullptr) {
    set_error("ta_lanetree_workspace_size: bad arguments (T a power of two in [4, 4096], chunk dividing T, "
              "D 16, 32 or 64)");
    return TA_ERR_ARG;
  }
  const int64_t P = (int64_t)B * H * (T / chunk);
  *bytes = P * T * ((int64_t)D * 4 + 8);
  return TA_OK;
}

extern "C" int ta_lanetree_build(const void* k, int dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int T,
                                 int D, int chunk, int kmeans_iters, void* ws, int64_t ws_bytes, void* stream) {
  int64_t need = 0;
  if (ta_lanetree_workspace_size(B, H, T, D, chunk, &need) != TA_OK) return TA_ERR_ARG;
  if (k == nullptr || ws == nullptr || ws_bytes < need || kmeans_iters < 0 || ((uintptr_t)ws % 16)) {
    set_error("ta_lanetree_build: bad arguments (null pointer, workspace too small or unaligned, or negative "
              "kmeans_iters)");
    return TA_ERR_ARG;
  }
  const int es = dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)k % 16) || (ksb * es) % 16 || (ksh * es) % 16 || (kst * es) % 16) {
    set_error("ta_lanetree_build: key rows 16-byte aligned");
    return TA_ERR_ARG;
  }
  const int64_t P = (int64_t)B * H * (T / chunk);
  const size_t red = (size_t)kWave * (D + 4) * 4;
  const size_t lds = (size_t)T * 4 + ((size_t)T * 8 > red ? (size_t)T * 8 : red) +
                     (size_t)2 * kLtGroups * (D + 4) * 4 + (size_t)2 * kLtGroups * 4 + (size_t)T;
  hipStream_t st = (hipStream_t)stream;
#define TA_LB(TT, DD)                                                                                          \
  hipLaunchKernelGGL((lanetree_build_kernel<TT, DD>), dim3((unsigned)P), dim3(kWave), lds, st, (const TT*)k, \
                     ksb, ksh, kst, H, T, T / chunk, chunk, kmeans_iters, (float*)ws, P)
#define TA_LB_D(TT)                  \
  switch (D) {                       \
    case 16: TA_LB(TT, 16); break;   \
    case 32: TA_LB(TT, 32); break;   \
    default: TA_LB(TT, 64); break;   \
  }
  switch (dtype) {
    case TA_F32: TA_LB_D(float); break;
    case TA_BF16: TA_LB_D(bf16_t); break;
    case TA_F16: TA_LB_D(f16_t); break;
    default:
      set_error("ta_lanetree_build: unsupported dtype");
      return TA_ERR_ARG;
  }
#undef TA_LB_D
#undef TA_LB
  return check_launch("ta_lanetree_build");
}

extern "C" int ta_lanetree_walk(const void* q, const void* k, int dtype, int64_t qsb, int64_t qsh, int64_t qst,
                                int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int T, int D, int chunk,
                                const int32_t* lhat, int wmax, int nb_window, int nb_store, float nb_rho,
                                int nb_probe, int nb_cap_min, int neighbors, void* ws, int64_t ws_bytes,
                                int32_t* tree_pos, uint8_t* leaf_ok, int32_t* nb_pos, int32_t* n_tree,
                                int32_t* nb_leaves, void* stream) {
  int64_t need = 0;
  if (ta_lanetree_workspace_size(B, H, T, D, chunk, &need) != TA_OK) return TA_ERR_ARG;
  const int nlev = lanetree_levels(T);
  const int wl = wmax < (1 << nlev) ? wmax : (1 << nlev);
  if (q == nullptr || k == nullptr || lhat == nullptr || ws == nullptr || ws_bytes < need || tree_pos == nullptr ||
      leaf_ok == nullptr || nb_pos == nullptr || n_tree == nullptr || nb_leaves == nullptr || wmax < 1 ||
      wmax > kLaneMaxW || nb_window < 1 || nb_store < 1 || nb_window * nb_store > kLaneMaxNb || nb_store > wl ||
      nb_probe < 0 || !(nb_rho == nb_rho)) {
    set_error("ta_lanetree_walk: bad arguments (1 <= wmax <= 32, nb_window * nb_store <= 64, nb_store at most "
              "the leaves per query, workspace from ta_lanetree_workspace_size)");
    return TA_ERR_ARG;
  }
  const int es = dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)q % 16) || (qsb * es) % 16 || (qsh * es) % 16 || (qst * es) % 16) {
    set_error("ta_lanetree_walk: query rows 16-byte aligned");
    return TA_ERR_ARG;
  }
  LaneWalk p{};
  p.q = q; p.k = k;
  p.qsb = qsb; p.qsh = qsh; p.qst = qst; p.ksb = ksb; p.ksh = ksh; p.kst = kst;
  p.lhat = lhat;
  p.ws = (float*)ws;
  p.P = (int64_t)B * H * (T / chunk);
  p.H = H; p.T = T; p.C = T; p.nlev = nlev; p.nlane = T / chunk; p.chunk = chunk;
  p.wmax = wmax; p.wl = wl; p.Wn = nb_window; p.NS = nb_store; p.probe = nb_probe * nb_store;
  p.cap_min = nb_cap_min; p.neighbors = neighbors ? 1 : 0; p.rho = nb_rho;
  p.tree_pos = tree_pos; p.leaf_ok = leaf_ok; p.nb_pos = nb_pos; p.n_tree = n_tree; p.nb_leaves = nb_leaves;
  // the top levels of every tree stay in LDS during the walk: as many whole levels as fit in 40 KB
  const int rowb = (D + 4) * 4 + 4;
  int ntop = 1;
  while (2 * ntop + 1 <= T - 1 && (2 * ntop + 1) * rowb <= 40960) ntop = 2 * ntop + 1;
  p.ntop = ntop;
  const size_t lds = (size_t)ntop * rowb + (size_t)T * 4;   // + the leaf slots
  hipStream_t st = (hipStream_t)stream;
#define TA_LW(TT, DD) \
  hipLaunchKernelGGL((lanetree_walk_kernel<TT, DD>), dim3((unsigned)p.P), dim3(kWave), lds, st, p)
#define TA_LW_D(TT)                  \
  switch (D) {                       \
    case 16: TA_LW(TT, 16); break;   \
    case 32: TA_LW(TT, 32); break;   \
    default: TA_LW(TT, 64); break;   \
  }
  switch (dtype) {
    case TA_F32: TA_LW_D(float); break;
    case TA_BF16: TA_LW_D(bf16_t); break;
    case TA_F16: TA_LW_D(f16_t); break;
    default:
      set_error("ta_lanetree_walk: unsupported dtype");
      return TA_ERR_ARG;
  }
#undef TA_LW_D
#undef TA_LW
  return check_launch("ta_lanetree_walk");
}
