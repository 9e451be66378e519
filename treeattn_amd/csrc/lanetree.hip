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
__device__ __forceinline__ int seg_argmax_idx(float v, int i, int L) {
  for (int h = L >> 1; h >= 1; h >>= 1) {
    const float ov = __shfl_xor(v, h, kWave);
    const int oi = __shfl_xor(i, h, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  return i;
}

// The group member (index inside the group) with the largest squared distance to ref among the real keys,
// the first on ties; -1 stands for empty slots (masked_fill(~valid, -1)).
template <typename T, int D>
__device__ __forceinline__ int lt_farthest(const T* kb, int64_t kst, const int32_t* s_perm, const uint8_t* s_val,
                                           int wb, int gb, int lane, int M, int L, bool live,
                                           const float (&ref)[D], float (&x)[D]) {
  float bv = -1.0f;
  int bi = 0;
  for (int t = 0; t < M; ++t) {
    const int s = wb + lane + kWave * t;
    float d2 = -1.0f;
    if (live) {
      load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
      const float dd = lane_dot<D>([&](int i) { return x[i] - ref[i]; }, [&](int i) { return x[i] - ref[i]; });
      d2 = s_val[s] ? dd : -1.0f;
    }
    if (t == 0 || d2 > bv) {
      bv = d2;
      bi = s - gb;
    }
  }
  return seg_argmax_idx(bv, bi, L);
}

// ---------------------------------------------------------------------------------------------------- build
// One wavefront per lane tree (dyntree.py:34-82).  Every level splits each group of S = C >> lvl slots by a
// masked 2-means projection; the group's real keys are then laid out half and half (the larger half first),
// empty slots after each half's keys.  Groups of S >= 64 slots are done one at a time, lane j holding members
// j, j + 64, ...; smaller groups side by side, one member per lane.  The permutation, validity and projections
// live in LDS; key rows are read from k on every pass.
template <typename T, int D>
__global__ __launch_bounds__(kWave) void lanetree_build_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                                               int64_t kst, int H, int C, int nlane, int chunk,
                                                               int iters, float* __restrict__ ws, int64_t P) {
  extern __shared__ __align__(16) unsigned char s_raw[];
  int32_t* s_perm = reinterpret_cast<int32_t*>(s_raw);
  float* s_proj = reinterpret_cast<float*>(s_perm + C);
  int32_t* s_np = reinterpret_cast<int32_t*>(s_proj + C);
  uint8_t* s_val = reinterpret_cast<uint8_t*>(s_np + C);
  uint8_t* s_nv = s_val + C;
  const int lane = lane_id();
  const int64_t pt = blockIdx.x;
  const int ln = (int)(pt % nlane);
  const int64_t bh = pt / nlane;
  const T* kb = k + (bh / H) * ksb + (bh % H) * ksh;
  const int n0 = ln * chunk;
  const LaneTree tr = lane_tree(ws, P, C, D, pt);
  for (int c = lane; c < C; c += kWave) {
    s_perm[c] = c;
    s_val[c] = (c >= 1 && c < n0) ? 1 : 0;
  }
  wave_sync();
  const int nlev = lt_log2(C) - 1;
  float x[D], c0[D], c1[D], acc[D];
  for (int lvl = 0; lvl < nlev; ++lvl) {
    const int S = C >> lvl;
    const int L = S < kWave ? S : kWave;       // partial sums per group
    const int M = S < kWave ? 1 : S / kWave;   // members per lane
    const int Wz = S < kWave ? kWave : S;      // slots per window
    const int nwin = C > Wz ? C / Wz : 1;
    for (int win = 0; win < nwin; ++win) {
      const int wb = win * Wz;
      const int gb = S < kWave ? wb + (lane & ~(S - 1)) : wb;   // this lane's group
      const bool live = wb + lane < C;                          // C < 64: lanes past the tree sit out
      // (1) valid count and masked mean
      float cntp = 0.0f;
      for (int t = 0; t < M; ++t) {
        const int s = wb + lane + kWave * t;
        const float v = live && s_val[s] ? 1.0f : 0.0f;
        if (live) load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const float xv = live ? x[d] * v : 0.0f;
          acc[d] = t == 0 ? xv : acc[d] + xv;
        }
        cntp = t == 0 ? v : cntp + v;
      }
      const float cnt = seg_sum(cntp, L);
      const int ng = (int)cnt;
      const float den = fmaxf(cnt, 1.0f);
#pragma unroll
      for (int d = 0; d < D; ++d) c0[d] = seg_sum(acc[d], L) / den;   // c0 = the mean for now
      const bool work = __ballot(live && ng > 0) != 0;           // no real key in the window: identity order
      if (work) {
        // (2) a = the member farthest from the mean, b = the member farthest from a
        const int ia = lt_farthest<T, D>(kb, kst, s_perm, s_val, wb, gb, lane, M, L, live, c0, x);
        if (live) load_row_g<T, D>(kb + (int64_t)s_perm[gb + ia] * kst, c0);
        const int ib = lt_farthest<T, D>(kb, kst, s_perm, s_val, wb, gb, lane, M, L, live, c0, x);
        if (live) load_row_g<T, D>(kb + (int64_t)s_perm[gb + ib] * kst, c1);
        // (3) Lloyd iterations over the two centroids
        for (int it = 0; it < iters; ++it) {
          const float cc0 = lane_dot<D>([&](int i) { return c0[i]; }, [&](int i) { return c0[i]; });
          const float cc1 = lane_dot<D>([&](int i) { return c1[i]; }, [&](int i) { return c1[i]; });
          uint64_t lab = 0;   // bit t: member t of this lane is nearer c1
          for (int t = 0; t < M; ++t) {
            const int s = wb + lane + kWave * t;
            if (!live) continue;
            load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
            const float xx = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return x[i]; });
            const float xc0 = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c0[i]; });
            const float xc1 = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c1[i]; });
            const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
            if (dist1 < dist0) lab |= 1ull << t;
          }
          for (int j = 0; j < 2; ++j) {
            float cp = 0.0f;
            for (int t = 0; t < M; ++t) {
              const int s = wb + lane + kWave * t;
              const bool in = live && s_val[s] && (((lab >> t) & 1ull) == (uint64_t)j);
              const float m = in ? 1.0f : 0.0f;
              if (live) load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
#pragma unroll
              for (int d = 0; d < D; ++d) {
                const float xv = live ? x[d] * m : 0.0f;
                acc[d] = t == 0 ? xv : acc[d] + xv;
              }
              cp = t == 0 ? m : cp + m;
            }
            const float cj = seg_sum(cp, L);
            const float dj = fmaxf(cj, 1.0f);
#pragma unroll
            for (int d = 0; d < D; ++d) {
              const float nc = seg_sum(acc[d], L) / dj;
              if (j == 0) c0[d] = cj > 0.0f ? nc : c0[d];
              else c1[d] = cj > 0.0f ? nc : c1[d];
            }
          }
        }
        // (4) projections on c0 - c1, empty slots last
        for (int t = 0; t < M; ++t) {
          const int s = wb + lane + kWave * t;
          if (!live) continue;
          load_row_g<T, D>(kb + (int64_t)s_perm[s] * kst, x);
          const float pr = lane_dot<D>([&](int i) { return x[i]; }, [&](int i) { return c0[i] - c1[i]; });
          s_proj[s] = s_val[s] ? pr : __int_as_float(0x7f800000);
        }
        wave_sync();
      }
      // (5) stable ranks, then the balanced layout: ranks [0, nl) to the left half, [nl, ng) to the right half
      const int nl = (ng + 1) / 2, nr = ng - nl, half = S / 2;
      for (int t = 0; t < M; ++t) {
        const int s = wb + lane + kWave * t;
        if (!live) continue;
        const int mi = s - gb;
        int rank = mi;
        if (work) {
          const float pi = s_proj[s];
          rank = 0;
          for (int j = 0; j < S; ++j) {
            const float pj = s_proj[gb + j];
            rank += (pj < pi || (pj == pi && j < mi)) ? 1 : 0;
          }
        }
        const int pm = s_perm[s];
        int r = -1;
        if (rank < nl) r = rank;
        else if (rank < ng) r = half + rank - nl;
        if (r >= 0) {
          s_np[gb + r] = pm;
          s_nv[gb + r] = 1;
        } else if (rank == S - 1) {
          s_np[gb + S - 1] = pm;   // every empty slot of the group takes the last-ranked member's position
        }
      }
      wave_sync();
      for (int t = 0; t < M; ++t) {
        const int s = wb + lane + kWave * t;
        if (!live) continue;
        const int r = s - gb;
        const bool filled = r < half ? r < nl : (r - half) < nr;
        if (!filled) {
          s_np[s] = s_np[gb + S - 1];
          s_nv[s] = 0;
        }
      }
      wave_sync();
      for (int t = 0; t < M; ++t) {
        const int s = wb + lane + kWave * t;
        if (!live) continue;
        s_perm[s] = s_np[s];
        s_val[s] = s_nv[s];
      }
      wave_sync();
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
  float rho;
  int32_t* tree_pos;   // (B, H, T, 2 wl)
  uint8_t* leaf_ok;    // (B, H, T, wl)
  int32_t* nb_pos;     // (B, H, T, 2 Wn NS)
  int32_t* n_tree;     // (B, H, T)
  int32_t* nb_leaves;  // (B, H, T)
};

// Canonical dot of two D-vectors held one element per lane (lane d < D holds a[d] * b[d] in `prod`): the
// halving tree inside groups of R = D/16 consecutive lanes, then over the 16 groups (lanes R apart).
template <int D>
__device__ __forceinline__ float dims_dot(float prod) {
  constexpr int R = D < 16 ? 1 : D / 16;
  for (int h = R >> 1; h >= 1; h >>= 1) prod = prod + __shfl_xor(prod, h, kWave);
  for (int h = 8 * R; h >= R; h >>= 1) prod = prod + __shfl_xor(prod, h, kWave);
  return prod;
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
  __shared__ int32_t s_cid[kWave];   // the level's children
  __shared__ float s_csc[kWave];
  __shared__ uint8_t s_ccv[kWave];
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
  const int WN = p.Wn * p.NS, wl = p.wl, nlev = p.nlev;
  const float kInf = __int_as_float(0x7f800000);
  const int start = ln * p.chunk;
  for (int i = 0; i < p.chunk; ++i) {
    const int t = start + i;
    const int64_t orow = bh * p.T + t;
    float qv[D];
    load_row_g<T, D>(qb + (int64_t)t * p.qst, qv);
    const float kd = lane < D ? to_f32(kb[(int64_t)t * p.kst + lane]) : 0.0f;
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
          const int cn = tr.cnt[node];
          float row[D];
          load_row_g<float, D>(tr.sums + (int64_t)node * D, row);
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
      const int s0 = tr.slot[2 * id], s1 = tr.slot[2 * id + 1];
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
      s_bok[0] = tr.cnt[0] > 0;
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
          const int cn = tr.cnt[node];
          float row[D];
          load_row_g<float, D>(tr.sums + (int64_t)node * D, row);
          cv = cn > 0;
          if (cv)
            sc = lane_dot<D>([&](int e) { return qv[e]; }, [&](int e) { return row[e]; }) / (float)(cn > 1 ? cn : 1);
        }
        s_cid[lane] = cid;
        s_csc[lane] = sc;
        s_ccv[lane] = cv;
      }
      wave_sync();
      const int w = nch < p.wmax ? nch : p.wmax;
      if (lane < nch) {
        int rank = 0;
        for (int j = 0; j < nch; ++j) {
          const bool vj = s_ccv[j] != 0;
          bool before;
          if (vj != cv) before = vj;
          else if (cv) before = s_csc[j] > sc || (s_csc[j] == sc && s_cid[j] < cid);
          else before = j < lane;
          rank += before ? 1 : 0;
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
      const int s0 = tr.slot[2 * lid], s1 = tr.slot[2 * lid + 1];
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
    if (lane < D) tr.sums[lane] = tr.sums[lane] + kva;
    if (lane == 0) tr.cnt[0] = tr.cnt[0] + act;
    int node = 0;
    for (int lv = 0; lv < nlev; ++lv) {
      const int base = (2 << lv) - 1, lc = 2 * node, cap = p.C >> (lv + 1);
      const int cL = tr.cnt[base + lc], cR = tr.cnt[base + lc + 1];
      const float xL = lane < D ? tr.sums[(int64_t)(base + lc) * D + lane] : 0.0f;
      const float xR = lane < D ? tr.sums[(int64_t)(base + lc + 1) * D + lane] : 0.0f;
      const float dL = dims_dot<D>(kd * xL), dR = dims_dot<D>(kd * xR);
      float sL = cL == 0 ? -1e9f : dL / (float)(cL > 1 ? cL : 1);
      float sR = cR == 0 ? -1e9f : dR / (float)(cR > 1 ? cR : 1);
      if (cL >= cap) sL = -kInf;
      if (cR >= cap) sR = -kInf;
      const bool right = sR > sL;
      node = lc + (right ? 1 : 0);
      if (lane < D) tr.sums[(int64_t)(base + node) * D + lane] = (right ? xR : xL) + kva;
      if (lane == 0) tr.cnt[base + node] = (right ? cR : cL) + act;
    }
    if (lane == 0 && act) {
      const int s0 = tr.slot[2 * node];
      tr.slot[2 * node + (s0 >= 0 ? 1 : 0)] = t;
    }
    __threadfence_block();
    wave_sync();
  }
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
  const size_t lds = (size_t)T * 14;
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
  hipStream_t st = (hipStream_t)stream;
#define TA_LW(TT, DD) \
  hipLaunchKernelGGL((lanetree_walk_kernel<TT, DD>), dim3((unsigned)p.P), dim3(kWave), 0, st, p)
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
