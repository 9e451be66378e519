// LaneTree: the key selection of the reference's 'dyn' attention.  The sequence is cut into lanes of `chunk`
// positions; lane l owns one balanced binary tree of capacity T over the keys [1, l * chunk) (the tree a
// sequential decoder would hold when it reaches the lane), then walks through the lane's positions one at a time:
// neighbour search over the leaves the lane's previous positions stored, beam search over the tree, store,
// insertion of the position's key.  The build runs a launch per level of groups above 64 slots (a workgroup per
// group), then one with a workgroup per window of 64 slots for the levels below, then the node sums above the
// windows; the walk runs a workgroup per lane tree.  The lane trees run in parallel.
//
// Inside a workgroup a row of D dimensions is held 16 dimensions per lane by Q = D / 16 consecutive lanes (a
// "slot"), so the workgroup's Q wavefronts form 64 slots: 64 members of the group or window being split (build)
// or 64 candidates being scored (walk) at a time.  A dot product of two rows is finished across the slot's lanes by
// DPP exchanges; reductions over slots run as xor butterflies inside a wavefront and through LDS across them.
//
// Reference functions replaced: dyntree.py:6-31 masked_two_means_order, dyntree.py:34-82 LaneTree.__init__,
// dyntree.py:84-106 insert, dyntree.py:108-127 search, dyntree.py:129-131 leaf_keys and dyntree.py:148-243
// select_keys.  The candidate list and the attention over it are the segment tree's (selection.assemble,
// ta_sparse_attn_fwd / ta_sparse_attn_bwd), as in attention_dyn.py:74-96.
//
// Arithmetic order (the CPU oracle's canonical mode computes the same, bit for bit):
//  * a mean or centroid over the S members of a group: L = min(S, 64) partial sums, partial j adding members
//    j, j + L, j + 2L, ... in that order, then the halving tree over the L partials; divided by the member
//    count (at least 1);
//  * dot products: per-dimension float32 products in canon_dot's order; node score = dot / max(count, 1);
//    dist = (|x|^2 - 2 x.c) + |c|^2;
//  * argmax: the first index; member order: stable ascending sort of the projections, empty slots last;
//  * the initial node sums: adjacent pairs over the slots, empty slots contributing key * 0; later insertions
//    add the key in insertion order;
//  * search ranking: valid first, score descending, node id ascending (invalid candidates by slot).
#pragma clang fp contract(off)

#include <type_traits>

#include "canon.hpp"
#include "trace.hpp"

namespace ta {

constexpr int kLaneMaxT = 262144;      // tree capacity = sequence length
constexpr int kLaneLdsMaxT = 16384;    // up to here the build keeps its 8 bytes per slot in LDS, above in HBM
constexpr int kLaneMaxW = 64;      // wmax: the 2 * wmax children of a level are scored in rounds of 64 slots
constexpr int kLaneMaxNb = 64;     // nb_window * nb_store neighbour entries, one per slot
constexpr int kLaneDQ = 16;        // dimensions of a row held by one lane
constexpr int kLaneSlots = 64;     // slots of a workgroup
constexpr int kLtGroups = 16;      // groups side by side in a 64-slot window (the smallest group has 4 slots)

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

// canon_dot's value for two D-vectors held by the Q lanes of a slot, 16 dimensions each (fa(i), fb(i) give
// element i of this lane's dimensions [16 q, 16 q + 16)): each lane reduces its 16 / Q whole groups of D / 16
// products by the halving tree, then the halving tree over the 16 groups runs as an xor butterfly in which a
// step pairs groups held by different lanes of the slot.  Every lane of the slot ends with the value.
template <int N, int GQ>
__device__ __forceinline__ void lt_groups_step(float (&g)[GQ]) {
  if constexpr (N >= GQ) {
#pragma unroll
    for (int i = 0; i < GQ; ++i) g[i] = g[i] + xor_lane<N / GQ>(g[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) g[i] = g[i] + g[i + N];
  }
}
template <int D, int Q, typename FA, typename FB>
__device__ __forceinline__ float slice_dot(FA fa, FB fb) {
  static_assert(D % 16 == 0 && Q * kLaneDQ == D, "16 dimensions per lane");
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
  lt_groups_step<8, GQ>(g);
  lt_groups_step<4, GQ>(g);
  lt_groups_step<2, GQ>(g);
  lt_groups_step<1, GQ>(g);
  return g[0];
}

// Integer sum over the Q lanes of a slot.
template <int Q>
__device__ __forceinline__ int slot_isum(int v) {
  if constexpr (Q >= 2) v += xor_lane<1>(v);
  if constexpr (Q >= 4) v += xor_lane<2>(v);
  if constexpr (Q >= 8) v += xor_lane<4>(v);
  return v;
}

// In-wavefront part of a reduction over the L slots of an aligned group of slots, every lane of a slot holding
// the slot's value (span = min(L * Q, 64) lanes): xor butterflies over the slot bits.  The operations used are
// exact whatever the order: integer counts held as floats, min / max, and the argmax (the largest value, the
// smallest index among equals).
template <int Q, typename V, typename Op>
__device__ __forceinline__ V wave_grp(V v, int span, Op op) {
  if constexpr (Q <= 1) {
    if (1 < span) v = op(v, xor_lane<1>(v));
  }
  if constexpr (Q <= 2) {
    if (2 < span) v = op(v, xor_lane<2>(v));
  }
  if constexpr (Q <= 4) {
    if (4 < span) v = op(v, xor_lane<4>(v));
  }
  if constexpr (Q <= 8) {
    if (8 < span) v = op(v, xor_lane<8>(v));
  }
  if (16 < span) v = op(v, xor_lane<16>(v));
  if (32 < span) v = op(v, xor_lane<32>(v));
  return v;
}
template <int H>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  const float ov = xor_lane<H>(v);
  const int oi = xor_lane<H>(i);
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}
template <int Q>
__device__ __forceinline__ void wave_grp_argmax(float& v, int& i, int span) {
  if constexpr (Q <= 1) {
    if (1 < span) argmax_step<1>(v, i);
  }
  if constexpr (Q <= 2) {
    if (2 < span) argmax_step<2>(v, i);
  }
  if constexpr (Q <= 4) {
    if (4 < span) argmax_step<4>(v, i);
  }
  if constexpr (Q <= 8) {
    if (8 < span) argmax_step<8>(v, i);
  }
  if (16 < span) argmax_step<16>(v, i);
  if (32 < span) argmax_step<32>(v, i);
}

// Cross-wavefront words (8 per wavefront) in two LDS buffers used in turn: a buffer is written again only after
// every thread has passed the barrier of the exchange in between, so one workgroup barrier per exchange
// suffices.  Every thread makes the same sequence of exchanges.
struct LtXchg {
  int* buf;   // [2][8 wavefronts][8]
  int sel;
  __device__ __forceinline__ int* next() {
    int* b = buf + sel * 64;
    sel ^= 1;
    return b;
  }
};

// Sort key of a projection: ascending float order (-0 taken as +0, as the comparison does).  With the member
// index as the second key, sorting is the stable sort of the projections.
__device__ __forceinline__ uint32_t lt_sort_key(float p) {
  const uint32_t u = __float_as_uint(p + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Ascending bitonic sort of the pairs (key[i], idx[i]), i < n2 (a power of two; the indices unique), by the
// whole workgroup.
template <typename IW>
__device__ __forceinline__ void lt_bitonic_sort(uint32_t* key, IW* idx, int n2, int tid, int nt) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < (n2 >> 1); i += nt) {
        const int a = ((i & ~(j - 1)) << 1) | (i & (j - 1)), b = a + j;
        const uint32_t ka = key[a], kb = key[b];
        const IW ia = idx[a], ib = idx[b];
        const bool gt = ka > kb || (ka == kb && ia > ib);
        if (gt == ((a & k) == 0)) {
          key[a] = kb;
          key[b] = ka;
          idx[a] = ib;
          idx[b] = ia;
        }
      }
      __syncthreads();
    }
  }
}

// The same sort with the pairs in registers: n2 = E * (workgroup size), thread t holding entries [t E, t E + E) as
// (key << 32 | index).  Each step of the network exchanges within a thread (distance below E), between lanes of
// a wavefront (below 64 E) or through the LDS arrays (the rest, a few steps); the arrays hold the sorted pairs
// at the end.
template <int J, int E>
__device__ __forceinline__ void lt_reg_step(uint64_t (&v)[E], int k, int i0) {
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if ((e & J) == 0) {
      const bool asc = ((i0 + e) & k) == 0;
      const uint64_t a = v[e], b = v[e | J];
      const bool sw = (a > b) == asc;
      v[e] = sw ? b : a;
      v[e | J] = sw ? a : b;
    }
  }
}
template <int E, typename IW>
__device__ __forceinline__ void lt_bitonic_sort_reg(uint32_t* key, IW* idx, int tid, int nt) {
  static_assert(E >= 2 && E <= 16 && (E & (E - 1)) == 0, "2 to 16 pairs per thread");
  const int n2 = E * nt, i0 = tid * E;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = ((uint64_t)key[i0 + e] << 32) | (uint32_t)idx[i0 + e];
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < E) {
        switch (j) {
          case 1: lt_reg_step<1, E>(v, k, i0); break;
          case 2: if constexpr (E > 2) lt_reg_step<2, E>(v, k, i0); break;
          case 4: if constexpr (E > 4) lt_reg_step<4, E>(v, k, i0); break;
          default: if constexpr (E > 8) lt_reg_step<8, E>(v, k, i0); break;
        }
      } else if (j < E * kWave) {
        const int m = j / E;
        const bool lower = (tid & m) == 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int hi = __shfl_xor((int)(v[e] >> 32), m, kWave), lo = __shfl_xor((int)(uint32_t)v[e], m, kWave);
          const uint64_t o = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
          const bool keepmin = lower == (((i0 + e) & k) == 0);
          v[e] = keepmin ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          key[i0 + e] = (uint32_t)(v[e] >> 32);
          idx[i0 + e] = (IW)(uint32_t)v[e];
        }
        __syncthreads();
        const bool lower = (i0 & j) == 0;   // j >= 64 E: the same for the thread's E entries
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int pi = (i0 + e) ^ j;
          const uint64_t o = ((uint64_t)key[pi] << 32) | (uint32_t)idx[pi];
          const bool keepmin = lower == (((i0 + e) & k) == 0);
          v[e] = keepmin ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
        }
        __syncthreads();
      }
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    key[i0 + e] = (uint32_t)(v[e] >> 32);
    idx[i0 + e] = (IW)(uint32_t)v[e];
  }
  __syncthreads();
}

// Canonical sums of the groups of L consecutive slots (64 / L groups, L in {4, ..., 64}), for NSET sets of slot
// rows at once.  Each slot writes its partial (lt_group_row: this lane's 16 dimensions) into its row of a set
// (64 rows of stride D + 4), and the group's member count is left in gc as nseg partial counts per group (set s,
// group g at gc[16 s + nseg g + j], integers); lt_group_reduce then reduces every (set, group, dimension) in one
// thread: the halving tree over the group's L partials, divided by max(count, 1).  The value goes to dst + set *
// 16 (D + 4) + group (D + 4) + dimension when the count is positive or `always`.  All reads are issued before
// the first store.  MASK: the sets share one set of rows (zero where the slot holds no key), set s taking a slot's
// row where its label byte (lab, 64 of them) is s + 1 and zero elsewhere -- the values the separate rows held.
__device__ __forceinline__ void lt_group_row(const float (&v)[kLaneDQ], bool take, float* row) {
#pragma unroll
  for (int d = 0; d < kLaneDQ; d += 4)
    *reinterpret_cast<float4*>(row + d) = take ? make_float4(v[d], v[d + 1], v[d + 2], v[d + 3])
                                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}
template <int L>
__device__ __forceinline__ void lt_label_mask(float (&p)[L], const uint8_t* lab, int g, int set) {
#pragma unroll
  for (int j4 = 0; j4 < L; j4 += 4) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(lab)[(g * L + j4) >> 2];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (((w >> (8 * b)) & 0xffu) != (uint32_t)(set + 1)) p[j4 + b] = 0.0f;
  }
}
template <int D, int L, int NT, int NSET, bool MASK = false, int GC = kLtGroups, int GB = kLtGroups>
__device__ __forceinline__ void lt_group_outputs(const float* red, const float* gc, int nseg, bool always, float* dst,
                                                 int tid, const uint8_t* lab = nullptr) {
  constexpr int RS = D + 4, nout1 = (kLaneSlots / L) * D, nout = NSET * nout1, NU = (nout + NT - 1) / NT;
  float p[NU][L], c[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int o = tid + NT * u, set = o / nout1, r = o - set * nout1, g = r / D, d = r - g * D;
    const bool in = o < nout;
    const float* base = red + ((MASK ? 0 : set * kLaneSlots) + g * L) * RS;
#pragma unroll
    for (int j = 0; j < L; ++j) p[u][j] = in ? base[j * RS + d] : 0.0f;
    if constexpr (MASK) lt_label_mask<L>(p[u], lab, g, set);
    float cs = 0.0f;
    for (int j = 0; j < nseg; ++j) cs = cs + (in ? gc[set * GC + g * nseg + j] : 0.0f);
    c[u] = cs;
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
    const int o = tid + NT * u, set = o / nout1, r = o - set * nout1, g = r / D, d = r - g * D;
    if (o < nout && (always || c[u] > 0.0f)) dst[(set * GB + g) * RS + d] = p[u][0];
  }
}
// LMIN: the smallest group width L the caller passes (narrower widths are not compiled in); GC and GB: the strides
// between the sets' counts (in counts) and between their banks (in rows).
template <int D, int NT, int NSET, bool MASK = false, int LMIN = 4, int GC = kLtGroups, int GB = kLtGroups>
__device__ __forceinline__ void lt_group_reduce(const float* red, const float* gc, int nseg, int L, bool always,
                                                float* dst, int tid, const uint8_t* lab = nullptr) {
  __syncthreads();
  switch (L) {
    case 4: if constexpr (LMIN <= 4) lt_group_outputs<D, 4, NT, NSET, MASK>(red, gc, nseg, always, dst, tid, lab); break;
    case 8: if constexpr (LMIN <= 8) lt_group_outputs<D, 8, NT, NSET, MASK>(red, gc, nseg, always, dst, tid, lab); break;
    case 16:
      if constexpr (LMIN <= 16) lt_group_outputs<D, 16, NT, NSET, MASK>(red, gc, nseg, always, dst, tid, lab);
      break;
    case 32:
      if constexpr (LMIN <= 32) lt_group_outputs<D, 32, NT, NSET, MASK>(red, gc, nseg, always, dst, tid, lab);
      break;
    default: lt_group_outputs<D, 64, NT, NSET, MASK, GC, GB>(red, gc, nseg, always, dst, tid, lab); break;
  }
  __syncthreads();
}

// lt_group_reduce for groups that lie inside one wavefront (L * Q <= 64): the wavefront reduces the outputs of
// its own groups (64 / (Q L) of them, from group wave * 64 / (Q L) on), between wavefront barriers.
template <int D, int Q, int L, int NSET, bool MASK = false>
__device__ __forceinline__ void lt_group_outputs_w(const float* red, const float* gc, bool always, float* dst, int lane,
                                                   int wv, const uint8_t* lab) {
  if constexpr (L * Q <= kWave) {
    constexpr int RS = D + 4, gpw = kWave / (Q * L), nout1 = gpw * D, nout = NSET * nout1;
    constexpr int NU = (nout + kWave - 1) / kWave;
    float p[NU][L], c[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int o = lane + kWave * u, set = o / nout1, r = o - set * nout1, gg = wv * gpw + r / D, d = r % D;
      const bool in = o < nout;
      const float* base = red + ((MASK ? 0 : set * kLaneSlots) + gg * L) * RS;
#pragma unroll
      for (int j = 0; j < L; ++j) p[u][j] = in ? base[j * RS + d] : 0.0f;
      if constexpr (MASK) lt_label_mask<L>(p[u], lab, gg, set);
      c[u] = in ? gc[set * kLtGroups + gg] : 0.0f;
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
      const int o = lane + kWave * u, set = o / nout1, r = o - set * nout1, gg = wv * gpw + r / D, d = r % D;
      if (o < nout && (always || c[u] > 0.0f)) dst[(set * kLtGroups + gg) * RS + d] = p[u][0];
    }
  }
}
template <int D, int Q, int NSET, bool MASK = false>
__device__ __forceinline__ void lt_group_reduce_w(const float* red, const float* gc, int L, bool always, float* dst,
                                                  int lane, int wv, const uint8_t* lab = nullptr) {
  wave_sync();
  switch (L) {
    case 4: lt_group_outputs_w<D, Q, 4, NSET, MASK>(red, gc, always, dst, lane, wv, lab); break;
    case 8: lt_group_outputs_w<D, Q, 8, NSET, MASK>(red, gc, always, dst, lane, wv, lab); break;
    case 16: lt_group_outputs_w<D, Q, 16, NSET, MASK>(red, gc, always, dst, lane, wv, lab); break;
    case 32: lt_group_outputs_w<D, Q, 32, NSET, MASK>(red, gc, always, dst, lane, wv, lab); break;
    default: lt_group_outputs_w<D, Q, 64, NSET, MASK>(red, gc, always, dst, lane, wv, lab); break;
  }
  wave_sync();
}

// The split launch's LDS (one group of S slots): the row area (two sets of 64 slot rows: the mean's partials, then
// the two Lloyd clusters' partials, the first in the mean's set once the mean is reduced; or the group's sort keys
// and indices, 6 bytes per slot), the group's slots as 16-bit words (key position, bit 15 set when the slot holds
// a real key), the group's three centroids (the mean, c0, c1), the cross-wavefront words and the counts (the
// mean's, then a partial per wavefront for each cluster).  Above kLaneLdsMaxT slots (BIG) the slot words (32-bit:
// bit 31 the real-key bit) stay in the tree's slot array and the sort keys and indices (4 + 4 bytes per slot) go
// to the group's part of the node-sum area ([2 g S, 2 g S + 2 S) for group g), both in HBM and unused until the
// tail writes the node sums; the LDS then holds the rest only.
__host__ __device__ constexpr int lt_rows_bytes(int C, int D, bool big) {
  return !big && 6 * C > 2 * kLaneSlots * (D + 4) * 4 ? ((6 * C + 15) & ~15) : 2 * kLaneSlots * (D + 4) * 4;
}
__host__ __device__ constexpr int lt_build_lds_bytes(int C, int D, bool big) {
  return lt_rows_bytes(C, D, big) + (big ? 0 : ((2 * C + 15) & ~15)) + 3 * (D + 4) * 4 + 2 * 64 * 4 + 3 * 8 * 4;
}

// ---------------------------------------------------------------------------------------------------- build
// The lane trees (dyntree.py:34-82) in three launches.  Every level splits each group of S = C >> lvl slots of a
// tree by a masked 2-means projection; the group's real keys are then laid out half and half (the larger half
// first), empty slots after each half's keys, every empty slot holding the position of the group's last empty
// slot (the one the stable sort ranks last).  Empty slots add key * 0 to the masked sums; they are skipped, which
// changes at most the sign of a zero.
//
// lanetree_split_kernel, one launch per level whose groups hold more than 64 slots and one workgroup per group
// (the groups of a level touch disjoint slots): workgroup slot j holds members j, j + 64, j + 128, ... (partial j
// of the canonical sums, their rows requested U at a time); the order by a bitonic sort of (projection, index)
// over the span of the group's real keys (its pairs in registers, 2 to 16 per thread, when the span fits).  The
// slot words (key position, bit 31 set for a real key) go from the tree's slot array into LDS and back; level 0
// starts them (key j in slot j, real for 1 <= j < the lane's start).
// (Four wavefronts per SIMD requested at D = 128 and for large trees at D = 64, for a few spilled registers: two
// groups per CU at D = 128; measured faster there, slightly slower for D = 64 below kLaneLdsMaxT.)
template <typename T, int D, int Q, bool BIG>
__global__ __launch_bounds__(kWave * Q) __attribute__((amdgpu_waves_per_eu(Q >= 8 || (BIG && Q >= 4) ? 4 : 1, 8)))
void lanetree_split_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                                                   int64_t kst, int H, int C, int nlane, int chunk,
                                                                   int iters, float* __restrict__ ws, int64_t P,
                                                                   int lvl) {
  constexpr int RS = D + 4, DQ = kLaneDQ, NT = kWave * Q, U = Q >= 8 ? 2 : 4;   // U: member rows requested at a time
  using SW = std::conditional_t<BIG, uint32_t, uint16_t>;   // slot words and sort indices
  constexpr uint32_t VBIT = BIG ? 0x80000000u : 0x8000u;     // the slot holds a real key
  extern __shared__ __align__(16) unsigned char s_raw[];
  const int S = C >> lvl, half = S >> 1, M = S / kLaneSlots;
  const int64_t pt = blockIdx.x >> lvl;
  const int gb0 = (int)(blockIdx.x - (pt << lvl)) * S;   // the group's first slot
  const LaneTree tr = lane_tree(ws, P, C, D, pt);
  const int rowsb = lt_rows_bytes(S, D, BIG);
  float* s_rows = reinterpret_cast<float*>(s_raw);                                    // [2][64][RS]
  uint32_t* s_sk = BIG ? reinterpret_cast<uint32_t*>(tr.sums + 2 * gb0) : reinterpret_cast<uint32_t*>(s_raw);   // [S]
  SW* s_si = BIG ? reinterpret_cast<SW*>(tr.sums + 2 * gb0 + S) : reinterpret_cast<SW*>(s_raw + 4 * S);         // [S]
  SW* s_pv = BIG ? reinterpret_cast<SW*>(tr.slot + gb0) : reinterpret_cast<SW*>(s_raw + rowsb);                 // [S]
  float* s_cen = reinterpret_cast<float*>(s_raw + rowsb + (BIG ? 0 : ((2 * S + 15) & ~15)));   // [3][RS]
  LtXchg xw{reinterpret_cast<int*>(s_cen + 3 * RS), 0};
  float* s_gc = s_cen + 3 * RS + 2 * 64;   // [3][8] counts: the mean's, then the two clusters' partials
  const int tid = threadIdx.x, m = tid / Q, q = tid % Q, d0 = q * DQ, wv = wave_id();
  const int ln = (int)(pt % nlane);
  const int64_t bh = pt / nlane;
  const T* kb = k + (bh / H) * ksb + (bh % H) * ksh + d0;
  const int n0 = ln * chunk;
  const float kInf = __int_as_float(0x7f800000);
  auto perm = [&](int s) { return (int)(s_pv[s] & (VBIT - 1)); };
  auto val = [&](int s) { return (s_pv[s] & VBIT) != 0; };
  auto fadd = [](float a, float b) { return a + b; };
  auto imin = [](int a, int b) { return min(a, b); };
  auto imax = [](int a, int b) { return max(a, b); };
  if (lvl == 0) {
    for (int c = tid; c < C; c += NT) s_pv[c] = (SW)((uint32_t)c | ((c >= 1 && c < n0) ? VBIT : 0u));
  } else if constexpr (!BIG) {
    for (int c = tid; c < S; c += NT) {
      const uint32_t w = (uint32_t)tr.slot[gb0 + c];
      s_pv[c] = (SW)((w & 0x7fffffffu) | ((w & 0x80000000u) ? VBIT : 0u));
    }
  }
  __syncthreads();
  float* meanp = s_cen + d0;   // the group's mean, c0 and c1 (this lane's part)
  float* c0b = s_cen + RS + d0;
  float* c1b = s_cen + 2 * RS + d0;
  float* rowA = s_rows + m * RS;   // this slot's rows: the mean's or the first cluster's (A), the second's (B)
  float* rowB = rowA + kLaneSlots * RS;
  float acc0[DQ], acc1[DQ];
  if (S > kLaneSlots) {   // (a tree of at most 64 slots only has its slot words started here)
    {
      constexpr int gb = 0;   // slot indices below are the group's
      auto scan = [&](auto&& f) __attribute__((always_inline)) {
        for (int t0 = 0; t0 < M; t0 += U) {
          float xb[U][DQ];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int t = t0 + u < M ? t0 + u : M - 1;
            load_row_g<T, DQ>(kb + (int64_t)perm(gb + m + kLaneSlots * t) * kst, xb[u]);
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (t0 + u < M) f(m + kLaneSlots * (t0 + u), xb[u]);
        }
      };
      // (1) counts and the masked mean
      float cntp = 0.0f;
      int vlo = S, vhi = -1, lastinv = -1;
#pragma unroll
      for (int d = 0; d < DQ; ++d) acc0[d] = 0.0f;
      scan([&](int i, const float(&r)[DQ]) {
        if (val(gb + i)) {
#pragma unroll
          for (int d = 0; d < DQ; ++d) acc0[d] = acc0[d] + r[d];
          cntp = cntp + 1.0f;
          vlo = min(vlo, i);
          vhi = max(vhi, i);
        } else {
          lastinv = i;
        }
      });
      float cnt = wave_grp<Q>(cntp, kWave, fadd);
      vlo = wave_grp<Q>(vlo, kWave, imin);
      vhi = wave_grp<Q>(vhi, kWave, imax);
      lastinv = wave_grp<Q>(lastinv, kWave, imax);
      bool work = __ballot(cntp > 0.0f) != 0;
      if constexpr (Q > 1) {   // the group's statistics across the wavefronts
        int* xb = xw.next();
        if (lane_id() == 0) {
          int* e = xb + wv * 8;
          e[0] = __float_as_int(cnt);
          e[1] = vlo;
          e[2] = vhi;
          e[3] = lastinv;
          e[4] = work ? 1 : 0;
        }
        __syncthreads();
        cnt = 0.0f;
        vlo = S;
        vhi = -1;
        lastinv = -1;
        work = false;
        for (int j = 0; j < Q; ++j) {
          const int* e = xb + j * 8;
          cnt = cnt + __int_as_float(e[0]);
          vlo = min(vlo, e[1]);
          vhi = max(vhi, e[2]);
          lastinv = max(lastinv, e[3]);
          work = work || e[4] != 0;
        }
      }
      const int ng = (int)cnt;
      // the group argmax of (value, member index)
      auto argmax_grp = [&](float v, int i) {
        wave_grp_argmax<Q>(v, i, kWave);
        if constexpr (Q > 1) {
          int* xb = xw.next();
          if (lane_id() == 0) {
            xb[wv * 8] = __float_as_int(v);
            xb[wv * 8 + 1] = i;
          }
          __syncthreads();
          v = __int_as_float(xb[0]);
          i = xb[1];
          for (int j = 1; j < Q; ++j) {
            const float ov = __int_as_float(xb[j * 8]);
            const int oi = xb[j * 8 + 1];
            if (ov > v || (ov == v && oi < i)) {
              v = ov;
              i = oi;
            }
          }
        }
        return i;
      };
      if (work) {
        lt_group_row(acc0, true, rowA + d0);
        if (m == 0 && q == 0) s_gc[0] = cnt;
        lt_group_reduce<D, NT, 1, false, kLaneSlots, 8, 1>(s_rows, s_gc, 1, kLaneSlots, true, s_cen, tid);   // the mean
        // a = the real key farthest from the mean, then b = the real key farthest from a (into the banks)
        for (int pass = 0; pass < 2; ++pass) {
          const float* ref = pass == 0 ? meanp : c0b;
          float bv = -1.0f;
          int bi = 0;
          scan([&](int i, const float(&r)[DQ]) {
            if (!val(gb + i)) return;
            const float d2 =
                slice_dot<D, Q>([&](int e) { return r[e] - ref[e]; }, [&](int e) { return r[e] - ref[e]; });
            if (d2 > bv) {
              bv = d2;
              bi = i;
            }
          });
          const int sel = argmax_grp(bv, bi);
          float* bank = pass == 0 ? c0b : c1b;
          load_row_g<T, DQ>(kb + (int64_t)perm(gb + sel) * kst, acc1);
#pragma unroll
          for (int d = 0; d < DQ; d += 4)
            *reinterpret_cast<float4*>(bank + d) = make_float4(acc1[d], acc1[d + 1], acc1[d + 2], acc1[d + 3]);
          __syncthreads();
        }
        // Lloyd iterations: labels from the current centroids, then both masked sums, in one pass and one
        // reduction (sets B and C into the banks c0 and c1; an empty cluster keeps its centroid)
        for (int it = 0; it < iters; ++it) {
          const float cc0 = slice_dot<D, Q>([&](int e) { return c0b[e]; }, [&](int e) { return c0b[e]; });
          const float cc1 = slice_dot<D, Q>([&](int e) { return c1b[e]; }, [&](int e) { return c1b[e]; });
          float cp0 = 0.0f, cp1 = 0.0f;
#pragma unroll
          for (int d = 0; d < DQ; ++d) {
            acc0[d] = 0.0f;
            acc1[d] = 0.0f;
          }
          scan([&](int i, const float(&r)[DQ]) {
            if (!val(gb + i)) return;
            const float xx = slice_dot<D, Q>([&](int e) { return r[e]; }, [&](int e) { return r[e]; });
            const float xc0 = slice_dot<D, Q>([&](int e) { return r[e]; }, [&](int e) { return c0b[e]; });
            const float xc1 = slice_dot<D, Q>([&](int e) { return r[e]; }, [&](int e) { return c1b[e]; });
            const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
            if (dist1 < dist0) {
#pragma unroll
              for (int d = 0; d < DQ; ++d) acc1[d] = acc1[d] + r[d];
              cp1 = cp1 + 1.0f;
            } else {
#pragma unroll
              for (int d = 0; d < DQ; ++d) acc0[d] = acc0[d] + r[d];
              cp0 = cp0 + 1.0f;
            }
          });
          lt_group_row(acc0, true, rowA + d0);
          lt_group_row(acc1, true, rowB + d0);
          // the clusters' counts: a partial per wavefront
          const float w0 = wave_grp<Q>(cp0, kWave, fadd), w1 = wave_grp<Q>(cp1, kWave, fadd);
          if (lane_id() == 0) {
            s_gc[8 + wv] = w0;
            s_gc[16 + wv] = w1;
          }
          lt_group_reduce<D, NT, 2, false, kLaneSlots, 8, 1>(s_rows, s_gc + 8, Q, kLaneSlots, false, s_cen + RS,
                                                              tid);
        }
      }
      const int nl = (ng + 1) / 2, nr = ng - nl;
      // projections on c0 - c1 over the span of the real keys (empty slots inside it: +inf), padded to a power
      // of two with entries that sort last; bitonic sort
      if (ng > 0) {
        const int n = vhi - vlo + 1;
        int n2 = 1;
        while (n2 < n) n2 <<= 1;
        scan([&](int i, const float(&r)[DQ]) {
          if (i < vlo || i > vhi) return;
          float pr = kInf;
          if (val(gb + i))
            pr = slice_dot<D, Q>([&](int e) { return r[e]; }, [&](int e) { return c0b[e] - c1b[e]; });
          if (q == 0) {
            s_sk[i - vlo] = lt_sort_key(pr);
            s_si[i - vlo] = (SW)(i - vlo);
          }
        });
        for (int r = n + tid; r < n2; r += NT) {
          s_sk[r] = lt_sort_key(kInf);
          s_si[r] = (SW)r;
        }
        __syncthreads();
        if constexpr (!BIG) {   // the pairs in registers, 2 to 16 per thread
          switch (n2 / NT) {
            case 2: lt_bitonic_sort_reg<2>(s_sk, s_si, tid, NT); break;
            case 4: lt_bitonic_sort_reg<4>(s_sk, s_si, tid, NT); break;
            case 8: lt_bitonic_sort_reg<8>(s_sk, s_si, tid, NT); break;
            case 16: lt_bitonic_sort_reg<16>(s_sk, s_si, tid, NT); break;
            default: lt_bitonic_sort(s_sk, s_si, n2, tid, NT); break;
          }
        } else {
          lt_bitonic_sort(s_sk, s_si, n2, tid, NT);
        }
      }
      // layout: sorted ranks [0, nl) to the left half, [nl, ng) to the right half (phase A rewrites each entry as
      // (position, key position) -- one 32-bit word, or the index and key words when BIG -- before phase B moves
      // the slots)
      for (int r = tid; r < ng; r += NT) {
        const int mm = vlo + (int)s_si[r];
        const int pos = r < nl ? r : half + r - nl;
        if constexpr (BIG) {
          s_si[r] = (SW)pos;
          s_sk[r] = (uint32_t)perm(gb + mm);
        } else {
          s_sk[r] = ((uint32_t)pos << 16) | (uint32_t)perm(gb + mm);
        }
      }
      const int fillp = lastinv >= 0 ? perm(gb + lastinv) : 0;
      __syncthreads();
      for (int r = tid; r < ng; r += NT) {
        const uint32_t e = s_sk[r];
        if constexpr (BIG) s_pv[gb + (int)s_si[r]] = (SW)(e | VBIT);
        else s_pv[gb + (int)(e >> 16)] = (SW)((e & 0xffffu) | VBIT);
      }
      for (int pp = tid; pp < S; pp += NT) {
        const bool filled = pp < half ? pp < nl : (pp - half) < nr;
        if (!filled) s_pv[gb + pp] = (SW)fillp;
      }
      __syncthreads();
    }
  }
  if constexpr (!BIG) {
    for (int c = tid; c < S; c += NT)
      tr.slot[gb0 + c] = (int32_t)((uint32_t)perm(c) | (val(c) ? 0x80000000u : 0u));
  }
}

// lanetree_tail_kernel, one workgroup per (tree, window of 64 slots): the levels whose groups hold at most 64
// slots.  From the first of them on a window's keys stay inside it, so windows are independent and the launch
// has C / 64 workgroups per tree.  Slot j holds one member, its key row in registers and (zero where the slot
// holds no key) in LDS, the Lloyd clusters marked by a label byte per slot; groups of S < 64 slots sit side by
// side, the two farthest members are read from the slot rows, and the order comes from ranks by counting.
// Then the window's node sums and counts (its leaves and the nodes above them up to the window's root) and its
// final slots (key position, or -1).
// (Four wavefronts per SIMD requested for D >= 64: more windows resident per CU, which the window's chain of LDS
// round trips needs, for a few spilled registers; measured faster than three at D = 128 and at T >= 2048 for
// D = 64.)
template <typename T, int D, int Q>
__global__ __launch_bounds__(kWave * Q) __attribute__((amdgpu_waves_per_eu(Q >= 4 ? 4 : 1, 8))) void lanetree_tail_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                                                  int64_t kst, int H, int C, int nlane, int iters,
                                                                  float* __restrict__ ws, int64_t P) {
  constexpr int RS = D + 4, DQ = kLaneDQ, NT = kWave * Q;
  constexpr uint32_t VB = 0x80000000u;
  __shared__ __align__(16) float s_x[kLaneSlots * RS];          // slot rows; the window's node rows at the end
  __shared__ __align__(16) float s_cen[3 * kLtGroups * RS];     // banks: the groups' means, c0, c1
  __shared__ float s_key[kLaneSlots];                           // rank keys
  __shared__ uint32_t s_pv[kLaneSlots];                         // slot words
  __shared__ __align__(4) uint8_t s_lab[kLaneSlots];            // cluster labels (1: c0, 2: c1, 0: no key)
  __shared__ int s_xwb[2 * 64];
  __shared__ float s_gc[3 * kLtGroups];
  __shared__ int s_nc[kLaneSlots];                              // the window's node counts
  const int tid = threadIdx.x, m = tid / Q, q = tid % Q, d0 = q * DQ, wv = wave_id();
  const int nw = C > kLaneSlots ? C / kLaneSlots : 1;
  const int64_t pt = blockIdx.x / nw;
  const int win = (int)(blockIdx.x - pt * nw);
  const int W = C < kLaneSlots ? C : kLaneSlots, base = win * kLaneSlots;
  const int64_t bh = pt / nlane;
  const T* kb = k + (bh / H) * ksb + (bh % H) * ksh + d0;
  const LaneTree tr = lane_tree(ws, P, C, D, pt);
  const bool live = m < W;   // C < 64: slots past the tree sit out
  const float kInf = __int_as_float(0x7f800000);
  TA_DMARK(0);   // phase marks (trace.hpp): 0 start; level k (from the first): 1 + 3k statistics exchanged,
                 // 2 + 3k Lloyd iterations done, 3 + 3k laid out
  if (tid < W) s_pv[tid] = (uint32_t)tr.slot[base + tid];
  LtXchg xw{s_xwb, 0};
  [[maybe_unused]] int mk = 0;   // the level's first mark
  auto perm = [&](int s) { return (int)(s_pv[s] & (VB - 1)); };
  auto val = [&](int s) { return (s_pv[s] & VB) != 0; };
  auto fadd = [](float a, float b) { return a + b; };
  auto imin = [](int a, int b) { return min(a, b); };
  auto imax = [](int a, int b) { return max(a, b); };
  const int nlev = lt_log2(C) - 1;
  float* rowx = s_x + m * RS + d0;
  auto level = [&](auto loc, int S, const float(&x)[DQ]) __attribute__((always_inline)) {
    constexpr bool local = decltype(loc)::value;   // every group inside one wavefront: wavefront barriers
    auto sync = [&]() {
      if constexpr (local) wave_sync();
      else __syncthreads();
    };
    const int half = S >> 1, L = S, g = m / L, gl = m & (L - 1), span = L * Q < kWave ? L * Q : kWave;
    float* meanp = s_cen + g * RS + d0;
    float* c0b = s_cen + (kLtGroups + g) * RS + d0;
    float* c1b = s_cen + (2 * kLtGroups + g) * RS + d0;
    // (1) counts
    float cntp = 0.0f;
    int vlo = S, vhi = -1, lastinv = -1;
    if (live) {
      if (val(m)) {
        cntp = 1.0f;
        vlo = vhi = gl;
      } else {
        lastinv = gl;
      }
    }
    float cnt = wave_grp<Q>(cntp, span, fadd);
    vlo = wave_grp<Q>(vlo, span, imin);
    vhi = wave_grp<Q>(vhi, span, imax);
    lastinv = wave_grp<Q>(lastinv, span, imax);
    bool work = __ballot(cntp > 0.0f) != 0;
    if constexpr (Q > 1 && !local) {   // the group's statistics across wavefronts, and whether any group has keys
      int* xb = xw.next();
      if (lane_id() == 0) {
        int* e = xb + wv * 8;
        e[0] = __float_as_int(cnt);
        e[1] = vlo;
        e[2] = vhi;
        e[3] = lastinv;
        e[4] = work ? 1 : 0;
      }
      __syncthreads();
      if (L * Q > kWave) {
        const int nwv = L * Q / kWave, w0 = wv & ~(nwv - 1);
        cnt = 0.0f;
        vlo = S;
        vhi = -1;
        lastinv = -1;
        for (int j = 0; j < nwv; ++j) {
          const int* e = xb + (w0 + j) * 8;
          cnt = cnt + __int_as_float(e[0]);
          vlo = min(vlo, e[1]);
          vhi = max(vhi, e[2]);
          lastinv = max(lastinv, e[3]);
        }
      }
      work = false;
      for (int j = 0; j < Q; ++j) work = work || xb[j * 8 + 4] != 0;
    }
    if (mk < 16) TA_DMARK(mk);
    const int ng = (int)cnt;
    // the group argmax of (value, member index)
    auto argmax_grp = [&](float v, int i) {
      wave_grp_argmax<Q>(v, i, span);
      if (L * Q > kWave) {
        int* xb = xw.next();
        if (lane_id() == 0) {
          xb[wv * 8] = __float_as_int(v);
          xb[wv * 8 + 1] = i;
        }
        __syncthreads();
        const int nwv = L * Q / kWave, w0 = wv & ~(nwv - 1);
        v = __int_as_float(xb[w0 * 8]);
        i = xb[w0 * 8 + 1];
        for (int j = 1; j < nwv; ++j) {
          const float ov = __int_as_float(xb[(w0 + j) * 8]);
          const int oi = xb[(w0 + j) * 8 + 1];
          if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
          }
        }
      }
      return i;
    };
    if (work) {
      lt_group_row(x, cntp > 0.0f, rowx);
      if (gl == 0 && q == 0) s_gc[g] = cnt;
      if constexpr (local) lt_group_reduce_w<D, Q, 1>(s_x, s_gc, L, true, s_cen, lane_id(), wv);   // the means
      else lt_group_reduce<D, NT, 1, false, 2 * kWave / Q>(s_x, s_gc, 1, L, true, s_cen, tid);
      // a = the real key farthest from the mean, then b = the real key farthest from a: their slot rows, copied
      // into the centroid banks, which the Lloyd outputs keep for an empty cluster and the projection reads
      const float* pa = c0b;
      const float* pb = c1b;
      for (int pass = 0; pass < 2; ++pass) {
        const float* ref = pass == 0 ? meanp : pa;
        float bv = -1.0f;
        int bi = 0;
        if (live && cntp > 0.0f) {
          bv = slice_dot<D, Q>([&](int e) { return x[e] - ref[e]; }, [&](int e) { return x[e] - ref[e]; });
          bi = gl;
        }
        const int sel = argmax_grp(bv, bi);
        float* bank = pass == 0 ? c0b : c1b;
        const float* src = s_x + (g * L + sel) * RS + d0;
        if (pass == 0) pa = src;
        else pb = src;
        if (live) {
#pragma unroll
          for (int d = 0; d < DQ; d += 4)
            *reinterpret_cast<float4*>(bank + d) = *reinterpret_cast<const float4*>(src + d);
        }
      }
      // Lloyd iterations: labels from the current centroids, then both clusters' sums in one reduction (into the
      // banks c0 and c1; an empty cluster keeps its centroid)
      for (int it = 0; it < iters; ++it) {
        const float* r0 = it == 0 ? pa : c0b;
        const float* r1 = it == 0 ? pb : c1b;
        const float cc0 = slice_dot<D, Q>([&](int e) { return r0[e]; }, [&](int e) { return r0[e]; });
        const float cc1 = slice_dot<D, Q>([&](int e) { return r1[e]; }, [&](int e) { return r1[e]; });
        float cp0 = 0.0f, cp1 = 0.0f;
        if (live && cntp > 0.0f) {
          const float xx = slice_dot<D, Q>([&](int e) { return x[e]; }, [&](int e) { return x[e]; });
          const float xc0 = slice_dot<D, Q>([&](int e) { return x[e]; }, [&](int e) { return r0[e]; });
          const float xc1 = slice_dot<D, Q>([&](int e) { return x[e]; }, [&](int e) { return r1[e]; });
          const float dist0 = (xx - 2.0f * xc0) + cc0, dist1 = (xx - 2.0f * xc1) + cc1;
          if (dist1 < dist0) cp1 = 1.0f;
          else cp0 = 1.0f;
        }
        if (q == 0) s_lab[m] = cp1 > 0.0f ? 2 : (cp0 > 0.0f ? 1 : 0);
        // the clusters' counts: a partial per aligned segment of `span` lanes (a group inside a wavefront, or a
        // group's part in one wavefront)
        const float w0 = wave_grp<Q>(cp0, span, fadd), w1 = wave_grp<Q>(cp1, span, fadd);
        if ((tid & (span - 1)) == 0) {
          s_gc[kLtGroups + tid / span] = w0;
          s_gc[2 * kLtGroups + tid / span] = w1;
        }
        if constexpr (local)
          lt_group_reduce_w<D, Q, 2, true>(s_x, s_gc + kLtGroups, L, false, s_cen + kLtGroups * RS, lane_id(), wv,
                                           s_lab);
        else
          lt_group_reduce<D, NT, 2, true, 2 * kWave / Q>(s_x, s_gc + kLtGroups, L * Q / span, L, false,
                                                         s_cen + kLtGroups * RS, tid, s_lab);
      }
      if (iters == 0) sync();   // the banks' copies of a and b, for the projection
    }
    if (mk + 1 < 16) TA_DMARK(mk + 1);
    // ranks by counting, the stable order of the projections on c0 - c1
    const int nl = (ng + 1) / 2, nr = ng - nl;
    const bool v = live && val(m);
    float key = kInf;
    if (v) key = slice_dot<D, Q>([&](int e) { return x[e]; }, [&](int e) { return c0b[e] - c1b[e]; });
    const int pm = live ? perm(m) : 0;
    const int fillp = live && lastinv >= 0 ? perm(g * S + lastinv) : 0;
    if (live && q == 0) s_key[m] = key;
    sync();
    int rank = 0;
    if (v) {
      for (int j = 0; j < S; ++j) {
        const float kj = s_key[g * S + j];
        rank += (kj < key || (kj == key && j < gl)) ? 1 : 0;
      }
    }
    if (v && q == 0) s_pv[g * S + (rank < nl ? rank : half + rank - nl)] = (uint32_t)pm | VB;
    if (live && q == 0) {
      const bool filled = gl < half ? gl < nl : (gl - half) < nr;
      if (!filled) s_pv[m] = (uint32_t)fillp;
    }
  };
  __syncthreads();
  for (int lvl = lt_log2(C / W); lvl < nlev; ++lvl) {
    const int S = C >> lvl;
    float x[DQ];
    if (live) {
      load_row_g<T, DQ>(kb + (int64_t)perm(m) * kst, x);
    } else {
#pragma unroll
      for (int d = 0; d < DQ; ++d) x[d] = 0.0f;
    }
    mk = 1 + 3 * (lvl - lt_log2(C / W));
    if (S * Q <= kWave) level(std::true_type{}, S, x);
    else level(std::false_type{}, S, x);
    __syncthreads();
    if (mk + 2 < 16) TA_DMARK(mk + 2);
  }
  // the window's leaves (slots 2i, 2i + 1): node sums and counts, kept in LDS rows [0, W / 2) and stored
  const int wl = W / 2, nleaf = C / 2;
  if (m < wl) {
    float x[DQ], y[DQ];
    load_row_g<T, DQ>(kb + (int64_t)perm(2 * m) * kst, x);
    load_row_g<T, DQ>(kb + (int64_t)perm(2 * m + 1) * kst, y);
    const float v0 = val(2 * m) ? 1.0f : 0.0f, v1 = val(2 * m + 1) ? 1.0f : 0.0f;
    float* row = tr.sums + (int64_t)(nleaf - 1 + win * wl + m) * D + d0;
#pragma unroll
    for (int d = 0; d < DQ; d += 4) {
      const float4 s4 = make_float4(x[d] * v0 + y[d] * v1, x[d + 1] * v0 + y[d + 1] * v1,
                                    x[d + 2] * v0 + y[d + 2] * v1, x[d + 3] * v0 + y[d + 3] * v1);
      *reinterpret_cast<float4*>(row + d) = s4;
      *reinterpret_cast<float4*>(rowx + d) = s4;
    }
    if (q == 0) {
      const int c2 = (int)val(2 * m) + (int)val(2 * m + 1);
      tr.cnt[nleaf - 1 + win * wl + m] = c2;
      s_nc[m] = c2;
    }
  }
  if (tid < W) {
    const int32_t sl = val(tid) ? perm(tid) : -1;
    tr.slot[base + tid] = sl;
  }
  // the nodes above the leaves up to the window's root, by adjacent pairs (LDS rows after the leaves' rows)
  int cofs = 0, pofs = wl;
  for (int lv = nlev - 1, nn = wl / 2; nn >= 1; --lv, nn >>= 1) {
    __syncthreads();
    const int64_t nb = ((int64_t)1 << lv) - 1 + (int64_t)win * nn;
    for (int w = tid; w < nn * (D / 4); w += NT) {
      const int i = w / (D / 4), d = (w - i * (D / 4)) * 4;
      const float* a = s_x + (cofs + 2 * i) * RS + d;
      const float4 u = *reinterpret_cast<const float4*>(a);
      const float4 z = *reinterpret_cast<const float4*>(a + RS);
      const float4 s4 = make_float4(u.x + z.x, u.y + z.y, u.z + z.z, u.w + z.w);
      *reinterpret_cast<float4*>(s_x + (pofs + i) * RS + d) = s4;
      *reinterpret_cast<float4*>(tr.sums + (nb + i) * D + d) = s4;
    }
    if (tid < nn) {
      const int c2 = s_nc[cofs + 2 * tid] + s_nc[cofs + 2 * tid + 1];
      s_nc[pofs + tid] = c2;
      tr.cnt[nb + tid] = c2;
    }
    cofs = pofs;
    pofs += nn;
  }
}

// lanetree_top_kernel, one workgroup per tree of more than 64 slots: the node sums and counts above the windows'
// roots, by adjacent pairs.
template <int D, int Q>
__global__ __launch_bounds__(kWave * Q) void lanetree_top_kernel(float* __restrict__ ws, int64_t P, int C) {
  constexpr int NT = kWave * Q;
  const int tid = threadIdx.x;
  const LaneTree tr = lane_tree(ws, P, C, D, blockIdx.x);
  for (int lv = lt_log2(C / kLaneSlots) - 1; lv >= 0; --lv) {
    const int nn = 1 << lv, base = nn - 1, cb = 2 * nn - 1;
    for (int w = tid; w < nn * (D / 4); w += NT) {
      const int i = w / (D / 4), d = (w - i * (D / 4)) * 4;
      const float* a = tr.sums + (int64_t)(cb + 2 * i) * D + d;
      const float4 u = *reinterpret_cast<const float4*>(a);
      const float4 z = *reinterpret_cast<const float4*>(a + D);
      *reinterpret_cast<float4*>(tr.sums + (int64_t)(base + i) * D + d) =
          make_float4(u.x + z.x, u.y + z.y, u.z + z.z, u.w + z.w);
    }
    for (int i = tid; i < nn; i += NT) tr.cnt[base + i] = tr.cnt[cb + 2 * i] + tr.cnt[cb + 2 * i + 1];
    __syncthreads();
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

// The nodes of a lane tree during the walk: nodes [0, ntop) (its top levels, ntop = 2^ltop - 1) live in LDS for
// the whole walk (rows of stride D + 4 floats, and counts), deeper nodes in the workspace; the leaf slots (C
// entries) live in LDS too up to kLaneLdsMaxT slots, above that (BIG) in the workspace.  A lane reads and writes
// its 16 dimensions of a row.
template <int D, bool BIG>
struct LaneNodes {
  LaneTree tr;
  float* top;
  int32_t* tcnt;
  int32_t* slot;   // the leaf slots: an LDS copy, or the workspace's when BIG
  int ntop, C;
  // Node n's count and row (this lane's 16 dimensions): L = the node is one of the LDS-held ones (n < ntop), a
  // compile-time choice, so that every access has a known address space (an address chosen between LDS and the
  // workspace at run time is a flat access, whose wait covers every outstanding memory operation).
  template <bool L>
  __device__ __forceinline__ int cnt(int n) const {
    if constexpr (L) return tcnt[n];
    else return tr.cnt[n];
  }
  template <bool L>
  __device__ __forceinline__ void set_cnt(int n, int v) const {
    if constexpr (L) tcnt[n] = v;
    else tr.cnt[n] = v;
  }
  template <bool L>
  __device__ __forceinline__ void row(int n, int d0, float (&r)[kLaneDQ]) const {
    if constexpr (L) {
      const float* src = top + n * (D + 4) + d0;
#pragma unroll
      for (int d = 0; d < kLaneDQ; d += 4) {
        const float4 v = *reinterpret_cast<const float4*>(src + d);
        r[d] = v.x;
        r[d + 1] = v.y;
        r[d + 2] = v.z;
        r[d + 3] = v.w;
      }
    } else {
      load_row_g<float, kLaneDQ>(tr.sums + (int64_t)n * D + d0, r);
    }
  }
  template <bool L>
  __device__ __forceinline__ void set_row(int n, int d0, const float (&r)[kLaneDQ]) const {
    float* dst = L ? top + n * (D + 4) + d0 : tr.sums + (int64_t)n * D + d0;
#pragma unroll
    for (int d = 0; d < kLaneDQ; d += 4)
      *reinterpret_cast<float4*>(dst + d) = make_float4(r[d], r[d + 1], r[d + 2], r[d + 3]);
  }
  // workspace -> LDS (to_lds) or back
  __device__ __forceinline__ void copy(bool to_lds, int tid, int nt) const {
    for (int i = tid; i < ntop * (D / 4); i += nt) {
      const int n = i / (D / 4), d = (i - n * (D / 4)) * 4;
      float4* l = reinterpret_cast<float4*>(top + n * (D + 4) + d);
      float4* g = reinterpret_cast<float4*>(tr.sums + (int64_t)n * D + d);
      if (to_lds) *l = *g;
      else *g = *l;
    }
    for (int n = tid; n < ntop; n += nt) {
      if (to_lds) tcnt[n] = tr.cnt[n];
      else tr.cnt[n] = tcnt[n];
    }
    if constexpr (!BIG) {
      for (int n = tid; n < C; n += nt) {
        if (to_lds) slot[n] = tr.slot[n];
        else tr.slot[n] = slot[n];
      }
    }
  }
};

// Search ranking word: valid first, then score descending, node id ascending; invalid candidates by slot.
// Unique per candidate, so a candidate's rank is the number of smaller words.
__device__ __forceinline__ uint64_t lt_rank_word(bool valid, float sc, int id, int slot) {
  if (!valid) return (1ull << 63) | (uint32_t)slot;
  const uint32_t u = __float_as_uint(sc + 0.0f);
  const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)(~asc) << 31) | (uint32_t)id;
}

// One workgroup per lane tree (built by the three build launches), walking the lane's positions in order
// (dyntree.py:148-243).  Slot j scores neighbour entry j and the level's children j and j + 64; the lanes of
// slot 0 insert the position's key.  The barriers order LDS traffic only (lds_barrier), so the next position's
// query and key rows, requested at a position's start, and the output stores stay in flight across them; counts
// over the workgroup go through one LDS word per wavefront.  A position ends with wavefront 0 (the inserting
// lanes) waiting for its stores, then a barrier: the tree rows, counts and slots the insertion wrote to the
// workspace are read by other wavefronts at the next position.
template <typename T, int D, int Q, bool BIG>
__global__ __launch_bounds__(kWave * Q) void lanetree_walk_kernel(LaneWalk p) {
  constexpr int DQ = kLaneDQ, NT = kWave * Q;
  __shared__ int32_t s_stl[kLaneMaxNb];   // stored leaves of the last Wn positions (ring), NS each
  __shared__ float s_sts[kLaneMaxNb];
  __shared__ uint8_t s_sto[kLaneMaxNb];
  __shared__ int32_t s_nid[kLaneSlots];
  __shared__ __align__(16) uint64_t s_rw[2 * kLaneMaxW];   // the level's children's ranking words
  __shared__ int32_t s_cur[kLaneMaxW];                      // the beam
  __shared__ float s_bsc[kLaneMaxW];
  __shared__ uint8_t s_bok[kLaneMaxW];
  __shared__ int s_wc[3][8];   // per-wavefront counts: matches and stored entries in the probe, first occurrences
  __shared__ float s_isc[kLaneSlots];   // the insertion's candidate scores
  const int tid = threadIdx.x, m = tid / Q, q = tid % Q, d0 = q * DQ, wv = wave_id();
  const int64_t pt = blockIdx.x;
  const int ln = (int)(pt % p.nlane);
  const int64_t bh = pt / p.nlane;
  const int64_t b = bh / p.H, h = bh % p.H;
  const T* qb = static_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + d0;
  const T* kb = static_cast<const T*>(p.k) + b * p.ksb + h * p.ksh + d0;
  const LaneTree tr = lane_tree(p.ws, p.P, p.C, D, pt);
  extern __shared__ __align__(16) unsigned char s_dyn[];
  LaneNodes<D, BIG> nd;
  nd.tr = tr;
  nd.top = reinterpret_cast<float*>(s_dyn);
  nd.tcnt = reinterpret_cast<int32_t*>(nd.top + p.ntop * (D + 4));
  nd.slot = BIG ? tr.slot : nd.tcnt + p.ntop;
  nd.ntop = p.ntop;
  nd.C = p.C;
  nd.copy(true, tid, NT);
  __syncthreads();
  const int WN = p.Wn * p.NS, wl = p.wl, nlev = p.nlev;
  const int ltop = lt_log2(p.ntop + 1);   // levels 0 .. ltop - 1 are held in LDS
  const float kInf = __int_as_float(0x7f800000);
  const int start = ln * p.chunk;
  const bool ins = tid < Q;    // the lanes of slot 0 (the root's update, the leaf slot)
  const bool insw = wv == 0;   // wavefront 0 inserts the keys
  float qn[DQ], kn[DQ];        // the next position's query and key, requested while the current position runs
  load_row_g<T, DQ>(qb + (int64_t)start * p.qst, qn);
#pragma unroll
  for (int d = 0; d < DQ; ++d) kn[d] = 0.0f;
  if (insw) load_row_g<T, DQ>(kb + (int64_t)start * p.kst, kn);
  for (int i = 0; i < p.chunk; ++i) {
    const int t = start + i;
    const int64_t orow = bh * p.T + t;
    // phase marks (trace.hpp) of the lane's last position: 0 start, 1 neighbours scored and counted, 2 first
    // occurrences counted, 3 search started, 4 + l level l + 1 ranked (l < 8), 12 outputs, 13 insertion started,
    // 14 insertion done (wavefront 0), 15 position done
    const bool mk = i == p.chunk - 1;
    if (mk) TA_DMARK(0);
    float qv[DQ], kd[DQ];
#pragma unroll
    for (int d = 0; d < DQ; ++d) {
      qv[d] = qn[d];
      kd[d] = kn[d];
    }
    if (i + 1 < p.chunk) {
      load_row_g<T, DQ>(qb + (int64_t)(t + 1) * p.qst, qn);
      if (insw) load_row_g<T, DQ>(kb + (int64_t)(t + 1) * p.kst, kn);
    }
    // ---- neighbours: the leaves the last Wn positions of the lane stored, re-scored on the current tree
    int id = 0;
    bool ok0 = false, match = false;
    if (m < WN) {
      const int back = m / p.NS + 1, j = i - back;
      if (j >= 0) {
        const int rs = (j % p.Wn) * p.NS + m % p.NS;
        ok0 = s_sto[rs] != 0;
        id = s_stl[rs];
        if (ok0) {
          const int node = (1 << nlev) - 1 + id;
          auto score = [&](auto lds) {
            constexpr bool L = decltype(lds)::value;
            const int cn = nd.template cnt<L>(node);
            float row[DQ];
            nd.template row<L>(node, d0, row);
            const float sc = slice_dot<D, Q>([&](int e) { return qv[e]; }, [&](int e) { return row[e]; }) /
                             (float)(cn > 1 ? cn : 1);
            const float base = s_sts[rs];
            return cn > 0 && sc >= base - p.rho * fabsf(base);
          };
          match = nlev < ltop ? score(std::true_type{}) : score(std::false_type{});
        }
      }
    }
    const bool inprobe = m < p.probe;
    {
      const uint64_t bm = __ballot(match && inprobe && q == 0), bo = __ballot(ok0 && inprobe && q == 0);
      if (lane_id() == 0) {
        s_wc[0][wv] = __popcll(bm);
        s_wc[1][wv] = __popcll(bo);
      }
    }
    lds_barrier();
    int pm = 0, po = 0;
    for (int w = 0; w < Q; ++w) {
      pm += s_wc[0][w];
      po += s_wc[1][w];
    }
    if (mk) TA_DMARK(1);
    const float rate = (float)pm / fmaxf((float)po, 1.0f);
    const int cap = p.cap_min + (int)rintf((float)(p.Wn - p.cap_min) * rate);
    match = match && (m / p.NS + 1) <= cap && p.neighbors;
    if (q == 0) s_nid[m] = match ? id : -1;
    lds_barrier();
    bool first = match;
    for (int e = 0; e < m && first; ++e) first = s_nid[e] != id;
    {
      const uint64_t bf = __ballot(first && q == 0);
      if (lane_id() == 0) s_wc[2][wv] = __popcll(bf);
    }
    lds_barrier();
    int nL = 0;
    for (int w = 0; w < Q; ++w) nL += s_wc[2][w];
    if (mk) TA_DMARK(2);
    if (m < WN && q == 0) {
      const int s0 = nd.slot[2 * id], s1 = nd.slot[2 * id + 1];
      int32_t* o = p.nb_pos + orow * 2 * WN;
      o[m] = match && s0 >= 0 ? s0 : -1;
      o[WN + m] = match && s1 >= 0 ? s1 : -1;
    }
    // ---- budget (dyntree.py:218-222)
    const int Lq = p.lhat[orow];
    const int lo = (Lq + 1) >> 1, need = Lq - nL > 0 ? Lq - nL : 0, floor_b = nL < lo ? 2 : 1;
    int bt = nL >= Lq ? 0 : (need > floor_b ? need : floor_b);
    bt = bt < p.wmax ? bt : p.wmax;
    // ---- beam search from the root
    if (tid == 0) {
      s_cur[0] = 0;
      s_bok[0] = nd.template cnt<true>(0) > 0;
      s_bsc[0] = 0.0f;
    }
    lds_barrier();
    if (mk) TA_DMARK(3);
    int wp = 1;
    auto search_level = [&](auto lds, int lv) __attribute__((always_inline)) {
      constexpr bool L = decltype(lds)::value;
      const int nch = 2 * wp;
      int cid[2];
      bool cv[2];
      float sc[2];
      uint64_t mine[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int c = m + kLaneSlots * r;
        cid[r] = 0;
        cv[r] = false;
        sc[r] = -kInf;
        mine[r] = 0;
        if (c < nch) {
          const int par = c < wp ? c : c - wp;
          cid[r] = 2 * s_cur[par] + (c < wp ? 0 : 1);
          if (s_bok[par]) {
            const int node = (1 << lv) - 1 + cid[r];
            const int cn = nd.template cnt<L>(node);
            float row[DQ];
            nd.template row<L>(node, d0, row);
            cv[r] = cn > 0;
            if (cv[r])
              sc[r] = slice_dot<D, Q>([&](int e) { return qv[e]; }, [&](int e) { return row[e]; }) /
                      (float)(cn > 1 ? cn : 1);
          }
          mine[r] = lt_rank_word(cv[r], sc[r], cid[r], c);
          if (q == 0) s_rw[c] = mine[r];
        }
      }
      lds_barrier();
      const int w = nch < p.wmax ? nch : p.wmax;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int c = m + kLaneSlots * r;
        if (c < nch) {   // the slot's lanes count the smaller words among every Q-th word, then add up
          int rank = 0;
          for (int j = q; j < nch; j += Q) rank += s_rw[j] < mine[r] ? 1 : 0;
          rank = slot_isum<Q>(rank);
          if (q == 0 && rank < w) {
            s_cur[rank] = cid[r];
            s_bsc[rank] = sc[r];
            s_bok[rank] = cv[r];
          }
        }
      }
      lds_barrier();
      if (mk && lv <= 8) TA_DMARK(3 + lv);
      wp = w;
    };
    int lv = 1;
    for (; lv <= nlev && lv < ltop; ++lv) search_level(std::true_type{}, lv);
    for (; lv <= nlev; ++lv) search_level(std::false_type{}, lv);
    // ---- outputs, and the stored leaves of this position
    if (m < wl && q == 0) {
      const int lid = s_cur[m];
      const bool ok = s_bok[m] != 0;
      const int s0 = nd.slot[2 * lid], s1 = nd.slot[2 * lid + 1];
      int32_t* o = p.tree_pos + orow * 2 * wl;
      o[m] = ok && s0 >= 0 ? s0 : -1;
      o[wl + m] = ok && s1 >= 0 ? s1 : -1;
      p.leaf_ok[orow * wl + m] = ok ? 1 : 0;
    }
    if (tid == 0) {
      p.n_tree[orow] = bt;
      p.nb_leaves[orow] = nL;
    }
    if (m < p.NS && q == 0) {
      const int rs = (i % p.Wn) * p.NS + m;
      s_stl[rs] = s_cur[m];
      s_sts[rs] = s_bsc[m];
      s_sto[rs] = s_bok[m];
    }
    if (mk) TA_DMARK(12);
    // ---- insertion of this position's key (dyntree.py:84-106) by wavefront 0, once every wavefront has read the
    // leaf slots of its outputs (their loads returned: the output stores use them), since the key may go into one of
    // those leaves (dyntree.py:224-241 reads the leaves' keys before the insertion).  Each step scores, one slot
    // each, all 2 + 4 + ... + 2^kk nodes of the next kk levels below the current node (kk <= KI: as many as the
    // wavefront's 64 / Q slots hold), then follows the path through them: at each level the right child when its
    // score is greater (dyntree.py:94-101; the scores use the rows and counts before the insertion, which
    // changes only the path's nodes), and the path's slots add the key to their node.
    lds_barrier();
    if (mk) TA_DMARK(13);
    if (wv == 0) {
      constexpr int KI = Q == 1 ? 5 : Q == 2 ? 4 : Q == 4 ? 3 : 2;   // 2^(KI + 1) - 2 <= 64 / Q
      const int act = t >= 1 ? 1 : 0;
      float kva[DQ];
#pragma unroll
      for (int d = 0; d < DQ; ++d) kva[d] = kd[d] * (act ? 1.0f : 0.0f);
      if (ins) {
        float r0[DQ];
        nd.template row<true>(0, d0, r0);
#pragma unroll
        for (int d = 0; d < DQ; ++d) r0[d] = r0[d] + kva[d];
        nd.template set_row<true>(0, d0, r0);
        if (q == 0) nd.template set_cnt<true>(0, nd.template cnt<true>(0) + act);
      }
      int node = 0;   // index within its level of the path's node at level lv
      auto ins_step = [&](auto lds, int lv, int kk) __attribute__((always_inline)) {
        constexpr bool L = decltype(lds)::value;
        const bool on = m < (2 << kk) - 2;
        const int dep = 31 - __clz(m + 2), ci = m + 2 - (1 << dep);   // this slot's node: depth dep, index ci
        const int lvc = lv + dep, id = (1 << lvc) - 1 + (node << dep) + ci;
        int cn = 0;
        float row[DQ];
#pragma unroll
        for (int d = 0; d < DQ; ++d) row[d] = 0.0f;
        if (on) {
          cn = nd.template cnt<L>(id);
          nd.template row<L>(id, d0, row);
        }
        const float dt = slice_dot<D, Q>([&](int e) { return kd[e]; }, [&](int e) { return row[e]; });
        float sc = cn == 0 ? -1e9f : dt / (float)(cn > 1 ? cn : 1);
        if (cn >= (p.C >> lvc)) sc = -kInf;
        if (on && q == 0) s_isc[m] = sc;
        wave_sync();
        int pi = 0;   // the path's index at depth dd
        bool onpath = false;
        for (int dd = 1; dd <= kk; ++dd) {
          const int l = (1 << dd) - 2 + 2 * pi;
          pi = 2 * pi + (s_isc[l + 1] > s_isc[l] ? 1 : 0);
          onpath = onpath || (on && dep == dd && ci == pi);
        }
        if (onpath) {
#pragma unroll
          for (int d = 0; d < DQ; ++d) row[d] = row[d] + kva[d];
          nd.template set_row<L>(id, d0, row);
          if (q == 0) nd.template set_cnt<L>(id, cn + act);
        }
        node = (node << kk) + pi;
        wave_sync();   // the scores are read before the next step writes them
      };
      int il = 0;   // the path's level; steps never span the last LDS level and the first workspace one
      while (il < nlev && il + 1 < ltop) {
        const int kk = min(KI, min(nlev, ltop - 1) - il);
        ins_step(std::true_type{}, il, kk);
        il += kk;
      }
      while (il < nlev) {
        const int kk = min(KI, nlev - il);
        ins_step(std::false_type{}, il, kk);
        il += kk;
      }
      if (tid == 0 && act) {
        const int s0 = nd.slot[2 * node];
        nd.slot[2 * node + (s0 >= 0 ? 1 : 0)] = t;
      }
    }
    if (mk) TA_DMARK(14);
    if (wv == 0) wait_vmcnt_n<0>();   // the insertion's stores to the workspace are done
    lds_barrier();
    if (mk) TA_DMARK(15);
  }
  nd.copy(false, tid, NT);
}

bool lanetree_dim_ok(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

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
    set_error("ta_lanetree_workspace_size: bad arguments (T a power of two in [4, 262144], chunk dividing T, "
              "D 16, 32, 64 or 128)");
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
  const bool big = T > kLaneLdsMaxT;
  const int64_t nwin = T > kLaneSlots ? T / kLaneSlots : 1;
  hipStream_t st = (hipStream_t)stream;
  if (P * nwin * (D / kLaneDQ * kWave) > (int64_t)0xffffffff) {   // the tail launch's threads
    set_error("ta_lanetree_build: too many lane trees for one launch (B * H * (T / chunk) * T / 64 workgroups)");
    return TA_ERR_ARG;
  }
  // the levels of groups above 64 slots (a launch per level, a workgroup per group), the rest (a workgroup per
  // window of 64 slots), then the node sums above the windows
#define TA_LB(TT, DD)                                                                                                 \
  for (int lvl = 0; (T >> lvl) > kLaneSlots; ++lvl) {                                                                 \
    const size_t lds = (size_t)lt_build_lds_bytes(T >> lvl, DD, big);                                                 \
    if (big)                                                                                                          \
      hipLaunchKernelGGL((lanetree_split_kernel<TT, DD, DD / kLaneDQ, true>), dim3((unsigned)(P << lvl)),             \
                         dim3(DD / kLaneDQ * kWave), lds, st, (const TT*)k, ksb, ksh, kst, H, T, T / chunk, chunk,    \
                         kmeans_iters, (float*)ws, P, lvl);                                                           \
    else                                                                                                              \
      hipLaunchKernelGGL((lanetree_split_kernel<TT, DD, DD / kLaneDQ, false>), dim3((unsigned)(P << lvl)),            \
                         dim3(DD / kLaneDQ * kWave), lds, st, (const TT*)k, ksb, ksh, kst, H, T, T / chunk, chunk,    \
                         kmeans_iters, (float*)ws, P, lvl);                                                           \
  }                                                                                                                   \
  if (T <= kLaneSlots)                                                                                                \
    hipLaunchKernelGGL((lanetree_split_kernel<TT, DD, DD / kLaneDQ, false>), dim3((unsigned)P),                       \
                       dim3(DD / kLaneDQ * kWave), (size_t)lt_build_lds_bytes(T, DD, false), st, (const TT*)k, ksb,   \
                       ksh, kst, H, T, T / chunk, chunk, kmeans_iters, (float*)ws, P, 0);                             \
  hipLaunchKernelGGL((lanetree_tail_kernel<TT, DD, DD / kLaneDQ>), dim3((unsigned)(P * nwin)),                        \
                     dim3(DD / kLaneDQ * kWave), 0, st, (const TT*)k, ksb, ksh, kst, H, T, T / chunk, kmeans_iters,   \
                     (float*)ws, P);                                                                                  \
  if (T > kLaneSlots)                                                                                                 \
    hipLaunchKernelGGL((lanetree_top_kernel<DD, DD / kLaneDQ>), dim3((unsigned)P), dim3(DD / kLaneDQ * kWave), 0, st, \
                       (float*)ws, P, T)
#define TA_LB_D(TT)                  \
  switch (D) {                       \
    case 16: TA_LB(TT, 16); break;   \
    case 32: TA_LB(TT, 32); break;   \
    case 64: TA_LB(TT, 64); break;   \
    default: TA_LB(TT, 128); break;  \
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
    set_error("ta_lanetree_walk: bad arguments (1 <= wmax <= 64, nb_window * nb_store <= 64, nb_store at most "
              "the leaves per query, workspace from ta_lanetree_workspace_size)");
    return TA_ERR_ARG;
  }
  const int es = dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)q % 16) || (qsb * es) % 16 || (qsh * es) % 16 || (qst * es) % 16 || ((uintptr_t)k % 16) ||
      (ksb * es) % 16 || (ksh * es) % 16 || (kst * es) % 16) {
    set_error("ta_lanetree_walk: query and key rows 16-byte aligned");
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
  // the top levels of every tree stay in LDS during the walk: as many whole levels as fit in the CU's LDS shared
  // by the workgroups each CU holds (the trees over the CUs; 4 KB left for the kernel's own arrays), beside the
  // leaf slots, and at least 40 KB of them (the deeper levels are the walk's slowest dependent reads)
  const bool big = T > kLaneLdsMaxT;
  const int rowb = (D + 4) * 4 + 4;
  const int64_t slots_b = big ? 0 : (int64_t)T * 4;
  const int cus = device_cus() > 0 ? device_cus() : 256, lds_cu = device_lds_per_cu() > 0 ? device_lds_per_cu() : 65536;
  const int64_t per_cu = (p.P + cus - 1) / cus;
  int64_t budget = lds_cu / (per_cu < 1 ? 1 : per_cu) - 4096 - slots_b;
  if (budget < 40960) budget = 40960;
  int ntop = 1;
  while (2 * ntop + 1 <= T - 1 && (int64_t)(2 * ntop + 1) * rowb <= budget) ntop = 2 * ntop + 1;
  p.ntop = ntop;
  const size_t lds = (size_t)ntop * rowb + (size_t)slots_b;   // + the leaf slots
  hipStream_t st = (hipStream_t)stream;
#define TA_LW(TT, DD)                                                                                                 \
  if (big)                                                                                                            \
    hipLaunchKernelGGL((lanetree_walk_kernel<TT, DD, DD / kLaneDQ, true>), dim3((unsigned)p.P),                       \
                       dim3(DD / kLaneDQ * kWave), lds, st, p);                                                       \
  else                                                                                                                \
    hipLaunchKernelGGL((lanetree_walk_kernel<TT, DD, DD / kLaneDQ, false>), dim3((unsigned)p.P),                      \
                       dim3(DD / kLaneDQ * kWave), lds, st, p)
#define TA_LW_D(TT)                  \
  switch (D) {                       \
    case 16: TA_LW(TT, 16); break;   \
    case 32: TA_LW(TT, 32); break;   \
    case 64: TA_LW(TT, 64); break;   \
    default: TA_LW(TT, 128); break;  \
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

TA_TRACE_EXPORTS
