// The candidate list of the module forward (fastseg.py:367-381, attention_dyn.py:12-17 and 74-96), in one
// launch: for every query row, the candidates in the reference's order -- the tree leaves' keys (leaf groups of
// `leaf` positions: entry r * wl + j is position r of leaf j), the neighbour leaves' keys, the static keys (0, t,
// t - 1, ..., t - Lw + 1 with Lw = max(local, 3)) and, for leaf > 2, the query's own leaf group up to t -- each
// valid where the reference's mask says so (a tree entry: its leaf is among the first n_tree found ones and
// the position is not -1; every other entry: not -1), then only the first valid copy of each position kept
// (the dedupe, selection.dedupe_fast), written as the masked row (position or -1, int32) that the sparse
// attention takes, with the row's counts for the module's statistics: kept entries in all, among the tree
// entries and among the neighbour entries, and the leaves used.
//
// One wavefront per query row: the row's candidates and validity go to LDS, and lane e tests its entries e, e +
// 64, ... against every earlier valid entry (a row holds at most kCandMax entries).
#include "common.hpp"

namespace ta {

constexpr int kCandMax = 320;   // candidates per row
constexpr int kCandRows = 4;    // rows (wavefronts) per workgroup

__global__ __launch_bounds__(kWave * kCandRows) void assemble_candidates_kernel(
    const int64_t* __restrict__ tree_pos, const uint8_t* __restrict__ leaf_ok, const int64_t* __restrict__ n_tree,
    const int64_t* __restrict__ nb_pos, const int64_t* __restrict__ tq, int tq_batched, int B, int H, int N, int wl,
    int leaf, int nbk, int local, int KC, int32_t* __restrict__ cm, int32_t* __restrict__ counts) {
  __shared__ int32_t s_pos[kCandRows][kCandMax];
  __shared__ uint8_t s_val[kCandRows][kCandMax];
  const int lane = lane_id(), wv = wave_id();
  const int64_t row = (int64_t)blockIdx.x * kCandRows + wv;
  if (row >= (int64_t)B * H * N) return;   // a whole wavefront leaves; no workgroup barrier follows
  const int64_t b = row / ((int64_t)H * N), n = row % N;
  const int64_t t = tq[tq_batched ? b * N + n : n];
  const int ntr = (int)n_tree[row];
  const int lw = local > 3 ? local : 3, ntp = leaf * wl, ns = 1 + lw;
  int32_t* pos = s_pos[wv];
  uint8_t* val = s_val[wv];
  // the row's candidates and validity
  for (int e = lane; e < KC; e += kWave) {
    int64_t p = -1;
    bool v = false;
    if (e < ntp) {
      const int j = e % wl;
      p = tree_pos[row * ntp + e];
      v = p >= 0 && leaf_ok[row * wl + j] != 0 && j < ntr;
    } else if (e < ntp + nbk) {
      p = nb_pos[row * nbk + (e - ntp)];
      v = p >= 0;
    } else if (e < ntp + nbk + ns) {
      const int s = e - ntp - nbk;
      p = s == 0 ? 0 : t - (s - 1);
      if (p < 0) p = -1;
      v = p >= 0;
    } else {
      const int r = e - ntp - nbk - ns;
      p = (t / leaf) * leaf + r;
      if (p > t) p = -1;
      v = p >= 0;
    }
    pos[e] = (int32_t)p;
    val[e] = v ? 1 : 0;
  }
  wave_sync();
  // first valid copy of each position
  int kept = 0, kept_tree = 0, kept_nb = 0;
  for (int e = lane; e < KC; e += kWave) {
    const int32_t p = pos[e];
    bool keep = val[e] != 0;
    for (int j = 0; j < e && keep; ++j) keep = !(val[j] != 0 && pos[j] == p);
    cm[row * KC + e] = keep ? p : -1;
    kept += keep ? 1 : 0;
    kept_tree += keep && e < ntp ? 1 : 0;
    kept_nb += keep && e >= ntp && e < ntp + nbk ? 1 : 0;
  }
  int used = 0;
  for (int j = lane; j < wl; j += kWave) used += leaf_ok[row * wl + j] != 0 && j < ntr ? 1 : 0;
  for (int o = 32; o >= 1; o >>= 1) {
    kept += __shfl_xor(kept, o);
    kept_tree += __shfl_xor(kept_tree, o);
    kept_nb += __shfl_xor(kept_nb, o);
    used += __shfl_xor(used, o);
  }
  if (lane == 0) {
    int32_t* c = counts + row * 4;
    c[0] = kept;
    c[1] = kept_tree;
    c[2] = kept_nb;
    c[3] = used;
  }
}

}  // namespace ta

using namespace ta;

extern "C" int ta_assemble_candidates(const int64_t* tree_pos, const uint8_t* leaf_ok, const int64_t* n_tree,
                                      const int64_t* nb_pos, const int64_t* tq, int tq_batched, int B, int H, int N,
                                      int wl, int leaf, int nbk, int local, int32_t* cm, int32_t* counts,
                                      void* stream) {
  const int lw = local > 3 ? local : 3;
  const int64_t KC = (int64_t)leaf * wl + nbk + 1 + lw + (leaf > 2 ? leaf : 0);
  if (tree_pos == nullptr || leaf_ok == nullptr || n_tree == nullptr || tq == nullptr || cm == nullptr ||
      counts == nullptr || (nbk > 0 && nb_pos == nullptr) || B <= 0 || H <= 0 || N <= 0 || wl < 1 || leaf < 2 ||
      nbk < 0 || local < 0 || KC > kCandMax) {
    set_error("ta_assemble_candidates: bad arguments (at most 320 candidates per row: leaf * wl + nbk + 1 + "
              "max(local, 3) (+ leaf when leaf > 2))");
    return TA_ERR_ARG;
  }
  const int64_t rows = (int64_t)B * H * N;
  const int64_t grid = (rows + kCandRows - 1) / kCandRows;
  if (grid > 0x7fffffff) {
    set_error("ta_assemble_candidates: too many rows");
    return TA_ERR_ARG;
  }
  hipLaunchKernelGGL(assemble_candidates_kernel, dim3((unsigned)grid), dim3(kWave * kCandRows), 0,
                     (hipStream_t)stream, tree_pos, leaf_ok, n_tree, nb_pos, tq, tq_batched, B, H, N, wl, leaf, nbk,
                     local, (int)KC, cm, counts);
  return check_launch("ta_assemble_candidates");
}
