// Mean-log dilution gate of the node summaries (replaces seg.py:16-23 gate_apply, its use in seg.py:26-41
// level_sums and fastseg.py:238-251 level_sums_min, and the gated SegState.getU / add of engine.py:35-39, 47,
// 53-54).
//
// A node's gated vector depends only on the node, so it is formed where the node is: for every dimension the
// mean log-magnitude ml = lg / size (lg: the node's sum of log(|k| + 1e-6) over its positions, formed by the
// same adjacent-pair float32 additions as the raw sums); thr = the gate_q quantile of ml over the dimensions
// (linear interpolation between the order statistics at floor and ceil of gate_q * (D - 1), torch.quantile's
// rule, with the interpolation's product and difference each rounded to float32); kept dimensions ml >= thr;
// gated = (raw * kept) * (D / max(#kept, 1)).  The descent and the neighbour pass then score the gated vectors
// of the levels at or above gate_min_level instead of the raw sums.
//
// The logarithm is the float32 rounding of the double-precision log of the float32 value |k| + 1e-6 (the CPU
// oracle's canonical mode computes it the same way), so the gated vectors are the same on both sides.
#pragma clang fp contract(off)

#include "append.hpp"
#include "common.hpp"

namespace ta {

__device__ __forceinline__ float index_log(float x) { return (float)log((double)(fabsf(x) + 1e-6f)); }

// Gate of one node held by one wavefront: dimension d = lane + 64 i (i < EPL) in raw[i], lg[i] (lanes past D
// hold nothing).  lo / w: the quantile's lower order statistic and interpolation weight.  Returns the gated
// values in g[i].
template <int D>
__device__ __forceinline__ void gate_node_wave(const float (&raw)[(D + 63) / 64], const float (&lg)[(D + 63) / 64],
                                               float inv_size, int lo, float w, float (&g)[(D + 63) / 64]) {
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

// Range mode: nodes [0, n_nodes[j]) of level j = blockIdx.z, four per workgroup (a wavefront each).
template <int D>
__global__ __launch_bounds__(256) void gate_range_kernel(GateLevels gl, int H, int lo, float w) {
  constexpr int EPL = (D + 63) / 64;
  const int j = blockIdx.z;
  if (gl.out[j] == nullptr) return;
  const int64_t node = (int64_t)blockIdx.x * 4 + wave_id();
  if (node >= gl.n_nodes[j]) return;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int64_t o = b * gl.sb[j] + h * gl.sh[j] + node * D;
  const int lane = lane_id();
  float raw[EPL], lg[EPL], g[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int d = lane + 64 * i;
    raw[i] = d < D ? gl.raw[j][o + d] : 0.0f;
    lg[i] = d < D ? gl.lg[j][o + d] : 0.0f;
  }
  gate_node_wave<D>(raw, lg, 1.0f / (float)(1ll << gl.blevel[j]), lo, w, g);
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (lane + 64 * i < D) gl.out[j][o + lane + 64 * i] = g[i];
}

// Decode mode, one wavefront per (sequence, head), after the cache append of row t (raw nodes ending at t
// already formed): the log sums of the nodes ending at t (the leaf block's keys read back from the cache), then
// the gated vectors of those nodes on gated levels.  Lane d (and d + 64) keeps dimension d's carry stack in
// registers: at most 2 + log2(arity) entries per level are live, so a fixed 20-entry stack covers leaf blocks
// up to 2^14 and any arity.
template <typename T, int D>
__global__ __launch_bounds__(64) void gate_append_kernel(AppendIn ap, GateLevels gl, int n_levels, int arity_log2,
                                                         int H, const int32_t* __restrict__ t_pos, int lo, float w) {
  constexpr int EPL = (D + 63) / 64;
  const int bh = blockIdx.x, b = bh / H, h = bh % H;
  const int t = t_pos[b];
  if (t < 0 || t >= ap.Tcap || n_levels == 0) return;
  const int leaf_log2 = gl.blevel[0];
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
    const int64_t o = b * gl.sb[j] + h * gl.sh[j] + node * D;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (lane + 64 * e < D) const_cast<float*>(gl.lg[j])[o + lane + 64 * e] = y[e];
    if (gl.out[j] != nullptr) {
      float raw[EPL], g[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) raw[e] = lane + 64 * e < D ? gl.raw[j][o + lane + 64 * e] : 0.0f;
      gate_node_wave<D>(raw, y, 1.0f / (float)(1ll << gl.blevel[j]), lo, w, g);
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        if (lane + 64 * e < D) gl.out[j][o + lane + 64 * e] = g[e];
    }
  };
  emit(0, t >> leaf_log2);
  const int arity = 1 << arity_log2;
  for (int j = 1; j < n_levels; ++j) {
    const int lj = gl.blevel[j];
    if (((t + 1) & ((1 << lj) - 1)) != 0) break;
    const int64_t node = t >> lj;
    const float* child = gl.lg[j - 1] + b * gl.sb[j - 1] + h * gl.sh[j - 1] + node * arity * D;
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

// quantile position of gate_q over D values as torch.quantile computes it in float32
void gate_rank(float gate_q, int D, int& lo, float& w) {
  const float r = gate_q * (float)(D - 1);
  lo = (int)floorf(r);
  w = r - (float)lo;
}

}  // namespace ta

using namespace ta;

extern "C" int ta_gate_levels(int B, int H, int D, int n_levels, const float* const* raw, const float* const* lg,
                              float* const* out, const int64_t* sb, const int64_t* sh, const int32_t* blevel,
                              const int64_t* n_nodes, float gate_q, void* stream) {
  if (B <= 0 || H <= 0 || n_levels < 0 || n_levels > kMaxLevels || !(gate_q >= 0.0f && gate_q <= 1.0f) ||
      (D != 16 && D != 32 && D != 64 && D != 128)) {
    set_error("ta_gate_levels: bad arguments (D 16, 32, 64 or 128; 0 <= gate_q <= 1)");
    return TA_ERR_ARG;
  }
  GateLevels gl{};
  int64_t most = 0;
  for (int j = 0; j < n_levels; ++j) {
    gl.raw[j] = raw[j];
    gl.lg[j] = lg[j];
    gl.out[j] = out[j];
    gl.sb[j] = sb[j];
    gl.sh[j] = sh[j];
    gl.n_nodes[j] = n_nodes[j];
    gl.blevel[j] = blevel[j];
    if (out[j] != nullptr && (raw[j] == nullptr || lg[j] == nullptr || blevel[j] < 0 || blevel[j] > 62)) {
      set_error("ta_gate_levels: a gated level needs its raw and log sums");
      return TA_ERR_ARG;
    }
    if (out[j] != nullptr && n_nodes[j] > most) most = n_nodes[j];
  }
  if (most == 0) return TA_OK;
  int lo;
  float w;
  gate_rank(gate_q, D, lo, w);
  const dim3 grid((unsigned)((most + 3) / 4), B * H, n_levels);
  hipStream_t st = (hipStream_t)stream;
  switch (D) {
    case 16: hipLaunchKernelGGL((gate_range_kernel<16>), grid, dim3(256), 0, st, gl, H, lo, w); break;
    case 32: hipLaunchKernelGGL((gate_range_kernel<32>), grid, dim3(256), 0, st, gl, H, lo, w); break;
    case 64: hipLaunchKernelGGL((gate_range_kernel<64>), grid, dim3(256), 0, st, gl, H, lo, w); break;
    default: hipLaunchKernelGGL((gate_range_kernel<128>), grid, dim3(256), 0, st, gl, H, lo, w); break;
  }
  return check_launch("gate_range_kernel");
}

extern "C" int ta_gate_append(const void* Kc, int dtype, int64_t csb, int64_t csh, int64_t cst, int Tcap, int B,
                              int H, int D, const int32_t* t_pos, int n_levels, const float* const* raw,
                              float* const* lg, float* const* out, const int64_t* sb, const int64_t* sh,
                              const int32_t* blevel, int arity_log2, float gate_q, const ta_kv_pages* pages,
                              void* stream) {
  if (B <= 0 || H <= 0 || n_levels < 0 || n_levels > kMaxLevels || Tcap <= 0 || t_pos == nullptr ||
      arity_log2 < 1 || arity_log2 > 4 || !(gate_q >= 0.0f && gate_q <= 1.0f) ||
      (D != 16 && D != 32 && D != 64 && D != 128)) {
    set_error("ta_gate_append: bad arguments");
    return TA_ERR_ARG;
  }
  if (n_levels == 0) return TA_OK;
  GateLevels gl{};
  for (int j = 0; j < n_levels; ++j) {
    if (raw[j] == nullptr || lg[j] == nullptr || blevel[j] < 1 || blevel[j] > 30) {
      set_error("ta_gate_append: every level needs its raw and log sums");
      return TA_ERR_ARG;
    }
    gl.raw[j] = raw[j];
    gl.lg[j] = lg[j];
    gl.out[j] = out[j];
    gl.sb[j] = sb[j];
    gl.sh[j] = sh[j];
    gl.blevel[j] = blevel[j];
  }
  if (gl.blevel[0] > 14) {
    set_error("ta_gate_append: leaf blocks of at most 2^14 positions");
    return TA_ERR_ARG;
  }
  if (pages && (pages->table == nullptr || pages->block_log2 != gl.blevel[0] || pages->num_pages <= 0 ||
                pages->page_stride < (cst << gl.blevel[0]))) {
    set_error("ta_gate_append: bad page description (block must be the leaf block)");
    return TA_ERR_ARG;
  }
  AppendIn ap{nullptr, nullptr, 0, 0, 0, 0, const_cast<void*>(Kc), nullptr, csb, csh, cst, Tcap};
  if (pages != nullptr) {
    ap.ptab = pages->table;
    ap.pt_sb = pages->sb;
    ap.pt_sh = pages->sh;
    ap.pstride = pages->page_stride;
    ap.npages = pages->num_pages;
  }
  int lo;
  float w;
  gate_rank(gate_q, D, lo, w);
  hipStream_t st = (hipStream_t)stream;
#define TA_GA(TT, DD) \
  hipLaunchKernelGGL((gate_append_kernel<TT, DD>), dim3(B * H), dim3(64), 0, st, ap, gl, n_levels, arity_log2, H, t_pos, lo, w)
#define TA_GA_D(TT)                    \
  switch (D) {                         \
    case 16: TA_GA(TT, 16); break;     \
    case 32: TA_GA(TT, 32); break;     \
    case 64: TA_GA(TT, 64); break;     \
    default: TA_GA(TT, 128); break;    \
  }
  switch (dtype) {
    case TA_F32: TA_GA_D(float); break;
    case TA_F16: TA_GA_D(f16_t); break;
    case TA_BF16: TA_GA_D(bf16_t); break;
    default: set_error("ta_gate_append: unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_GA_D
#undef TA_GA
  return check_launch("gate_append_kernel");
}
