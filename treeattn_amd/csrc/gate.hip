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

#include "gate.hpp"

namespace ta {


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

// Decode mode, one wavefront per (sequence, head) (gate_append_wave).
template <typename T, int D>
__global__ __launch_bounds__(64) void gate_append_kernel(AppendIn ap, GateLevels gl, int n_levels, int arity_log2,
                                                         int H, const int32_t* __restrict__ t_pos, int lo, float w) {
  const int bh = blockIdx.x, b = bh / H, h = bh % H;
  gate_append_wave<T, D>(ap, GateLevelsView{gl}, n_levels, arity_log2, b, h, t_pos[b], lo, w);
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
