// Segment-tree key selection on gfx950: level-sum pyramid builder, beam descent with per-query top-k,
// and gather-dot scoring.  Every score that decides a selection is computed in the canonical float32
// order (products rounded separately, grouped halving-tree sum), so results are bit-identical to the CPU
// oracle's canonical mode.  This file is compiled with -ffp-contract=off.
//
// Reference functions replaced: seg.py:26-41 level_sums, fastseg.py:238-251 level_sums_min (no gate),
// seg.py:44-70 tree_pass, fastseg.py:254-271 tree_pass_fast, fastseg.py:118-130 gather_dot.
#pragma clang fp contract(off)

#include "append.hpp"
#include "common.hpp"
#include "descend.hpp"
#include "gate.hpp"

namespace ta {

// ----------------------------------------------------------------------------------------- pyramid build
struct LevelOut {
  float* ptr[kMaxLevels];
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
  int8_t slot_of_blevel[64];  // binary level -> output level index, -1 when not written
};

__device__ __forceinline__ void store_node(const LevelOut& lo, int blevel, int b, int h, int64_t node, int D,
                                           int d, float x) {
  if (blevel < 64) {
    int j = lo.slot_of_blevel[blevel];
    if (j >= 0) lo.ptr[j][b * lo.sb[j] + h * lo.sh[j] + node * D + d] = x;
  }
}

// One pass over rows of granularity 2^base (base 0: the keys).  Thread (d, seg): dimension d of a segment
// of 64 consecutive rows, reduced by adjacent pairs with a carry stack (left + right, float32); the
// workgroup then combines its NSEG segment sums the same way.  Nodes are written when their binary level
// is an output level; the workgroup's total (the node of size 64*NSEG rows) goes to `tot` when complete.
// LOGT: the rows are index keys whose log-magnitudes are summed instead (the gate's statistic): each key
// value x (after the sink is zeroed) enters as the float32 rounding of the double log of |x| + 1e-6.
__device__ __forceinline__ float index_log_key(float x) { return (float)log((double)(fabsf(x) + 1e-6f)); }

template <typename T, int D, bool LOGT = false>
__global__ __launch_bounds__(256) void level_pass_kernel(const T* __restrict__ in, int64_t isb, int64_t ish,
                                                         int64_t isr, int H, int n_rows, int base,
                                                         int zero_first, LevelOut lo, float* __restrict__ tot,
                                                         int n_chunks) {
  constexpr int NSEG = 256 / D;
  constexpr int LOG_NSEG = NSEG == 1 ? 0 : NSEG == 2 ? 1 : NSEG == 4 ? 2 : NSEG == 8 ? 3 : 4;
  __shared__ float seg_sum[NSEG][D];
  const int d = threadIdx.x % D;
  const int seg = threadIdx.x / D;
  const int chunk = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int64_t row0 = (int64_t)chunk * 64 * NSEG + seg * 64;
  const T* src = in + b * isb + h * ish + d;

  float carry[7];
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const int64_t r = row0 + i;
    if (r < n_rows) {
      float x = (zero_first && r == 0) ? 0.0f : to_f32(src[r * isr]);
      if constexpr (LOGT) x = index_log_key(x);
      int lv = 0;
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        if (((i >> k) & 1) == 0) break;
        x = __fadd_rn(carry[k], x);
        lv = k + 1;
        store_node(lo, base + lv, b, h, r >> lv, D, d, x);
      }
      carry[lv] = x;
    }
  }
  const bool seg_full = row0 + 63 < n_rows;
  if (seg_full) seg_sum[seg][d] = carry[6];
  __syncthreads();
  if (seg == 0) {
    float c2[LOG_NSEG + 1];
    const int64_t gseg0 = (int64_t)chunk * NSEG;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      if ((gseg0 + s) * 64 + 63 < n_rows) {
        float x = seg_sum[s][d];
        int lv = 0;
#pragma unroll
        for (int k = 0; k < LOG_NSEG; ++k) {
          if (((s >> k) & 1) == 0) break;
          x = __fadd_rn(c2[k], x);
          lv = k + 1;
          store_node(lo, base + 6 + lv, b, h, (gseg0 + s) >> lv, D, d, x);
        }
        c2[lv] = x;
      }
    }
    if (tot != nullptr && (int64_t)(chunk + 1) * 64 * NSEG <= n_rows)
      tot[((int64_t)bh * n_chunks + chunk) * D + d] = c2[LOG_NSEG];
  }
}

// The same pass with each thread holding VEC = 16 / sizeof(T) consecutive dimensions of a row, read with one
// 16-byte load per row: TPR = D / VEC threads cover a row, so a wavefront's load instruction reads whole row
// slices of 64 / TPR rows (64 rows apart), and each thread keeps 16 rows in flight.  Thread (slice, seg):
// dimensions [slice VEC, slice VEC + VEC) of a segment of 64 consecutive rows, reduced by adjacent pairs with a
// carry stack; the workgroup's NSEG = 256 / TPR segment sums are then combined pairwise in LDS, one tree level
// per step.  Every node is (left + right) of its two children, so the nodes equal level_pass_kernel's bit for
// bit whatever the thread layout.  Rows, level rows and the strides must keep 16-byte slices aligned.
// (A thread holds 16 rows' loads: two batches of 8.)
template <typename T>
struct VecPass {
  static constexpr int VEC = 16 / (int)sizeof(T);
};

template <int VEC>
__device__ __forceinline__ void store_node_vec(const LevelOut& lo, int blevel, int b, int h, int64_t node, int D,
                                               int d0, const float (&x)[VEC]) {
  if (blevel < 64) {
    const int j = lo.slot_of_blevel[blevel];
    if (j >= 0) {
      float* p = lo.ptr[j] + b * lo.sb[j] + h * lo.sh[j] + node * D + d0;
#pragma unroll
      for (int c = 0; c < VEC; c += 4) *reinterpret_cast<float4*>(p + c) = make_float4(x[c], x[c + 1], x[c + 2], x[c + 3]);
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void level_vec_kernel(const T* __restrict__ in, int64_t isb, int64_t ish,
                                                        int64_t isr, int H, int n_rows, int base, int zero_first,
                                                        LevelOut lo, float* __restrict__ tot, int n_chunks) {
  constexpr int VEC = VecPass<T>::VEC;
  constexpr int TPR = D / VEC;
  constexpr int NSEG = 256 / TPR;
  constexpr int LOG_NSEG = NSEG == 2 ? 1 : NSEG == 4 ? 2 : NSEG == 8 ? 3 : NSEG == 16 ? 4 : NSEG == 32 ? 5 :
                           NSEG == 64 ? 6 : 7;
  constexpr int RB = 8;    // rows per load batch; two batches in flight
  static_assert(TPR >= 1 && (1 << LOG_NSEG) == NSEG, "layout");
  __shared__ __align__(16) float seg_sum[NSEG][D];
  const int sl = threadIdx.x % TPR;
  const int seg = threadIdx.x / TPR;
  const int d0 = sl * VEC;
  const int chunk = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int64_t crow0 = (int64_t)chunk * 64 * NSEG;
  const int64_t row0 = crow0 + seg * 64;
  const T* src = in + b * isb + h * ish + d0;
  const int64_t last = n_rows - 1;

  float carry[7][VEC];
  uint4 buf[2][RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int64_t r = row0 + i < last ? row0 + i : last;
    buf[0][i] = ldg16(src + r * isr);
  }
#pragma unroll
  for (int bt = 0; bt < 64 / RB; ++bt) {
    if (bt + 1 < 64 / RB) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int64_t rr = row0 + (bt + 1) * RB + i;
        const int64_t r = rr < last ? rr : last;
        buf[(bt + 1) & 1][i] = ldg16(src + r * isr);
      }
    }
#pragma unroll
    for (int i0 = 0; i0 < RB; ++i0) {
      const int i = bt * RB + i0;
      const int64_t r = row0 + i;
      if (r < n_rows) {
        float x[VEC];
        const T* e = reinterpret_cast<const T*>(&buf[bt & 1][i0]);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          x[v] = (zero_first && r == 0) ? 0.0f : to_f32(e[v]);
        }
        int lv = 0;
#pragma unroll
        for (int k = 0; k < 6; ++k) {
          if (((i >> k) & 1) == 0) break;
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = __fadd_rn(carry[k][v], x[v]);
          lv = k + 1;
          store_node_vec<VEC>(lo, base + lv, b, h, r >> lv, D, d0, x);
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) carry[lv][v] = x[v];
      }
    }
  }
  if (row0 + 63 < n_rows) {
#pragma unroll
    for (int v = 0; v < VEC; v += 4)
      *reinterpret_cast<float4*>(&seg_sum[seg][d0 + v]) =
          make_float4(carry[6][v], carry[6][v + 1], carry[6][v + 2], carry[6][v + 3]);
  }
  // pairwise combination of the segment sums: at step k the node of binary level base + 6 + k + 1 with index p
  // in this chunk is seg_sum[2p << k] + seg_sum[(2p + 1) << k], kept in the left child's slot
  for (int k = 0; k < LOG_NSEG; ++k) {
    __syncthreads();
    const int npairs = NSEG >> (k + 1);
    for (int e = threadIdx.x; e < npairs * TPR; e += 256) {
      const int p = e / TPR, s2 = e % TPR;
      const int64_t node_rows = (int64_t)64 << (k + 1);
      if (crow0 + (p + 1) * node_rows <= n_rows) {
        float* lft = &seg_sum[(2 * p) << k][s2 * VEC];
        const float* rgt = &seg_sum[(2 * p + 1) << k][s2 * VEC];
        float x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) x[v] = __fadd_rn(lft[v], rgt[v]);
#pragma unroll
        for (int v = 0; v < VEC; ++v) lft[v] = x[v];
        store_node_vec<VEC>(lo, base + 6 + k + 1, b, h, (int64_t)chunk * (NSEG >> (k + 1)) + p, D, s2 * VEC, x);
      }
    }
  }
  if (tot != nullptr && crow0 + 64 * NSEG <= n_rows) {
    __syncthreads();
    for (int e = threadIdx.x; e < D / 4; e += 256)
      *reinterpret_cast<float4*>(tot + ((int64_t)bh * n_chunks + chunk) * D + 4 * e) =
          *reinterpret_cast<const float4*>(&seg_sum[0][4 * e]);
  }
}

// ----------------------------------------------------------------------------------------- descent
// The mean-log gate's share of a fused decode append: the log-sum and gated-vector levels (same strides as the
// levels the append forms; out[j] null where the level is not gated) and the quantile's order statistic / weight.
struct GateAppendIn {
  float* lg[kMaxLevels];
  float* out[kMaxLevels];
  int lo;
  float w;
};

// The gate append's view of a fused descent's levels: the raw sums are the append's own targets.
struct DescentGateView {
  const LevelIn& raw_lv;
  const GateAppendIn& ga;
  __device__ __forceinline__ const float* raw(int j) const { return raw_lv.ptr[j]; }
  __device__ __forceinline__ float* lg(int j) const { return ga.lg[j]; }
  __device__ __forceinline__ float* out(int j) const { return ga.out[j]; }
  __device__ __forceinline__ int64_t sb(int j) const { return raw_lv.sb[j]; }
  __device__ __forceinline__ int64_t sh(int j) const { return raw_lv.sh[j]; }
  __device__ __forceinline__ int blevel(int j) const { return raw_lv.blevel[j]; }
};

// Descent of one query per WPQ wavefronts; with APPEND (one query per (sequence, head)) the decode-cache
// append of ap (rows of the query's element type) runs in the same launch.
template <typename TQ, int D, int WPQ, bool APPEND, bool GATE>
__global__ __launch_bounds__(WPQ == 16 ? 1024 : 256) void descend_kernel(
    const TQ* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qsn, int H, int Nq, int T,
    const int32_t* __restrict__ tq, int64_t tq_sb, LevelIn lv, int n_levels, int arity_log2, int wmax, int wl,
    int cmax4, int32_t* __restrict__ ids, uint8_t* __restrict__ vld, float* __restrict__ sct, AppendIn ap,
    LevelIn alv, ta_leaf_store_out so, GateAppendIn ga) {
  constexpr int NT = kWave * WPQ;      // threads per query
  extern __shared__ int32_t smem_i[];
  const int lane = lane_id(), w = wave_id();
  const int qw = w / WPQ;              // query slot in the block
  const int tid = (w % WPQ) * kWave + lane;
  const int n = blockIdx.x * ((int)blockDim.x / NT) + qw;
  if (n >= Nq) return;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int wmax4 = (wmax + 3) & ~3;
  // per query: rank keys (uint64), candidate ids and scores, kept ids and scores
  uint64_t* ckey = reinterpret_cast<uint64_t*>(smem_i + qw * (4 * cmax4 + 2 * wmax4));
  int32_t* cid = reinterpret_cast<int32_t*>(ckey + cmax4);
  float* csc = reinterpret_cast<float*>(cid + cmax4);
  int32_t* kid = cid + 2 * cmax4;
  float* ksc = reinterpret_cast<float*>(kid + wmax4);

  const int t = tq[b * tq_sb + n];
  TA_DMARK(12);
  if constexpr (APPEND) {
    // row t and the nodes ending at t; the descent below reads only nodes that end before t
    if (tid < D && t >= 0 && t < ap.Tcap) {
      float* stk = reinterpret_cast<float*>(smem_i + 4 * cmax4 + 2 * wmax4);   // one query per block
      TQ *kbase, *vbase;
      const KvRows rows = append_rows<TQ>(ap, b, h, lv.blevel[0], kbase, vbase);
      append_dim<TQ>(tid, D, t, reinterpret_cast<const TQ*>(ap.kn) + b * ap.nsb + h * ap.nsh,
                     reinterpret_cast<const TQ*>(ap.vn) + b * ap.vnsb + h * ap.vnsh, kbase, vbase, rows, n_levels,
                     lv.blevel[0], arity_log2, stk,
                     [&](int j) { return const_cast<float*>(alv.ptr[j]) + b * alv.sb[j] + h * alv.sh[j]; });
    }
  }
  TA_DMARK(13);
  const int64_t obase = ((int64_t)bh * Nq + n) * wl;
  const int nk = descend_query<TQ, D, WPQ>(q + b * qsb + h * qsh + n * qsn, t, T, b, h, lv, n_levels, arity_log2,
                                           wmax, tid, ckey, cid, csc, kid, ksc);
  TA_DMARK(14);
  for (int r = tid; r < wl; r += NT) {
    if (r < nk) {
      ids[obase + r] = kid[r];
      vld[obase + r] = 1;
      sct[obase + r] = ksc[r];
    } else {
      ids[obase + r] = -1;
      vld[obase + r] = 0;
      sct[obase + r] = -INFINITY;
    }
  }
  if (so.leaf != nullptr && t >= 0 && t < so.Tst) {
    // the neighbour store of position t: kept leaves first, empty slots as id 0, score 0, not ok
    const int64_t sbase = b * so.sb + h * so.sh + (int64_t)t * so.st;
    for (int r = tid; r < so.n; r += NT) {
      const bool ok = r < nk;
      so.leaf[sbase + r] = ok ? max(kid[r], 0) : 0;
      so.score[sbase + r] = ok ? ksc[r] : 0.0f;
      so.ok[sbase + r] = ok ? 1 : 0;
    }
  }
  if constexpr (APPEND && GATE) {
    // the gate's share of the append when position t completes a leaf block (one query per workgroup, so the
    // condition is the workgroup's): the block's keys and the raw nodes the append formed, written by this
    // workgroup's threads, are read back by its first wavefront after a barrier
    if (t >= 0 && t < ap.Tcap && n_levels > 0 && ((t + 1) & ((1 << lv.blevel[0]) - 1)) == 0) {
      __syncthreads();
      if (w == 0) gate_append_wave<TQ, D>(ap, DescentGateView{alv, ga}, n_levels, arity_log2, b, h, t, ga.lo, ga.w);
    }
  }
}

// ----------------------------------------------------------------------------------------- gather-dot
// One wavefront per query row; 4 candidates per round (16 lanes each).  blk != nullptr selects the
// leaf-block form: candidate c is row blk[c >> block_log2] * block + (c & (block - 1)).
template <typename TQ, typename TS, int D>
__global__ __launch_bounds__(256) void gather_dot_kernel(const TQ* __restrict__ q, int64_t qsb, int64_t qsh,
                                                         int64_t qsn, const TS* __restrict__ S, int64_t ssb,
                                                         int64_t ssh, int64_t ssn, const int32_t* __restrict__ cand,
                                                         const int32_t* __restrict__ blk, int block_log2, int NB_blk,
                                                         int H, int N, int M, int C, float scale,
                                                         float* __restrict__ out) {
  constexpr int R = D / 16;
  constexpr int NB = (64 / R) < 16 ? (64 / R) : 16;
  const int lane = lane_id(), w = wave_id();
  const int n = blockIdx.x * (blockDim.x / kWave) + w;
  if (n >= N) return;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int g = lane >> 4, j16 = lane & 15;
  float qr[R];
  load_row<TQ, R>(q + b * qsb + h * qsh + n * qsn + R * j16, qr);
  const TS* base = S + b * ssb + h * ssh + R * j16;
  const int64_t row = (int64_t)bh * N + n;
  for (int c0 = 0; c0 < C; c0 += 4 * NB) {
    float rows[NB][R];
#pragma unroll
    for (int r = 0; r < NB; ++r) {
      const int c = c0 + 4 * r + g;
      if (c < C) {
        int idx;
        if (blk != nullptr) {
          idx = (blk[row * NB_blk + (c >> block_log2)] << block_log2) + (c & ((1 << block_log2) - 1));
        } else {
          idx = cand[row * C + c];
        }
        idx = idx < 0 ? 0 : (idx > M - 1 ? M - 1 : idx);
        load_row<TS, R>(base + (int64_t)idx * ssn, rows[r]);
      } else {
#pragma unroll
        for (int i = 0; i < R; ++i) rows[r][i] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < NB; ++r) {
      const int c = c0 + 4 * r + g;
      const float s = __fmul_rn(canon_dot<R>(qr, rows[r]), scale);
      if (c < C && j16 == 0) out[row * C + c] = s;
    }
  }
}

// ----------------------------------------------------------------------------------------- host side
namespace {

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int log2i(int64_t x) {
  int l = 0;
  while ((int64_t(1) << l) < x) ++l;
  return l;
}

template <template <typename, int> class F, typename... A>
int dispatch_dt_d(int dt, int D, A&&... a) {
#define TA_CASE_D(T)                                            \
  switch (D) {                                                  \
    case 16: return F<T, 16>::run(std::forward<A>(a)...);       \
    case 32: return F<T, 32>::run(std::forward<A>(a)...);       \
    case 64: return F<T, 64>::run(std::forward<A>(a)...);       \
    case 128: return F<T, 128>::run(std::forward<A>(a)...);     \
    default: set_error("head dim must be 16, 32, 64 or 128"); return TA_ERR_UNSUPPORTED; \
  }
  switch (dt) {
    case TA_F32: TA_CASE_D(float)
    case TA_F16: TA_CASE_D(f16_t)
    case TA_BF16: TA_CASE_D(bf16_t)
    default: set_error("unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_CASE_D
}

int chunk_rows(int D) { return 64 * (256 / D); }

// Rows of the pass's input a workgroup reduces: 64 rows per segment, 256 / (threads per row) segments.
int chunk_rows_vec(int D, int elem) { return 64 * (256 / (D / (16 / elem))); }

template <typename T, int D>
struct LevelSumsRun {
  // The 16-byte-slice pass needs a slice of at least 4 floats per thread and aligned rows; the element pass
  // (level_pass_kernel) covers every other layout.
  static bool vec_ok(const void* p, int elem, int64_t sb, int64_t sh, int64_t sr, const LevelOut& lo, int n_out) {
    if (D * elem < 16 || (D * elem) % 16) return false;
    if ((uintptr_t)p % 16) return false;
    for (int64_t s : {sb, sh, sr})
      if ((s * elem) % 16) return false;
    for (int j = 0; j < n_out; ++j)
      if ((uintptr_t)lo.ptr[j] % 16 || (lo.sb[j] * 4) % 16 || (lo.sh[j] * 4) % 16) return false;
    return true;
  }

  static int run(const void* k, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int t_end, int zero_sink,
                 const LevelOut& lo, int n_out, int top_blevel, float* ws, hipStream_t st, bool logt = false) {
    // the workspace holds the chunk totals of the element pass's chunks (the smallest any pass uses)
    int64_t nA = ((int64_t)t_end / chunk_rows(D) + 1) * B * H * D;
    float* bufs[2] = {ws, ws + nA};
    int base = 0;
    int n_rows = t_end;
    int pass = 0;
    // pass 0 reads the keys; later passes read the previous pass's chunk totals
    const void* src = k;
    int64_t sb = ksb, sh = ksh, sr = kst;
    while (true) {
      const int elem = pass == 0 ? (int)sizeof(T) : 4;
      // the log-magnitude pass (the gate's statistic) stays on the element pass: its double-precision log is a
      // call, around which the 16-byte pass's row loop would not stay unrolled
      const bool vec = !(pass == 0 && logt) && vec_ok(src, elem, sb, sh, sr, lo, n_out);
      const int CH = vec ? chunk_rows_vec(D, elem) : chunk_rows(D);
      const int LCH = log2i(CH);
      const int n_chunks = (n_rows + CH - 1) / CH;
      if (n_chunks == 0) break;
      const bool more = top_blevel > base + LCH;
      float* tot = more ? bufs[pass & 1] : nullptr;
      const int tot_chunks = n_rows / CH;
      dim3 grid(n_chunks, B * H);
#define TA_LEVEL_PASS(KER, TT, ZF)                                                                                 \
  hipLaunchKernelGGL(KER, grid, dim3(256), 0, st, (const TT*)src, sb, sh, sr, H, n_rows, base, ZF, lo, tot, tot_chunks)
      if (pass == 0 && logt) {
        TA_LEVEL_PASS((level_pass_kernel<T, D, true>), T, zero_sink);
      } else if (pass == 0) {
        if (vec) TA_LEVEL_PASS((level_vec_kernel<T, D>), T, zero_sink);
        else TA_LEVEL_PASS((level_pass_kernel<T, D>), T, zero_sink);
      } else {
        if (vec) TA_LEVEL_PASS((level_vec_kernel<float, D>), float, 0);
        else TA_LEVEL_PASS((level_pass_kernel<float, D>), float, 0);
      }
#undef TA_LEVEL_PASS
      int rc = check_launch("level_pass_kernel");
      if (rc) return rc;
      if (!more) break;
      src = tot;
      sr = D;
      sh = (int64_t)tot_chunks * D;
      sb = sh * H;
      n_rows = tot_chunks;
      base += LCH;
      ++pass;
    }
    return TA_OK;
  }
};

template <typename T, int D>
struct DescendRun {
  static int run(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, int B, int H, int Nq, const int32_t* tq,
                 int64_t tq_sb, const LevelIn& lv, int n_levels, int Tgeo, int arity_log2, int wmax, int wl,
                 int32_t* ids, uint8_t* vld, float* sct, const AppendIn* ap, const LevelIn* alv,
                 const ta_leaf_store_out* so, const GateAppendIn* ga, hipStream_t st) {
    const int arity = 1 << arity_log2;
    const int cmax4 = (arity * wmax + arity - 1 + 3) & ~3;
    const int wmax4 = (wmax + 3) & ~3;
    // many queries (prefill): one wavefront per query, 4 per block; few (decode): four wavefronts per query;
    // very few (a single sequence): sixteen
    const int64_t nq_all = (int64_t)B * H * Nq;
    const int wpq = nq_all <= 256 ? 16 : (nq_all < 4096 ? 4 : 1);
    const bool wide = wpq > 1;
    const int qpb = wide ? 1 : 4;
    size_t lds = (size_t)qpb * (4 * cmax4 + 2 * wmax4) * sizeof(int32_t);
    if (ap) {
      if (!wide || Nq != 1) {
        set_error("descent with append: one query per (sequence, head) and fewer than 4096 of them");
        return TA_ERR_UNSUPPORTED;
      }
      lds += (size_t)16 * D * sizeof(float);   // the append's carry stack
    }
    if (lds > 64 * 1024) {
      set_error("descent beam too wide for LDS (arity * wmax too large)");
      return TA_ERR_UNSUPPORTED;
    }
    dim3 grid((Nq + qpb - 1) / qpb, B * H);
    const AppendIn none{};
    const ta_leaf_store_out no_store{};
    const GateAppendIn no_gate{};
#define TA_DESC(WPQ, NTH, APP, GT)                                                                                \
  hipLaunchKernelGGL((descend_kernel<T, D, WPQ, APP, GT>), grid, dim3(NTH), lds, st, (const T*)q, qsb, qsh, qsn, H, \
                     Nq, Tgeo, tq, tq_sb, lv, n_levels, arity_log2, wmax, wl, cmax4, ids, vld, sct,                  \
                     ap ? *ap : none, alv ? *alv : lv, so ? *so : no_store, ga ? *ga : no_gate)
    if (ap && ga) {
      if (wpq == 16) TA_DESC(16, 1024, true, true);
      else TA_DESC(4, 256, true, true);
    } else if (ap) {
      if (wpq == 16) TA_DESC(16, 1024, true, false);
      else TA_DESC(4, 256, true, false);
    } else {
      if (wpq == 16) TA_DESC(16, 1024, false, false);
      else if (wide) TA_DESC(4, 256, false, false);
      else TA_DESC(1, 256, false, false);
    }
#undef TA_DESC
    return check_launch("descend_kernel");
  }
};

template <typename TQ, int D>
struct GatherDotRun {
  template <typename TS>
  static int go(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* S, int64_t ssb, int64_t ssh,
                int64_t ssn, const int32_t* cand, const int32_t* blk, int block_log2, int NB_blk, int B, int H,
                int N, int M, int C, float scale, float* out, hipStream_t st) {
    dim3 grid((N + 3) / 4, B * H);
    hipLaunchKernelGGL((gather_dot_kernel<TQ, TS, D>), grid, dim3(256), 0, st, (const TQ*)q, qsb, qsh, qsn,
                       (const TS*)S, ssb, ssh, ssn, cand, blk, block_log2, NB_blk, H, N, M, C, scale, out);
    return check_launch("gather_dot_kernel");
  }
  static int run(int s_dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* S, int64_t ssb,
                 int64_t ssh, int64_t ssn, const int32_t* cand, const int32_t* blk, int block_log2, int NB_blk, int B,
                 int H, int N, int M, int C, float scale, float* out, hipStream_t st) {
    switch (s_dtype) {
      case TA_F32: return go<float>(q, qsb, qsh, qsn, S, ssb, ssh, ssn, cand, blk, block_log2, NB_blk, B, H, N, M, C, scale, out, st);
      case TA_F16: return go<f16_t>(q, qsb, qsh, qsn, S, ssb, ssh, ssn, cand, blk, block_log2, NB_blk, B, H, N, M, C, scale, out, st);
      case TA_BF16: return go<bf16_t>(q, qsb, qsh, qsn, S, ssb, ssh, ssn, cand, blk, block_log2, NB_blk, B, H, N, M, C, scale, out, st);
      default: set_error("unknown dtype"); return TA_ERR_ARG;
    }
  }
};

bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

int elem_size(int dt) { return dt == TA_F32 ? 4 : 2; }

// A row slice of R = D/16 elements per lane is read with loads of up to 16 bytes: the base and all row
// strides must keep that slice aligned.
bool rows_aligned(const void* p, int dt, int D, std::initializer_list<int64_t> strides) {
  int slice = (D / 16) * elem_size(dt);
  int a = slice >= 16 ? 16 : slice;
  if (!aligned(p, a)) return false;
  for (int64_t s : strides)
    if ((s * elem_size(dt)) % a) return false;
  return true;
}

}  // namespace
}  // namespace ta

using namespace ta;

extern "C" int64_t ta_level_sums_workspace_size(int B, int H, int t_end, int D) {
  if (D <= 0 || D > 256) return 0;
  int CH = chunk_rows(D);
  int64_t nA = ((int64_t)t_end / CH + 1) * B * H * D;
  int64_t nB = ((int64_t)t_end / CH / CH + 1) * B * H * D;
  return (nA + nB) * (int64_t)sizeof(float);
}

namespace {
int level_sums_impl(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int t_end,
                    int D, int zero_sink, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                    const int64_t* lv_sh, const int32_t* lv_blevel, float* ws, int64_t ws_bytes, void* stream,
                    bool logt);
}

extern "C" int ta_level_sums(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H,
                             int t_end, int D, int zero_sink, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                             const int64_t* lv_sh, const int32_t* lv_blevel, float* ws, int64_t ws_bytes,
                             void* stream) {
  return level_sums_impl(k, k_dtype, ksb, ksh, kst, B, H, t_end, D, zero_sink, n_levels, lv_ptr, lv_sb, lv_sh,
                         lv_blevel, ws, ws_bytes, stream, false);
}

extern "C" int ta_level_log_sums(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H,
                                 int t_end, int D, int zero_sink, int n_levels, float* const* lv_ptr,
                                 const int64_t* lv_sb, const int64_t* lv_sh, const int32_t* lv_blevel, float* ws,
                                 int64_t ws_bytes, void* stream) {
  return level_sums_impl(k, k_dtype, ksb, ksh, kst, B, H, t_end, D, zero_sink, n_levels, lv_ptr, lv_sb, lv_sh,
                         lv_blevel, ws, ws_bytes, stream, true);
}

namespace {
int level_sums_impl(const void* k, int k_dtype, int64_t ksb, int64_t ksh, int64_t kst, int B, int H, int t_end,
                    int D, int zero_sink, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                    const int64_t* lv_sh, const int32_t* lv_blevel, float* ws, int64_t ws_bytes, void* stream,
                    bool logt) {
  if (B <= 0 || H <= 0 || t_end < 0 || n_levels < 0 || n_levels > kMaxLevels) {
    set_error("ta_level_sums: bad sizes");
    return TA_ERR_ARG;
  }
  if (t_end == 0 || n_levels == 0) return TA_OK;
  LevelOut lo;
  for (int i = 0; i < 64; ++i) lo.slot_of_blevel[i] = -1;
  int prev = 0;
  for (int j = 0; j < n_levels; ++j) {
    if (lv_blevel[j] <= prev || lv_blevel[j] >= 63) {
      set_error("ta_level_sums: output levels must be increasing binary levels >= 1");
      return TA_ERR_ARG;
    }
    prev = lv_blevel[j];
    lo.ptr[j] = lv_ptr[j];
    lo.sb[j] = lv_sb[j];
    lo.sh[j] = lv_sh[j];
    lo.slot_of_blevel[lv_blevel[j]] = (int8_t)j;
  }
  if (ws_bytes < ta_level_sums_workspace_size(B, H, t_end, D)) {
    set_error("ta_level_sums: workspace too small");
    return TA_ERR_WORKSPACE;
  }
  return dispatch_dt_d<LevelSumsRun>(k_dtype, D, k, ksb, ksh, kst, B, H, t_end, zero_sink, lo, n_levels, prev, ws,
                                    (hipStream_t)stream, logt);
}
}  // namespace

namespace {
bool store_ok(const ta_leaf_store_out* so, int wl) {
  return so == nullptr || (so->leaf != nullptr && so->score != nullptr && so->ok != nullptr && so->Tst >= 0 &&
                           so->n >= 0 && so->n <= wl);
}

int tree_descend_impl(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, int B, int H, int Nq, int D,
                      const int32_t* tq, int64_t tq_sb, int n_levels, const float* const* lv_ptr,
                      const int64_t* lv_sb, const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax,
                      int wl, int32_t* ids, uint8_t* vld, float* sct, const ta_leaf_store_out* so, void* stream) {
  if (B <= 0 || H <= 0 || Nq < 0 || wmax < 1 || wl < 0 || n_levels < 0 || n_levels > kMaxLevels || !pow2(T) ||
      leaf_log2 < 1 || arity_log2 < 1 || !store_ok(so, wl)) {
    set_error("ta_tree_descend: bad sizes (or store: arrays missing, n > wl)");
    return TA_ERR_ARG;
  }
  if (Nq == 0) return TA_OK;
  if (!rows_aligned(q, q_dtype, D, {qsb, qsh, qsn})) {
    set_error("ta_tree_descend: q rows not aligned");
    return TA_ERR_ARG;
  }
  LevelIn lv;
  for (int j = 0; j < n_levels; ++j) {
    lv.ptr[j] = lv_ptr[j];
    lv.sb[j] = lv_sb[j];
    lv.sh[j] = lv_sh[j];
    lv.blevel[j] = leaf_log2 + j * arity_log2;
    if (!aligned(lv_ptr[j], 16)) {
      set_error("ta_tree_descend: level pointer not 16-byte aligned");
      return TA_ERR_ARG;
    }
  }
  return dispatch_dt_d<DescendRun>(q_dtype, D, q, qsb, qsh, qsn, B, H, Nq, tq, tq_sb, lv, n_levels, T, arity_log2,
                                   wmax, wl, ids, vld, sct, (const AppendIn*)nullptr, (const LevelIn*)nullptr, so,
                                   (const GateAppendIn*)nullptr, (hipStream_t)stream);
}

int tree_descend_append_impl(const void* q, int dtype, int64_t qsb, int64_t qsh, int B, int H, int D,
                             const int32_t* t_pos, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                             const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax, int wl,
                             int32_t* ids, uint8_t* vld, float* sct, const void* k_new, const void* v_new,
                             int64_t nsb, int64_t nsh, int64_t vnsb, int64_t vnsh, void* Kc, void* Vc, int64_t csb,
                             int64_t csh, int64_t cst, int Tcap, const ta_kv_pages* pages, float* const* app_ptr,
                             const int64_t* app_sb, const int64_t* app_sh, float* const* gate_lg,
                             float* const* gate_out, float gate_q, const ta_leaf_store_out* so, void* stream) {
  if (B <= 0 || H <= 0 || wmax < 1 || wl < 0 || n_levels < 0 || n_levels > kMaxLevels || !pow2(T) ||
      leaf_log2 < 1 || leaf_log2 > 14 || arity_log2 < 1 || arity_log2 > 4 || Tcap <= 0 || D > 256 ||
      !store_ok(so, wl)) {
    set_error("ta_tree_descend_append: bad sizes (or store: arrays missing, n > wl)");
    return TA_ERR_ARG;
  }
  if (!rows_aligned(q, dtype, D, {qsb, qsh})) {
    set_error("ta_tree_descend_append: q rows not aligned");
    return TA_ERR_ARG;
  }
  LevelIn lv;
  for (int j = 0; j < n_levels; ++j) {
    lv.ptr[j] = lv_ptr[j];
    lv.sb[j] = lv_sb[j];
    lv.sh[j] = lv_sh[j];
    lv.blevel[j] = leaf_log2 + j * arity_log2;
    if (!aligned(lv_ptr[j], 16)) {
      set_error("ta_tree_descend_append: level pointer not 16-byte aligned");
      return TA_ERR_ARG;
    }
  }
  if (n_levels == 0) lv.blevel[0] = leaf_log2;
  AppendIn ap{k_new, v_new, nsb, nsh, vnsb, vnsh, Kc, Vc, csb, csh, cst, Tcap};
  if (pages) {
    if (pages->table == nullptr || pages->block_log2 != leaf_log2 || pages->num_pages <= 0 ||
        pages->page_stride < ((int64_t)cst << leaf_log2)) {
      set_error("ta_tree_descend_append: bad page description (block must be the leaf block)");
      return TA_ERR_ARG;
    }
    ap.ptab = pages->table;
    ap.pt_sb = pages->sb;
    ap.pt_sh = pages->sh;
    ap.pstride = pages->page_stride;
    ap.npages = pages->num_pages;
  }
  // the levels the append forms nodes in: the scored ones unless given apart (gated levels are scored from
  // their gated vectors while the append forms the raw sums)
  LevelIn alv = lv;
  if (app_ptr != nullptr) {
    for (int j = 0; j < n_levels; ++j) {
      alv.ptr[j] = app_ptr[j];
      alv.sb[j] = app_sb[j];
      alv.sh[j] = app_sh[j];
      if (!aligned(app_ptr[j], 16)) {
        set_error("ta_tree_descend_append: append level pointer not 16-byte aligned");
        return TA_ERR_ARG;
      }
    }
  }
  // the gate's log sums and gated vectors of the nodes the append completes (the leaf level log-summed even
  // when no level is gated)
  GateAppendIn ga{};
  if (gate_lg != nullptr) {
    if (n_levels == 0 || !(gate_q >= 0.0f && gate_q <= 1.0f) || leaf_log2 > 14 || D > 128) {
      set_error("ta_tree_descend_append_ex: gate needs levels, gate_q in [0, 1], leaf <= 2^14, D <= 128");
      return TA_ERR_ARG;
    }
    for (int j = 0; j < n_levels; ++j) {
      ga.lg[j] = gate_lg[j];
      ga.out[j] = gate_out != nullptr ? gate_out[j] : nullptr;
      if (ga.lg[j] == nullptr) {
        set_error("ta_tree_descend_append_ex: a log-sum level is missing");
        return TA_ERR_ARG;
      }
    }
    gate_rank(gate_q, D, ga.lo, ga.w);
  }
  return dispatch_dt_d<DescendRun>(dtype, D, q, qsb, qsh, (int64_t)0, B, H, 1, t_pos, (int64_t)1, lv, n_levels, T,
                                   arity_log2, wmax, wl, ids, vld, sct, (const AppendIn*)&ap, (const LevelIn*)&alv,
                                   so, gate_lg != nullptr ? &ga : (const GateAppendIn*)nullptr, (hipStream_t)stream);
}
}  // namespace

extern "C" int ta_tree_descend(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, int B, int H,
                               int Nq, int D, const int32_t* tq, int64_t tq_sb, int n_levels,
                               const float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh, int T,
                               int leaf_log2, int arity_log2, int wmax, int wl, int32_t* ids, uint8_t* vld,
                               float* sct, void* stream) {
  return tree_descend_impl(q, q_dtype, qsb, qsh, qsn, B, H, Nq, D, tq, tq_sb, n_levels, lv_ptr, lv_sb, lv_sh, T,
                           leaf_log2, arity_log2, wmax, wl, ids, vld, sct, nullptr, stream);
}

extern "C" int ta_tree_descend_store(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, int B, int H,
                                     int Nq, int D, const int32_t* tq, int64_t tq_sb, int n_levels,
                                     const float* const* lv_ptr, const int64_t* lv_sb, const int64_t* lv_sh, int T,
                                     int leaf_log2, int arity_log2, int wmax, int wl, int32_t* ids, uint8_t* vld,
                                     float* sct, const ta_leaf_store_out* store, void* stream) {
  if (store == nullptr) {
    set_error("ta_tree_descend_store: store missing");
    return TA_ERR_ARG;
  }
  return tree_descend_impl(q, q_dtype, qsb, qsh, qsn, B, H, Nq, D, tq, tq_sb, n_levels, lv_ptr, lv_sb, lv_sh, T,
                           leaf_log2, arity_log2, wmax, wl, ids, vld, sct, store, stream);
}

extern "C" int ta_tree_descend_append(const void* q, int dtype, int64_t qsb, int64_t qsh, int B, int H, int D,
                                      const int32_t* t_pos, int n_levels, float* const* lv_ptr,
                                      const int64_t* lv_sb, const int64_t* lv_sh, int T, int leaf_log2,
                                      int arity_log2, int wmax, int wl, int32_t* ids, uint8_t* vld, float* sct,
                                      const void* k_new, const void* v_new, int64_t nsb, int64_t nsh, int64_t vnsb,
                                      int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst,
                                      int Tcap, const ta_kv_pages* pages, void* stream) {
  return tree_descend_append_impl(q, dtype, qsb, qsh, B, H, D, t_pos, n_levels, lv_ptr, lv_sb, lv_sh, T, leaf_log2,
                                  arity_log2, wmax, wl, ids, vld, sct, k_new, v_new, nsb, nsh, vnsb, vnsh, Kc, Vc,
                                  csb, csh, cst, Tcap, pages, nullptr, nullptr, nullptr, nullptr, nullptr, 0.0f,
                                  nullptr, stream);
}

extern "C" int ta_tree_descend_append_ex(const void* q, int dtype, int64_t qsb, int64_t qsh, int B, int H, int D,
                                         const int32_t* t_pos, int n_levels, float* const* lv_ptr,
                                         const int64_t* lv_sb, const int64_t* lv_sh, int T, int leaf_log2,
                                         int arity_log2, int wmax, int wl, int32_t* ids, uint8_t* vld, float* sct,
                                         const void* k_new, const void* v_new, int64_t nsb, int64_t nsh, int64_t vnsb,
                                         int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst,
                                         int Tcap, const ta_kv_pages* pages, float* const* app_lv_ptr,
                                         const int64_t* app_lv_sb, const int64_t* app_lv_sh, float* const* gate_lg,
                                         float* const* gate_out, float gate_q, const ta_leaf_store_out* store,
                                         void* stream) {
  return tree_descend_append_impl(q, dtype, qsb, qsh, B, H, D, t_pos, n_levels, lv_ptr, lv_sb, lv_sh, T, leaf_log2,
                                  arity_log2, wmax, wl, ids, vld, sct, k_new, v_new, nsb, nsh, vnsb, vnsh, Kc, Vc,
                                  csb, csh, cst, Tcap, pages, app_lv_ptr, app_lv_sb, app_lv_sh, gate_lg, gate_out,
                                  gate_q, store, stream);
}

extern "C" int ta_gather_dot(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, const void* S,
                             int s_dtype, int64_t ssb, int64_t ssh, int64_t ssn, const int32_t* cand, int B, int H,
                             int N, int M, int C, int D, float scale, float* out, void* stream) {
  if (B <= 0 || H <= 0 || N < 0 || M <= 0 || C < 0) {
    set_error("ta_gather_dot: bad sizes");
    return TA_ERR_ARG;
  }
  if (N == 0 || C == 0) return TA_OK;
  if (!rows_aligned(q, q_dtype, D, {qsb, qsh, qsn}) || !rows_aligned(S, s_dtype, D, {ssb, ssh, ssn})) {
    set_error("ta_gather_dot: rows not aligned");
    return TA_ERR_ARG;
  }
  return dispatch_dt_d<GatherDotRun>(q_dtype, D, s_dtype, q, qsb, qsh, qsn, S, ssb, ssh, ssn, cand,
                                     (const int32_t*)nullptr, 0, 0, B, H, N, M, C, scale, out, (hipStream_t)stream);
}

extern "C" int ta_gather_dot_blocks(const void* q, const void* K, int dtype, int64_t qsb, int64_t qsh, int64_t qsn,
                                    int64_t ksb, int64_t ksh, int64_t ksn, const int32_t* blk, int B, int H, int N,
                                    int M, int NB, int block, int D, float scale, float* out, void* stream) {
  if (B <= 0 || H <= 0 || N < 0 || M <= 0 || NB < 0 || !pow2(block)) {
    set_error("ta_gather_dot_blocks: bad sizes");
    return TA_ERR_ARG;
  }
  if (N == 0 || NB == 0) return TA_OK;
  if (!rows_aligned(q, dtype, D, {qsb, qsh, qsn}) || !rows_aligned(K, dtype, D, {ksb, ksh, ksn})) {
    set_error("ta_gather_dot_blocks: rows not aligned");
    return TA_ERR_ARG;
  }
  const int rc = gather_blocks_mfma(q, K, dtype, qsb, qsh, qsn, ksb, ksh, ksn, blk, B, H, N, M, NB, block, D, scale,
                                    out, stream);
  if (rc != TA_ERR_UNSUPPORTED) return rc;
  return dispatch_dt_d<GatherDotRun>(dtype, D, dtype, q, qsb, qsh, qsn, K, ksb, ksh, ksn, (const int32_t*)nullptr, blk,
                                     log2i(block), NB, B, H, N, M, NB * block, scale, out, (hipStream_t)stream);
}

TA_TRACE_EXPORTS
