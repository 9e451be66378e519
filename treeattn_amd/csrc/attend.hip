// Sparse softmax attention on gfx950 over the keys a query selected, and the decode-cache append.
//
// One wavefront per (query, split).  The query's keys are enumerated as a flat list (selected leaf blocks,
// the own partial leaf block, the static keys not already covered -- or an explicit candidate list); a
// chunk of the list maps one key to each lane (two lanes per key when D = 128).  Each lane reads its key's
// K and V rows (a leaf block is a run of consecutive rows, so a chunk reads contiguous memory), keeps a
// running max/sum (online softmax, float32) and its own weighted V accumulator; the wavefront reduces
// the accumulators once at the end (reduce-scatter over lanes).  With nsplit > 1 the partial (max, sum,
// accumulator) of every split goes to a workspace; the split that finishes last for a query (a per-query
// arrival counter, reset by that split) merges them, so one launch does the whole attention.
//
// Reference functions replaced: fastseg.py:50-78 (_attn_fwd), fastseg.py:134-177 (sparse_attn),
// fastseg.py:367-383 (candidate assembly + dedupe_fast), engine.py:107-119 (decode attention),
// engine.py:41-55 (SegState.add).
#include <utility>

#include "common.hpp"

namespace ta {

struct AttnParams {
  const void* q;
  int64_t qsb, qsh, qsn;
  const void* k;
  int64_t ksb, ksh, kst;
  const void* v;
  int64_t vsb, vsh, vst;
  int H, Nq, Tk;
  const int32_t* tq;
  int64_t tq_sb;
  const int32_t* cand;  // explicit candidate list mode when non-null
  int KC;
  const int32_t* ids;
  const uint8_t* vld;
  const int32_t* n_tree;
  int wl, leaf_log2, Lw;
  float scale;
  int nsplit;
  void* out;
  int64_t osb, osh, osn;
  float* lse;
  float* keys;
  float* ws;           // partials (query, split, D + 2)
  unsigned* cnt;       // per-query arrival counters, zero between launches
};

constexpr float kNegBig = -1e30f;

// Sum acc[DPL] over the lanes that share (lane % LPK); afterwards lane holds E = result length values of
// dims [dim0, dim0 + E) of its LPK-slice.  Lanes whose `dup` bits are set hold duplicate results.
template <int DPL, int LPK>
struct LaneReduce {
  static constexpr int steps_halve() {
    int len = DPL, n = 0;
    for (int o = 32; o >= LPK; o >>= 1)
      if (len > 1) { len >>= 1; ++n; }
    return n;
  }
  static constexpr int E = DPL >> steps_halve();
  static constexpr int dup_mask() {
    int len = DPL, m = 0;
    for (int o = 32; o >= LPK; o >>= 1) {
      if (len > 1) len >>= 1; else m |= o;
    }
    return m;
  }
  __device__ static int run(float (&acc)[DPL], int lane) {
    int dim0 = 0;
    int len = DPL;
#pragma unroll
    for (int o = 32; o >= LPK; o >>= 1) {
      if (len > 1) {
        const int half = len >> 1;
        const bool up = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < DPL / 2; ++i) {
          if (i < half) {
            const float mine = up ? acc[i + half] : acc[i];
            const float other = up ? acc[i] : acc[i + half];
            acc[i] = mine + __shfl_xor(other, o, kWave);
          }
        }
        if (up) dim0 += half;
        len = half;
      } else {
        acc[0] += __shfl_xor(acc[0], o, kWave);
      }
    }
    return dim0;
  }
};

// SPLIT: several wavefronts per query with the in-kernel merge (decode); otherwise one wavefront per query.
template <typename T, int D, bool SPLIT>
__global__ __launch_bounds__(256) void attn_kernel(AttnParams p) {
  constexpr int LPK = D > 64 ? D / 64 : 1;  // lanes per key
  constexpr int DPL = D / LPK;              // dims per lane
  constexpr int KPC = kWave / LPK;          // keys per chunk
  using Red = LaneReduce<DPL, LPK>;
  extern __shared__ float smem_f[];
  const int lane = lane_id(), w = wave_id();
  const int wi = blockIdx.x * (blockDim.x / kWave) + w;
  const int n = wi / p.nsplit, split = wi % p.nsplit;
  if (n >= p.Nq) return;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int64_t qi = (int64_t)bh * p.Nq + n;
  const int wl_pad = p.cand ? 0 : ((p.wl + 3) & ~3);
  float* qf = smem_f + w * (D + wl_pad + kWave);
  int32_t* s_ids = reinterpret_cast<int32_t*>(qf + D);
  int32_t* s_ext = s_ids + wl_pad;

  // query row -> LDS (float32)
  {
    const T* qr = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + n * p.qsn;
    for (int d = lane; d < D; d += kWave) qf[d] = to_f32(qr[d]);
  }

  // key list of this query
  int N, nused = 0, lb = 0, nloc = 0, nseg = 0;
  const int leaf = 1 << p.leaf_log2;
  if (p.cand) {
    N = p.KC;
  } else {
    int t = p.tq[b * p.tq_sb + n];
    if (t >= p.Tk) t = -1;  // out of range: attend nothing
    const int32_t* idr = p.ids + qi * p.wl;
    const uint8_t* vr = p.vld + qi * p.wl;
    int nv = 0;
    for (int i0 = 0; i0 < p.wl; i0 += kWave) {
      const int i = i0 + lane;
      const bool v = i < p.wl && vr[i] != 0;
      nv += __popcll(__ballot(v));
    }
    const int nt = p.n_tree ? p.n_tree[qi] : p.wl;
    nused = t < 0 ? 0 : (nv < nt ? nv : (nt > 0 ? nt : 0));
    for (int i = lane; i < nused; i += kWave) s_ids[i] = idr[i];
    lb = t < 0 ? 0 : (t >> p.leaf_log2) << p.leaf_log2;
    nloc = t < 0 ? 0 : t - lb + 1;
    wave_sync();
    // static keys [0, t, t-1, ..., t-Lw+1]: keep those >= 0, outside the own block, whose leaf block is
    // not used, and not a repeat of the sink
    int pe = -1;
    if (lane <= p.Lw && t >= 0) pe = lane == 0 ? 0 : t - (lane - 1);
    bool keep = pe >= 0 && pe < lb && !(lane > 0 && pe == 0);
    if (keep) {
      const int lf = pe >> p.leaf_log2;
      for (int i = 0; i < nused; ++i)
        if (s_ids[i] == lf) keep = false;
    }
    const uint64_t bal = __ballot(keep);
    if (keep) s_ext[__popcll(bal & ((1ull << lane) - 1))] = pe;
    nseg = __popcll(bal);
    N = nused * leaf + nloc + nseg;
  }
  wave_sync();

  const T* kb = reinterpret_cast<const T*>(p.k) + b * p.ksb + h * p.ksh;
  const T* vb = reinterpret_cast<const T*>(p.v) + b * p.vsb + h * p.vsh;
  const int kl = lane / LPK;        // key slot of this lane inside a chunk
  const int part = lane % LPK;      // dim slice of this lane
  const int nchunks = (N + KPC - 1) / KPC;
  const int nl = nused * leaf;

  float m = kNegBig, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;

  for (int c = split; c < nchunks; c += p.nsplit) {
    const int key = c * KPC + kl;
    int pos = -1;
    if (key < N) {
      if (p.cand) {
        pos = p.cand[qi * p.KC + key];
      } else if (key < nl) {
        pos = (s_ids[key >> p.leaf_log2] << p.leaf_log2) + (key & (leaf - 1));
      } else if (key < nl + nloc) {
        pos = lb + (key - nl);
      } else {
        pos = s_ext[key - nl - nloc];
      }
    }
    const bool valid = pos >= 0 && pos < p.Tk;
    const int64_t row = valid ? pos : 0;
    float kv[DPL];
    load_row<T, DPL>(kb + row * p.kst + part * DPL, kv);
    float vv[DPL];
    load_row<T, DPL>(vb + row * p.vst + part * DPL, vv);
    float dot = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; ++d) dot = fmaf(qf[part * DPL + d], kv[d], dot);
    if constexpr (LPK == 2) dot += __shfl_xor(dot, 1, kWave);
    const float sc = valid ? dot * p.scale : kNegBig;
    const float mn = fmaxf(m, wave_max(sc));
    const float pw = valid ? __expf(sc - mn) : 0.0f;
    if (mn != m) {
      const float alpha = __expf(m - mn);
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] *= alpha;
      l *= alpha;
    }
#pragma unroll
    for (int d = 0; d < DPL; ++d) acc[d] = fmaf(pw, vv[d], acc[d]);
    if (part == 0) l += pw;
    m = mn;
  }

  const float L = wave_sum(l);
  const int dim0 = Red::run(acc, lane) + part * DPL;
  const bool writer = (lane & Red::dup_mask()) == 0;
  if constexpr (!SPLIT) {
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (writer) {
      T* orow = reinterpret_cast<T*>(p.out) + b * p.osb + h * p.osh + n * p.osn;
#pragma unroll
      for (int e = 0; e < Red::E; ++e) orow[dim0 + e] = from_f32<T>(acc[e] * inv);
    }
    if (lane == 0) {
      if (p.lse) p.lse[qi] = L > 0.0f ? m + __logf(L) : kNegBig;
      if (p.keys) p.keys[qi] = (float)N;
    }
  } else {
    float* part_ws = p.ws + (qi * p.nsplit + split) * (D + 2);
    if (writer) {
#pragma unroll
      for (int e = 0; e < Red::E; ++e) part_ws[2 + dim0 + e] = acc[e];
    }
    if (lane == 0) {
      part_ws[0] = m;
      part_ws[1] = L;
      if (split == 0 && p.keys) p.keys[qi] = (float)N;
    }
    // publish the partial, count arrivals; the last split of this query merges all of them
    __threadfence();
    int last = 0;
    if (lane == 0) last = atomicAdd(p.cnt + qi, 1u) == (unsigned)(p.nsplit - 1);
    last = __shfl(last, 0, kWave);
    if (!last) return;
    __threadfence();
    const float* base = p.ws + qi * p.nsplit * (D + 2);
    float M = kNegBig;
    for (int s = 0; s < p.nsplit; ++s) {
      const float* ps = base + s * (D + 2);
      if (ps[1] > 0.0f) M = fmaxf(M, ps[0]);
    }
    float Lt = 0.0f;
    for (int s = 0; s < p.nsplit; ++s) {
      const float* ps = base + s * (D + 2);
      if (ps[1] > 0.0f) Lt += ps[1] * __expf(ps[0] - M);
    }
    const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
    T* orow = reinterpret_cast<T*>(p.out) + b * p.osb + h * p.osh + n * p.osn;
    for (int d = lane; d < D; d += kWave) {
      float a = 0.0f;
      for (int s = 0; s < p.nsplit; ++s) {
        const float* ps = base + s * (D + 2);
        if (ps[1] > 0.0f) a += ps[2 + d] * __expf(ps[0] - M);
      }
      orow[d] = from_f32<T>(a * inv);
    }
    if (lane == 0) {
      if (p.lse) p.lse[qi] = Lt > 0.0f ? M + __logf(Lt) : kNegBig;
      p.cnt[qi] = 0u;  // ready for the next launch
    }
  }
}

// ----------------------------------------------------------------------------------------- decode append
struct LevelRW {
  float* ptr[kMaxLevels];
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
};

// One thread per dimension of one (sequence, head).  Writes row t of K and V, then forms the nodes whose
// last position is t: the leaf block from its keys, each higher node from its children, both as
// adjacent-pair sums (carry stack in LDS, one column per thread).
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T* __restrict__ kn, const T* __restrict__ vn,
                                                        int64_t nsb, int64_t nsh, int64_t vnsb, int64_t vnsh,
                                                        T* __restrict__ Kc, T* __restrict__ Vc, int64_t csb,
                                                        int64_t csh, int64_t cst, int H, int D, int Tcap,
                                                        const int32_t* __restrict__ t_pos, LevelRW lv, int n_levels,
                                                        int leaf_log2, int arity_log2) {
  extern __shared__ float stk[];  // [16][D]
  const int d = threadIdx.x;
  if (d >= D) return;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int t = t_pos[b];
  if (t < 0 || t >= Tcap) return;
  T* krow = Kc + b * csb + h * csh;
  T* vrow = Vc + b * csb + h * csh;
  const T kx = kn[b * nsb + h * nsh + d];
  krow[(int64_t)t * cst + d] = kx;
  vrow[(int64_t)t * cst + d] = vn[b * vnsb + h * vnsh + d];
  if (n_levels == 0) return;
  const int leaf = 1 << leaf_log2;
  if (((t + 1) & (leaf - 1)) != 0) return;
  // leaf block [t+1-leaf, t]
  const int p0 = t + 1 - leaf;
  float x = 0.0f;
  for (int i = 0; i < leaf; ++i) {
    const int pp = p0 + i;
    x = pp == 0 ? 0.0f : (pp == t ? to_f32(kx) : to_f32(krow[(int64_t)pp * cst + d]));
    int lvl = 0;
    while ((i >> lvl) & 1) {
      x = __fadd_rn(stk[lvl * D + d], x);
      ++lvl;
    }
    stk[lvl * D + d] = x;
  }
  float* base0 = lv.ptr[0] + b * lv.sb[0] + h * lv.sh[0];
  base0[(int64_t)(t >> leaf_log2) * D + d] = x;
  const int arity = 1 << arity_log2;
  for (int j = 1; j < n_levels; ++j) {
    const int lj = leaf_log2 + j * arity_log2;
    if (((t + 1) & ((1 << lj) - 1)) != 0) break;
    const int64_t node = t >> lj;
    const float* child = lv.ptr[j - 1] + b * lv.sb[j - 1] + h * lv.sh[j - 1] + node * arity * D + d;
    for (int c = 0; c < arity; ++c) {
      x = child[(int64_t)c * D];
      int lvl = 0;
      while ((c >> lvl) & 1) {
        x = __fadd_rn(stk[lvl * D + d], x);
        ++lvl;
      }
      stk[lvl * D + d] = x;
    }
    lv.ptr[j][b * lv.sb[j] + h * lv.sh[j] + node * D + d] = x;
  }
}

// ----------------------------------------------------------------------------------------- host side
namespace {

int elem_size(int dt) { return dt == TA_F32 ? 4 : 2; }
bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// K/V rows are read D/LPK elements per lane with loads of up to 16 bytes.
bool kv_aligned(const void* p, int dt, int D, std::initializer_list<int64_t> strides) {
  const int LPK = D > 64 ? D / 64 : 1;
  int slice = (D / LPK) * elem_size(dt);
  int a = slice >= 16 ? 16 : slice;
  if (!aligned(p, a)) return false;
  for (int64_t s : strides)
    if ((s * elem_size(dt)) % a) return false;
  return true;
}

template <typename T, int D>
int launch_attn(const AttnParams& p, int B, hipStream_t st) {
  const int waves = 4;
  const int wl_pad = p.cand ? 0 : ((p.wl + 3) & ~3);
  const size_t lds = (size_t)waves * (D + wl_pad + kWave) * sizeof(float);
  const int64_t nw = (int64_t)p.Nq * p.nsplit;
  dim3 grid((unsigned)((nw + waves - 1) / waves), B * p.H);
  if (p.nsplit > 1) {
    hipLaunchKernelGGL((attn_kernel<T, D, true>), grid, dim3(waves * kWave), lds, st, p);
  } else {
    hipLaunchKernelGGL((attn_kernel<T, D, false>), grid, dim3(waves * kWave), lds, st, p);
  }
  return check_launch("attn_kernel");
}

int dispatch_attn(int dt, int D, const AttnParams& p, int B, hipStream_t st) {
#define TA_CASE_D(T)                                      \
  switch (D) {                                            \
    case 16: return launch_attn<T, 16>(p, B, st);         \
    case 32: return launch_attn<T, 32>(p, B, st);         \
    case 64: return launch_attn<T, 64>(p, B, st);         \
    case 128: return launch_attn<T, 128>(p, B, st);       \
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

}  // namespace
}  // namespace ta

using namespace ta;

extern "C" int ta_sparse_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                                  int64_t qst, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                                  int64_t vst, const int32_t* cand, int B, int H, int T, int Tk, int KC, int D,
                                  float scale, void* out, float* lse, void* stream) {
  if (B <= 0 || H <= 0 || T < 0 || Tk < 0 || KC < 0) {
    set_error("ta_sparse_attn_fwd: bad sizes");
    return TA_ERR_ARG;
  }
  if (T == 0) return TA_OK;
  if (!kv_aligned(k, dtype, D, {ksb, ksh, kst}) || !kv_aligned(v, dtype, D, {vsb, vsh, vst})) {
    set_error("ta_sparse_attn_fwd: k/v rows not aligned");
    return TA_ERR_ARG;
  }
  AttnParams p{};
  p.q = q; p.qsb = qsb; p.qsh = qsh; p.qsn = qst;
  p.k = k; p.ksb = ksb; p.ksh = ksh; p.kst = kst;
  p.v = v; p.vsb = vsb; p.vsh = vsh; p.vst = vst;
  p.H = H; p.Nq = T; p.Tk = Tk;
  p.cand = cand; p.KC = KC;
  p.leaf_log2 = 1;
  p.scale = scale;
  p.nsplit = 1;
  p.out = out; p.osb = (int64_t)H * T * D; p.osh = (int64_t)T * D; p.osn = D;
  p.lse = lse;
  return dispatch_attn(dtype, D, p, B, (hipStream_t)stream);
}

static int64_t counter_bytes(int B, int H, int Nq) { return (((int64_t)B * H * Nq * 4) + 255) / 256 * 256; }

extern "C" int64_t ta_seg_attn_workspace_size(int B, int H, int Nq, int D, int nsplit) {
  if (nsplit <= 1) return 0;
  return counter_bytes(B, H, Nq) + (int64_t)B * H * Nq * nsplit * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int ta_seg_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                               int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                               int64_t vst, int B, int H, int Nq, int D, int Tk, const int32_t* tq, int64_t tq_sb,
                               const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl, int leaf,
                               int local, float scale, void* out, int64_t osb, int64_t osh, int64_t osn, float* lse,
                               float* keys, int nsplit, float* ws, int64_t ws_bytes, void* stream) {
  if (B <= 0 || H <= 0 || Nq < 0 || wl < 0 || nsplit < 1 || leaf < 2 || (leaf & (leaf - 1))) {
    set_error("ta_seg_attn_fwd: bad sizes");
    return TA_ERR_ARG;
  }
  const int Lw = local > 3 ? local : 3;
  if (Lw + 1 > kWave) {
    set_error("ta_seg_attn_fwd: local window must be < 64");
    return TA_ERR_UNSUPPORTED;
  }
  if (wl > 1024) {
    set_error("ta_seg_attn_fwd: beam wider than 1024 leaves");
    return TA_ERR_UNSUPPORTED;
  }
  if (Nq == 0) return TA_OK;
  if (nsplit > 1 && ws_bytes < ta_seg_attn_workspace_size(B, H, Nq, D, nsplit)) {
    set_error("ta_seg_attn_fwd: workspace too small");
    return TA_ERR_WORKSPACE;
  }
  if (!kv_aligned(k, dtype, D, {ksb, ksh, kst}) || !kv_aligned(v, dtype, D, {vsb, vsh, vst})) {
    set_error("ta_seg_attn_fwd: k/v rows not aligned");
    return TA_ERR_ARG;
  }
  AttnParams p{};
  p.q = q; p.qsb = qsb; p.qsh = qsh; p.qsn = qsn;
  p.k = k; p.ksb = ksb; p.ksh = ksh; p.kst = kst;
  p.v = v; p.vsb = vsb; p.vsh = vsh; p.vst = vst;
  p.H = H; p.Nq = Nq; p.Tk = Tk;
  p.tq = tq; p.tq_sb = tq_sb;
  p.ids = ids; p.vld = vld; p.n_tree = n_tree; p.wl = wl;
  int ll = 0;
  while ((1 << ll) < leaf) ++ll;
  p.leaf_log2 = ll;
  p.Lw = Lw;
  p.scale = scale;
  p.nsplit = nsplit;
  p.out = out; p.osb = osb; p.osh = osh; p.osn = osn;
  p.lse = lse; p.keys = keys;
  if (nsplit > 1) {
    p.cnt = reinterpret_cast<unsigned*>(ws);
    p.ws = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + counter_bytes(B, H, Nq));
  }
  return dispatch_attn(dtype, D, p, B, (hipStream_t)stream);
}

extern "C" int ta_kv_append(const void* k_new, const void* v_new, int dtype, int64_t nsb, int64_t nsh, int64_t vnsb,
                            int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst, int B, int H,
                            int D, int Tcap, const int32_t* t_pos, int n_levels, float* const* lv_ptr,
                            const int64_t* lv_sb, const int64_t* lv_sh, int leaf_log2, int arity_log2,
                            void* stream) {
  if (B <= 0 || H <= 0 || D <= 0 || D > 256 || n_levels < 0 || n_levels > kMaxLevels || leaf_log2 < 1 ||
      leaf_log2 > 14 || arity_log2 < 1 || arity_log2 > 4) {
    set_error("ta_kv_append: bad sizes");
    return TA_ERR_ARG;
  }
  LevelRW lv;
  for (int j = 0; j < n_levels; ++j) {
    lv.ptr[j] = lv_ptr[j];
    lv.sb[j] = lv_sb[j];
    lv.sh[j] = lv_sh[j];
  }
  const size_t lds = (size_t)16 * D * sizeof(float);
  dim3 grid(B * H);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL((kv_append_kernel<float>), grid, dim3(D), lds, st, (const float*)k_new, (const float*)v_new,
                         nsb, nsh, vnsb, vnsh, (float*)Kc, (float*)Vc, csb, csh, cst, H, D, Tcap, t_pos, lv, n_levels,
                         leaf_log2, arity_log2);
      break;
    case TA_F16:
      hipLaunchKernelGGL((kv_append_kernel<f16_t>), grid, dim3(D), lds, st, (const f16_t*)k_new, (const f16_t*)v_new,
                         nsb, nsh, vnsb, vnsh, (f16_t*)Kc, (f16_t*)Vc, csb, csh, cst, H, D, Tcap, t_pos, lv, n_levels,
                         leaf_log2, arity_log2);
      break;
    case TA_BF16:
      hipLaunchKernelGGL((kv_append_kernel<bf16_t>), grid, dim3(D), lds, st, (const bf16_t*)k_new,
                         (const bf16_t*)v_new, nsb, nsh, vnsb, vnsh, (bf16_t*)Kc, (bf16_t*)Vc, csb, csh, cst, H, D,
                         Tcap, t_pos, lv, n_levels, leaf_log2, arity_log2);
      break;
    default:
      set_error("unknown dtype");
      return TA_ERR_ARG;
  }
  return check_launch("kv_append_kernel");
}
