// Sparse softmax attention on gfx950 over the keys a query selected, and the decode-cache append.
//
// One wavefront per (query, split).  The query's keys are enumerated as a flat list (selected leaf blocks,
// the own partial leaf block, the static keys not already covered -- or an explicit candidate list); a
// chunk of the list maps one key to each lane (two lanes per key when D = 128).  Each lane reads its key's
// K and V rows (a leaf block is a run of consecutive rows, so a chunk reads contiguous memory), keeps a
// running max/sum (online softmax, float32) and its own weighted V accumulator; the wavefront reduces
// the accumulators once at the end.  In split mode (few queries with many keys, as in decode) the four
// wavefronts of a workgroup share a query and merge in LDS; with more workgroups per query each writes its
// partial through to memory and the last of them to arrive (counted with a device-wide atomic) merges the
// partials and writes the output.
//
// Reference functions replaced: fastseg.py:50-78 (_attn_fwd), fastseg.py:134-177 (sparse_attn),
// fastseg.py:367-383 (candidate assembly + dedupe_fast), engine.py:107-119 (decode attention),
// engine.py:41-55 (SegState.add).
#include <utility>

#include "append.hpp"
#include "attend_query.hpp"
#include "attn.hpp"
#include "common.hpp"
#include "descend.hpp"

namespace ta {



// PIPE: the copy-free chunk loop of attn_query, for several workgroups per query (p.gsplit > 1).
template <typename T, int D, bool SPLIT, bool CAND, bool PIPE = false>
__global__ __launch_bounds__(256) void attn_kernel(AttnParams p) {
  extern __shared__ float smem_f[];
  const int w = wave_id();
  int n, g = 0;
  if constexpr (SPLIT) {
    n = blockIdx.x / p.gsplit;
    g = blockIdx.x % p.gsplit;
  } else {
    n = blockIdx.x * kWavesPerBlock + w;
  }
  if (n >= p.Nq) return;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int64_t qi = (int64_t)bh * p.Nq + n;
  const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + n * p.qsn;
  T* orow = reinterpret_cast<T*>(p.out) + b * p.osb + h * p.osh + n * p.osn;
  int t = 0, nt = 0;
  const int32_t* idr = nullptr;
  const uint8_t* vr = nullptr;
  if constexpr (!CAND) {
    t = p.tq[b * p.tq_sb + n];
    idr = p.ids + qi * p.wl;
    vr = p.vld + qi * p.wl;
    nt = p.n_tree ? p.n_tree[qi] : p.wl;
  }
  attn_query<T, D, SPLIT, CAND, PIPE>(p, n, g, b, h, qi, qrow, t, idr, vr, -1, nt, orow, smem_f);
}

// ----------------------------------------------------------------------------------------- decode attend
// One decode position per (sequence, head), everything in one workgroup of four wavefronts: the cache
// append of row t (and the nodes it completes), the beam descent (which reads only nodes ending before t),
// then the attention over the kept leaf blocks, the own block and the static keys.  The kept leaves stay in
// LDS; the selection is also written to ids / vld / sct as the descent kernel writes it.  Same device
// functions as the separate kernels, so the results equal ta_tree_descend_append followed by
// ta_seg_attn_fwd with one workgroup per query, bit for bit.
template <typename T, int D>
__global__ __launch_bounds__(kWavesPerBlock * kWave) void seg_attend_kernel(AttnParams p, LevelIn lv, int n_levels,
                                                                           int arity_log2, int Tgeo, int wmax,
                                                                           int cmax4, int32_t* __restrict__ ids,
                                                                           uint8_t* __restrict__ vld,
                                                                           float* __restrict__ sct, AppendIn ap) {
  extern __shared__ __align__(16) char sa_lds[];
  constexpr int NT = kWavesPerBlock * kWave;
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const int wmax4 = (wmax + 3) & ~3;
  uint64_t* ckey = reinterpret_cast<uint64_t*>(sa_lds);
  int32_t* cid = reinterpret_cast<int32_t*>(ckey + cmax4);
  float* csc = reinterpret_cast<float*>(cid + cmax4);
  int32_t* kid = cid + 2 * cmax4;
  float* ksc = reinterpret_cast<float*>(kid + wmax4);
  int32_t* kpg = reinterpret_cast<int32_t*>(ksc + wmax4);   // pages of the kept leaves (paged caches)
  int32_t* cpg = kpg + wmax4;                                // pages of the leaf-level candidates
  int32_t* s_pre = cpg + ((cmax4 + 63) & ~63);               // pages of the static keys' blocks [32]
  float* stk = reinterpret_cast<float*>(s_pre + 32);         // the append's carry stack, 16 * D
  float* att = stk + 16 * D;                                 // the attention's LDS

  const int t = p.tq[b];
  TA_DMARK(12);
  // paged caches: the pages of the static keys' blocks are requested now and stored after the descent, so
  // neither they nor the kept leaves' pages (read by the descent with the node rows) cost a round trip later
  const int32_t* ptrow = p.ptab ? p.ptab + b * p.pt_sb + h * p.pt_sh : nullptr;
  int pre = -1;
  if (ptrow != nullptr && tid <= p.Lw && t >= 0 && t < p.Tk) {
    const int pos = tid == 0 ? 0 : t - (tid - 1);
    if (pos >= 0) pre = ptrow[pos >> p.leaf_log2];
  }
  // The descent reads only nodes that end before t and the cache append writes row t and the nodes ending at
  // t, so the append's loads (the new rows, row t's page) are issued first and its stores follow the descent:
  // the first level's node rows are requested at once and the append is off that chain.
  const bool appends = tid < D && t >= 0 && t < ap.Tcap;
  T *kbase = nullptr, *vbase = nullptr;
  KvRows rows{};
  AppendPre<T> apre{};
  if (appends) {
    rows = append_rows<T>(ap, b, h, lv.blevel[0], kbase, vbase);
    apre = append_prefetch<T>(tid, t, reinterpret_cast<const T*>(ap.kn) + b * ap.nsb + h * ap.nsh,
                              reinterpret_cast<const T*>(ap.vn) + b * ap.vnsb + h * ap.vnsh, rows);
  }
  const T* qrow = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh;
  int nk = descend_query<T, D, kWavesPerBlock>(qrow, t, Tgeo, b, h, lv, n_levels, arity_log2, wmax, tid, ckey, cid,
                                               csc, kid, ksc, ptrow, cpg, kpg);
  TA_DMARK(13);
  if (appends)
    append_dim_with<T>(tid, D, t, apre, kbase, vbase, rows, n_levels, lv.blevel[0], arity_log2, stk,
                       [&](int j) { return const_cast<float*>(lv.ptr[j]) + b * lv.sb[j] + h * lv.sh[j]; });
  if (ptrow != nullptr && tid < 32) s_pre[tid] = pre;
  const int nkw = nk < p.wl ? nk : p.wl;   // the attention of the separate kernels sees the first wl of them
  // the appended row is visible to every wavefront: its stores (long since done) are waited for, then the
  // barrier; the selection's outputs are written after the attention, so that no wait here covers them
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int nt = p.n_tree ? p.n_tree[bh] : p.wl;
  T* orow = reinterpret_cast<T*>(p.out) + b * p.osb + h * p.osh;
  TA_DMARK(14);
  attn_query<T, D, true, false>(p, 0, 0, b, h, bh, qrow, t, kid, nullptr, nkw, nt, orow, att, kpg, s_pre);
  TA_DMARK(15);
  const int64_t obase = (int64_t)bh * p.wl;   // kid and ksc are not written by the attention
  for (int r = tid; r < p.wl; r += NT) {
    const bool ok = r < nk;
    ids[obase + r] = ok ? kid[r] : -1;
    vld[obase + r] = ok ? 1 : 0;
    sct[obase + r] = ok ? ksc[r] : -INFINITY;
  }
}

// ----------------------------------------------------------------------------------------- decode append
struct LevelRW {
  float* ptr[kMaxLevels];
  int64_t sb[kMaxLevels];
  int64_t sh[kMaxLevels];
};

// One thread per dimension of one (sequence, head): append_dim.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendIn ap, int H, int D, const int32_t* __restrict__ t_pos,
                                                        LevelRW lv, int n_levels, int leaf_log2, int arity_log2) {
  extern __shared__ float stk[];  // [16][D]
  const int d = threadIdx.x;
  if (d >= D) return;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int t = t_pos[b];
  if (t < 0 || t >= ap.Tcap) return;
  T *kbase, *vbase;
  const KvRows rows = append_rows<T>(ap, b, h, leaf_log2, kbase, vbase);
  append_dim<T>(d, D, t, reinterpret_cast<const T*>(ap.kn) + b * ap.nsb + h * ap.nsh,
                reinterpret_cast<const T*>(ap.vn) + b * ap.vnsb + h * ap.vnsh, kbase, vbase, rows, n_levels,
                leaf_log2, arity_log2, stk, [&](int j) { return lv.ptr[j] + b * lv.sb[j] + h * lv.sh[j]; });
}

// ----------------------------------------------------------------------------------------- host side
namespace {

int elem_size(int dt) { return dt == TA_F32 ? 4 : 2; }
bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// K/V/q rows are read in 16-byte slices.
bool kv_aligned(const void* p, int dt, int D, std::initializer_list<int64_t> strides) {
  const int a = 16;
  if (D * elem_size(dt) < 16 || (D * elem_size(dt)) % 16) return false;
  if (!aligned(p, a)) return false;
  for (int64_t s : strides)
    if ((s * elem_size(dt)) % a) return false;
  return true;
}

template <typename T, int D>
int launch_attn(const AttnParams& p, int B, bool split, hipStream_t st) {
  const int wl_pad = p.cand ? 0 : attn_list_cap(p.wl, p.nb_S);
  size_t lds = (size_t)kWavesPerBlock * attn_wave_ints(wl_pad) * sizeof(float);
  const dim3 blk(kWavesPerBlock * kWave);
  if (split) {
    lds += (size_t)kWavesPerBlock * (D + 2) * sizeof(float);
    dim3 grid((unsigned)((int64_t)p.Nq * p.gsplit), B * p.H);
    if (p.gsplit > 1) {
      if (p.cand) hipLaunchKernelGGL((attn_kernel<T, D, true, true, true>), grid, blk, lds, st, p);
      else hipLaunchKernelGGL((attn_kernel<T, D, true, false, true>), grid, blk, lds, st, p);
    } else {
      if (p.cand) hipLaunchKernelGGL((attn_kernel<T, D, true, true>), grid, blk, lds, st, p);
      else hipLaunchKernelGGL((attn_kernel<T, D, true, false>), grid, blk, lds, st, p);
    }
    return check_launch("attn_kernel");
  }
  dim3 grid((unsigned)((p.Nq + kWavesPerBlock - 1) / kWavesPerBlock), B * p.H);
  if (p.cand) hipLaunchKernelGGL((attn_kernel<T, D, false, true>), grid, blk, lds, st, p);
  else hipLaunchKernelGGL((attn_kernel<T, D, false, false>), grid, blk, lds, st, p);
  return check_launch("attn_kernel");
}

int dispatch_attn(int dt, int D, const AttnParams& p, int B, bool split, hipStream_t st) {
#define TA_CASE_D(T)                                             \
  switch (D) {                                                   \
    case 16: return launch_attn<T, 16>(p, B, split, st);         \
    case 32: return launch_attn<T, 32>(p, B, split, st);         \
    case 64: return launch_attn<T, 64>(p, B, split, st);         \
    case 128: return launch_attn<T, 128>(p, B, split, st);       \
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

// Paged K/V for the attention: checks the description against the leaf block and the row layout, and sets
// p (p.k / p.v stay the bases of page 0's rows; the per-sequence and per-head strides are zeroed).
int set_attn_pages(AttnParams& p, const ta_kv_pages* pages, int dt, int D, int leaf_log2, const char* who) {
  if (pages == nullptr) return TA_OK;
  // rows of K and V share one row index (page * rows-per-page + row in the page), an int32
  if (pages->table == nullptr || pages->num_pages <= 0 || pages->block_log2 != leaf_log2 || pages->page_stride <= 0 ||
      (pages->page_stride * elem_size(dt)) % 16 || p.kst < D || p.kst != p.vst || pages->page_stride % p.kst ||
      ((int64_t)p.kst << leaf_log2) > pages->page_stride ||
      pages->num_pages * (pages->page_stride / p.kst) > 0x7fffffffLL) {
    set_error(std::string(who) + ": bad page description (block must be the leaf block, pages 16-byte aligned, a "
                                 "whole number of rows and large enough for a block of rows, K and V rows alike, "
                                 "fewer than 2^31 rows in all)");
    return TA_ERR_ARG;
  }
  p.ptab = pages->table;
  p.pt_sb = pages->sb;
  p.pt_sh = pages->sh;
  p.kps = p.vps = pages->page_stride;
  p.npages = pages->num_pages;
  p.ksb = p.ksh = p.vsb = p.vsh = 0;
  return TA_OK;
}

void set_append_pages(AppendIn& ap, const ta_kv_pages* pages) {
  if (pages == nullptr) return;
  ap.ptab = pages->table;
  ap.pt_sb = pages->sb;
  ap.pt_sh = pages->sh;
  ap.pstride = pages->page_stride;
  ap.npages = pages->num_pages;
}

}  // namespace
}  // namespace ta

using namespace ta;

extern "C" int ta_sparse_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                                  int64_t qst, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                                  int64_t vst, const int32_t* cand, int B, int H, int T, int Tk, int KC, int D,
                                  float scale, void* out, float* lse, const ta_kv_pages* pages, void* stream) {
  if (B <= 0 || H <= 0 || T < 0 || Tk < 0 || KC < 0) {
    set_error("ta_sparse_attn_fwd: bad sizes");
    return TA_ERR_ARG;
  }
  if (T == 0) return TA_OK;
  if (!kv_aligned(q, dtype, D, {qsb, qsh, qst}) || !kv_aligned(k, dtype, D, {ksb, ksh, kst}) ||
      !kv_aligned(v, dtype, D, {vsb, vsh, vst})) {
    set_error("ta_sparse_attn_fwd: q/k/v rows not 16-byte aligned");
    return TA_ERR_ARG;
  }
  AttnParams p{};
  p.q = q; p.qsb = qsb; p.qsh = qsh; p.qsn = qst;
  p.k = k; p.ksb = ksb; p.ksh = ksh; p.kst = kst;
  p.v = v; p.vsb = vsb; p.vsh = vsh; p.vst = vst;
  p.H = H; p.Nq = T; p.Tk = Tk;
  p.cand = cand; p.KC = KC;
  p.leaf_log2 = pages ? pages->block_log2 : 1;   // dense: rows addressed as pairs of rows, row stride kst
  p.scale = scale;
  p.gsplit = 1;
  p.out = out; p.osb = (int64_t)H * T * D; p.osh = (int64_t)T * D; p.osn = D;
  p.lse = lse;
  if (pages && (pages->block_log2 < 1 || pages->block_log2 > 14)) {
    set_error("ta_sparse_attn_fwd: bad page block");
    return TA_ERR_ARG;
  }
  const int prc = set_attn_pages(p, pages, dtype, D, p.leaf_log2, "ta_sparse_attn_fwd");
  if (prc != TA_OK) return prc;
  return dispatch_attn(dtype, D, p, B, false, (hipStream_t)stream);
}


extern "C" int64_t ta_seg_attn_workspace_size(int B, int H, int Nq, int D, int nsplit) {
  const int gsplit = nsplit / kWavesPerBlock;
  if (gsplit <= 1 || B <= 0 || H <= 0 || Nq <= 0) return 0;
  return attn_counter_bytes(B, H, Nq) + (int64_t)B * H * Nq * gsplit * (D + 2) * (int64_t)sizeof(float);
}

namespace {

int seg_attn_fwd_impl(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                      int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                      int64_t vst, int B, int H, int Nq, int D, int Tk, const int32_t* tq, int64_t tq_sb,
                      const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl, int leaf,
                      int local, float scale, void* out, int64_t osb, int64_t osh, int64_t osn, float* lse,
                      float* keys, int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages,
                      const int32_t* nb_id, const uint8_t* nb_ok, int nb_S, void* stream) {
  if (B <= 0 || H <= 0 || Nq < 0 || wl < 0 || nsplit < 1 || leaf < 2 || (leaf & (leaf - 1)) ||
      (nsplit > 1 && nsplit % kWavesPerBlock) || nsplit > kWavesPerBlock * kWave) {
    set_error("ta_seg_attn_fwd: bad sizes (nsplit must be 1 or a multiple of 4, at most 256)");
    return TA_ERR_ARG;
  }
  if (nb_S < 0 || nb_S > kWave || (nb_S > 0 && (nb_id == nullptr || nb_ok == nullptr))) {
    set_error("ta_seg_attn_nb_fwd: neighbour slots must number at most 64, with ids and flags");
    return TA_ERR_ARG;
  }
  const int Lw = local > 3 ? local : 3;
  if (Lw + 1 > 32) {
    set_error("ta_seg_attn_fwd: local window must be < 32");
    return TA_ERR_UNSUPPORTED;
  }
  if (wl > 1024) {
    set_error("ta_seg_attn_fwd: beam wider than 1024 leaves");
    return TA_ERR_UNSUPPORTED;
  }
  if (Nq == 0) return TA_OK;
  const int64_t need = ta_seg_attn_workspace_size(B, H, Nq, D, nsplit);
  if (ws_bytes < need || (need > 0 && (ws == nullptr || (uintptr_t)ws % 256))) {
    set_error("ta_seg_attn_fwd: workspace missing, too small or not 256-byte aligned");
    return TA_ERR_WORKSPACE;
  }
  if (!kv_aligned(q, dtype, D, {qsb, qsh, qsn}) || !kv_aligned(k, dtype, D, {ksb, ksh, kst}) ||
      !kv_aligned(v, dtype, D, {vsb, vsh, vst})) {
    set_error("ta_seg_attn_fwd: q/k/v rows not 16-byte aligned");
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
  p.gsplit = nsplit > 1 ? nsplit / kWavesPerBlock : 1;
  p.out = out; p.osb = osb; p.osh = osh; p.osn = osn;
  p.lse = lse; p.keys = keys;
  if (need > 0) {
    p.cnt = reinterpret_cast<uint32_t*>(ws);
    p.ws = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + attn_counter_bytes(B, H, Nq));
  }
  p.nb_id = nb_id; p.nb_ok = nb_ok; p.nb_S = nb_S;
  const int prc = set_attn_pages(p, pages, dtype, D, ll, "ta_seg_attn_fwd");
  if (prc != TA_OK) return prc;
  if (nsplit == 1 && pages == nullptr && nb_S == 0) {
    // many queries (prefill): the matrix-core kernel when the shape fits it
    const int rc = prefill_attn_mfma(p, B, dtype, D, (hipStream_t)stream);
    if (rc != TA_ERR_UNSUPPORTED) return rc;
  }
  return dispatch_attn(dtype, D, p, B, nsplit > 1, (hipStream_t)stream);
}

}  // namespace

extern "C" int ta_seg_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                               int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                               int64_t vst, int B, int H, int Nq, int D, int Tk, const int32_t* tq, int64_t tq_sb,
                               const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl, int leaf,
                               int local, float scale, void* out, int64_t osb, int64_t osh, int64_t osn, float* lse,
                               float* keys, int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages,
                               void* stream) {
  return seg_attn_fwd_impl(q, k, v, dtype, qsb, qsh, qsn, ksb, ksh, kst, vsb, vsh, vst, B, H, Nq, D, Tk, tq, tq_sb,
                           ids, vld, n_tree, wl, leaf, local, scale, out, osb, osh, osn, lse, keys, nsplit, ws,
                           ws_bytes, pages, nullptr, nullptr, 0, stream);
}

extern "C" int ta_seg_attn_nb_fwd(const void* q, const void* k, const void* v, int dtype, int64_t qsb, int64_t qsh,
                                  int64_t qsn, int64_t ksb, int64_t ksh, int64_t kst, int64_t vsb, int64_t vsh,
                                  int64_t vst, int B, int H, int Nq, int D, int Tk, const int32_t* tq, int64_t tq_sb,
                                  const int32_t* ids, const uint8_t* vld, const int32_t* n_tree, int wl, int leaf,
                                  int local, float scale, const int32_t* nb_id, const uint8_t* nb_ok, int nb_S,
                                  void* out, int64_t osb, int64_t osh, int64_t osn, float* lse, float* keys,
                                  int nsplit, float* ws, int64_t ws_bytes, const ta_kv_pages* pages, void* stream) {
  return seg_attn_fwd_impl(q, k, v, dtype, qsb, qsh, qsn, ksb, ksh, kst, vsb, vsh, vst, B, H, Nq, D, Tk, tq, tq_sb,
                           ids, vld, n_tree, wl, leaf, local, scale, out, osb, osh, osn, lse, keys, nsplit, ws,
                           ws_bytes, pages, nb_id, nb_ok, nb_S, stream);
}

extern "C" int ta_seg_attend(const void* q, const void* k_new, const void* v_new, int dtype, int64_t qsb, int64_t qsh,
                             int64_t nsb, int64_t nsh, int64_t vnsb, int64_t vnsh, int B, int H, int D,
                             const int32_t* t_pos, int n_levels, float* const* lv_ptr, const int64_t* lv_sb,
                             const int64_t* lv_sh, int T, int leaf_log2, int arity_log2, int wmax, int wl, void* Kc,
                             void* Vc, int64_t csb, int64_t csh, int64_t cst, int Tcap, const int32_t* n_tree,
                             int local, float scale, int32_t* ids, uint8_t* vld, float* sct, void* out, int64_t osb,
                             int64_t osh, float* keys, const ta_kv_pages* pages, void* stream) {
  if (B <= 0 || H <= 0 || wmax < 1 || wl < 0 || wl > kWave || n_levels < 0 || n_levels > kMaxLevels || T <= 0 ||
      (T & (T - 1)) || leaf_log2 < 1 || leaf_log2 > 14 || arity_log2 < 1 || arity_log2 > 4 || Tcap <= 0) {
    set_error("ta_seg_attend: bad sizes (at most 64 kept leaves)");
    return TA_ERR_ARG;
  }
  if (D != 64 && D != 128) {
    set_error("ta_seg_attend: head dim must be 64 or 128");
    return TA_ERR_UNSUPPORTED;
  }
  const int Lw = local > 3 ? local : 3;
  if (Lw + 1 > 32) {
    set_error("ta_seg_attend: local window must be < 32");
    return TA_ERR_UNSUPPORTED;
  }
  if (!kv_aligned(q, dtype, D, {qsb, qsh}) || !kv_aligned(Kc, dtype, D, {csb, csh, cst}) ||
      !kv_aligned(k_new, dtype, D, {nsb, nsh}) || !kv_aligned(v_new, dtype, D, {vnsb, vnsh})) {
    set_error("ta_seg_attend: q/k/v rows not 16-byte aligned");
    return TA_ERR_ARG;
  }
  LevelIn lv;
  for (int j = 0; j < n_levels; ++j) {
    lv.ptr[j] = lv_ptr[j];
    lv.sb[j] = lv_sb[j];
    lv.sh[j] = lv_sh[j];
    lv.blevel[j] = leaf_log2 + j * arity_log2;
    if (!aligned(lv_ptr[j], 16)) {
      set_error("ta_seg_attend: level pointer not 16-byte aligned");
      return TA_ERR_ARG;
    }
  }
  if (n_levels == 0) lv.blevel[0] = leaf_log2;
  const int arity = 1 << arity_log2;
  const int cmax4 = (arity * wmax + arity - 1 + 3) & ~3;
  const int wmax4 = (wmax + 3) & ~3;
  const int wl_pad = (wl + 3) & ~3;
  const size_t lds = (size_t)(4 * cmax4 + 2 * wmax4 + (wmax4 + ((cmax4 + 63) & ~63) + 32) + 16 * D) * sizeof(float) +
                     (size_t)kWavesPerBlock * attn_wave_ints(wl_pad) * sizeof(float) +
                     (size_t)kWavesPerBlock * (D + 2) * sizeof(float);
  if (lds > 64 * 1024) {
    set_error("ta_seg_attend: beam too wide for LDS (arity * wmax too large)");
    return TA_ERR_UNSUPPORTED;
  }
  AttnParams p{};
  p.q = q; p.qsb = qsb; p.qsh = qsh; p.qsn = 0;
  p.k = Kc; p.ksb = csb; p.ksh = csh; p.kst = cst;
  p.v = Vc; p.vsb = csb; p.vsh = csh; p.vst = cst;
  p.H = H; p.Nq = 1; p.Tk = Tcap;
  p.tq = t_pos; p.tq_sb = 1;
  p.n_tree = n_tree; p.wl = wl;
  p.leaf_log2 = leaf_log2;
  p.Lw = Lw;
  p.scale = scale;
  p.gsplit = 1;
  p.out = out; p.osb = osb; p.osh = osh; p.osn = 0;
  p.keys = keys;
  const int prc = set_attn_pages(p, pages, dtype, D, leaf_log2, "ta_seg_attend");
  if (prc != TA_OK) return prc;
  AppendIn ap{k_new, v_new, nsb, nsh, vnsb, vnsh, Kc, Vc, csb, csh, cst, Tcap};
  set_append_pages(ap, pages);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(B * H), blk(kWavesPerBlock * kWave);
#define TA_SA(TT, DD) \
  hipLaunchKernelGGL((seg_attend_kernel<TT, DD>), grid, blk, lds, st, p, lv, n_levels, arity_log2, T, wmax, cmax4, ids, \
                     vld, sct, ap)
  switch (dtype) {
    case TA_F32: if (D == 64) TA_SA(float, 64); else TA_SA(float, 128); break;
    case TA_F16: if (D == 64) TA_SA(f16_t, 64); else TA_SA(f16_t, 128); break;
    case TA_BF16: if (D == 64) TA_SA(bf16_t, 64); else TA_SA(bf16_t, 128); break;
    default: set_error("unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_SA
  return check_launch("seg_attend_kernel");
}

extern "C" int ta_kv_append(const void* k_new, const void* v_new, int dtype, int64_t nsb, int64_t nsh, int64_t vnsb,
                            int64_t vnsh, void* Kc, void* Vc, int64_t csb, int64_t csh, int64_t cst, int B, int H,
                            int D, int Tcap, const int32_t* t_pos, int n_levels, float* const* lv_ptr,
                            const int64_t* lv_sb, const int64_t* lv_sh, int leaf_log2, int arity_log2,
                            const ta_kv_pages* pages, void* stream) {
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
  if (pages && (pages->table == nullptr || pages->block_log2 != leaf_log2 || pages->num_pages <= 0 ||
                pages->page_stride < ((int64_t)cst << leaf_log2))) {
    set_error("ta_kv_append: bad page description (block must be the leaf block)");
    return TA_ERR_ARG;
  }
  AppendIn ap{k_new, v_new, nsb, nsh, vnsb, vnsh, Kc, Vc, csb, csh, cst, Tcap};
  set_append_pages(ap, pages);
  const size_t lds = (size_t)16 * D * sizeof(float);
  dim3 grid(B * H);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL((kv_append_kernel<float>), grid, dim3(D), lds, st, ap, H, D, t_pos, lv, n_levels, leaf_log2,
                         arity_log2);
      break;
    case TA_F16:
      hipLaunchKernelGGL((kv_append_kernel<f16_t>), grid, dim3(D), lds, st, ap, H, D, t_pos, lv, n_levels, leaf_log2,
                         arity_log2);
      break;
    case TA_BF16:
      hipLaunchKernelGGL((kv_append_kernel<bf16_t>), grid, dim3(D), lds, st, ap, H, D, t_pos, lv, n_levels, leaf_log2,
                         arity_log2);
      break;
    default:
      set_error("unknown dtype");
      return TA_ERR_ARG;
  }
  return check_launch("kv_append_kernel");
}

TA_TRACE_EXPORTS
