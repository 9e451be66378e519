// Neighbour borrowing (reference-default selection mode): each query takes the leaf groups that the nearest
// earlier queries stored and keeps those it also scores well on.
//
// Reference functions replaced: seg.py:73-103 neighbor_pass, fastseg.py:274-299 neighbor_pass_fast, and the
// budget split of seg.py:111-117 (finish) when a budget is given.
//
// One wavefront per query.  Lane s < S = Wn * NS holds stored slot s: neighbour back = s / NS + 1 (position
// t - back), entry e = s % NS of that position's stored leaves.  The slots' leaf rows are scored by 16-lane
// groups with the canonical float32 dot (canon_dot: the same order as the descent and the gather-dot kernel),
// times the scale.  Then, per lane and with ballots over the slots:
//   ok0   = position >= 0 and the stored entry valid
//   match = ok0 and score >= base - rho * |base|          (each product and difference rounded to float32)
//   rate  = matches / max(valid, 1) over the first probe * NS slots (float32 division)
//   cap   = cap_min + round_half_even((Wn - cap_min) * rate);  match &= back <= cap;  all off without neighbours
//   nL    = distinct leaf ids among the matched slots
//   n_tree (with a budget L) = 0 if nL >= L, else max(L - nL, 2 if nL < ceil(L / 2) else 1), at most wmax.
#include "descend.hpp"

namespace ta {

struct NbParams {
  const void* q;              // (B, H, Nq, D) rows, element strides qsb, qsh, qsn
  int64_t qsb, qsh, qsn;
  const float* S0;            // leaf-level node sums (B, H, M, D) float32, rows contiguous
  int64_t ssb, ssh;
  int M;
  const int32_t* st_leaf;     // (B, H, Tst, NS) stored leaves, int32
  const float* st_score;      // their scores
  const uint8_t* st_ok;       // their validity (bytes)
  int64_t st_sb, st_sh, st_st;   // element strides (the NS entries of a position contiguous)
  int Tst;
  const int32_t* tq;          // positions (B, Nq), row stride tq_sb (0: one row shared by every sequence)
  int64_t tq_sb;
  int B, H, Nq;
  int Wn, NS, probe, cap_min, neighbors;
  float rho, scale;
  const int32_t* lhat;        // budgets per query (B, H, Nq) or null
  int wmax;
  int32_t* nid;               // out (B, H, Nq, Wn * NS): stored leaf ids (0 where the slot is empty)
  uint8_t* match;             // out: matched slots
  int32_t* nL;                // out (B, H, Nq): distinct matched leaves
  int32_t* n_tree;            // out (B, H, Nq): tree leaves to use (with lhat)
  ta_budget_head_in hd;       // with the budget head in the same launch (one query per (b, h)): its weights
  int hd_F;                   // the head's feature count
};

// LDS of the budget head's weights (floats): W1 transposed, W2, b1, b2, each rounded up to a copy round of 256
__host__ __device__ inline int nb_head_words(int F, int hid, int ncls) {
  return ((F * hid + 255) & ~255) + ((ncls * hid + 255) & ~255) + ((hid + 3) & ~3) + ((ncls + 3) & ~3);
}

// The budget head's class for one (sequence, head), by one wavefront: f holds its F features in LDS (the
// one-hot block at D + 1 .. D + H is not read: the head's column D + 1 + h is added instead, the product with the
// other zero features being exact zeros), hs its hid hidden units; W1 transposed (F x hid), W2 (ncls x hid) and
// the biases in LDS.  hidden = relu(W1 f + b1) (lane j forms units j, j + 64, ...), logits = W2 hidden + b2 (wave
// sums), the first maximum wins and a NaN logit counts as the maximum (torch's argmax).
__device__ __forceinline__ int budget_class(const float* f, float* hs, const float* wl, const float* w2l,
                                            const float* b1l, const float* b2l, int D, int H, int F, int hid,
                                            int ncls, int h) {
  const int lane = lane_id();
  wave_sync();
  for (int j = lane; j < hid; j += kWave) {
    float acc = 0.0f;
#pragma unroll 8
    for (int i = 0; i <= D; ++i) acc += wl[i * hid + j] * f[i];
    acc += wl[(D + 1 + h) * hid + j];
#pragma unroll 8
    for (int i = D + 1 + H; i < F; ++i) acc += wl[i * hid + j] * f[i];
    hs[j] = fmaxf(acc + b1l[j], 0.0f);
  }
  wave_sync();
  int best = 0;
  float bv = 0.0f;
  for (int c = 0; c < ncls; ++c) {
    float part = 0.0f;
    for (int j = lane; j < hid; j += kWave) part += w2l[c * hid + j] * hs[j];
    const float v = wave_sum(part) + b2l[c];
    if (c == 0 || (!(bv != bv) && (v > bv || v != v))) {
      best = c;
      bv = v;
    }
  }
  return best;
}

template <typename T, int D, bool HEAD>
__global__ __launch_bounds__(256) void neighbor_kernel(NbParams p) {
  constexpr int R = D / 16;
  const int lane = lane_id();
  const int64_t nq_all = (int64_t)p.B * p.H * p.Nq;
  const int64_t q_flat = (int64_t)blockIdx.x * 4 + wave_id();   // flat (b, h, n)
  const bool live = q_flat < nq_all;
  if (!HEAD && !live) return;
  // with the head every wavefront reaches its workgroup barrier: a wavefront past the end works on the last
  // query and writes nothing
  const int64_t qi = live ? q_flat : nq_all - 1;
  extern __shared__ float nb_lds[];
  float* w1l = nb_lds;
  float* w2l = w1l + ((p.hd_F * p.hd.hid + 255) & ~255);
  float* b1l = w2l + ((p.hd.ncls * p.hd.hid + 255) & ~255);
  float* b2l = b1l + ((p.hd.hid + 3) & ~3);
  float fq[(D + kWave - 1) / kWave], fs[(D + kWave - 1) / kWave], fk[(D + kWave - 1) / kWave];
  if constexpr (HEAD) {
    // the head's own inputs first (a wait for them must not wait for the copies below), then W1 and W2 into
    // LDS by direct loads, 1 KB per wavefront round, in flight while the neighbour pass runs
    const int bq = (int)(qi / p.H), hq = (int)(qi % p.H);
#pragma unroll
    for (int u = 0; u < (D + kWave - 1) / kWave; ++u) {
      const int i = lane + u * kWave < D ? lane + u * kWave : D - 1;
      fq[u] = to_f32(reinterpret_cast<const T*>(p.q)[bq * p.qsb + hq * p.qsh + i]);
      fs[u] = p.hd.ksum != nullptr ? p.hd.ksum[qi * D + i] : 0.0f;
      fk[u] = p.hd.k != nullptr ? to_f32(reinterpret_cast<const T*>(p.hd.k)[bq * p.hd.ksb + hq * p.hd.ksh + i])
                                : 0.0f;
    }
    const int n1 = (p.hd_F * p.hd.hid + 255) >> 8, n2 = (p.hd.ncls * p.hd.hid + 255) >> 8;
    for (int c = wave_id(); c < n1 + n2; c += 4) {
      const bool first = c < n1;
      const int cc = first ? c : c - n1;
      const int nw = first ? p.hd_F * p.hd.hid : p.hd.ncls * p.hd.hid;
      const int e = cc * 256 + lane * 4 < nw ? cc * 256 + lane * 4 : 0;   // a surplus lane copies word 0 again
      const float* src = (first ? p.hd.w1t : p.hd.w2) + e;
      float* dst = (first ? w1l : w2l) + cc * 256;
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)dst, 16, 0, 0);
    }
  }
  const int n = (int)(qi % p.Nq);
  const int bh = (int)(qi / p.Nq);
  const int b = bh / p.H, h = bh % p.H;
  const int t = p.tq[b * p.tq_sb + n];
  const int S = p.Wn * p.NS;

  // this lane's slot
  const int back = lane / p.NS + 1, e = lane % p.NS;
  const int j = t - back;
  bool ok0 = false;
  int id = 0;
  float base = 0.0f;
  if (lane < S && j >= 0 && j < p.Tst) {
    const int64_t o = b * p.st_sb + h * p.st_sh + (int64_t)j * p.st_st + e;
    id = p.st_leaf[o];
    base = p.st_score[o];
    ok0 = p.st_ok[o] != 0;
  }

  // scores: group g (16 lanes) takes slots g, g + 4, ...; lane j16 of a group holds elements [R j16, R j16 + R)
  const int g = lane >> 4, j16 = lane & 15;
  float qr[R];
  load_row<T, R>(reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn + R * j16, qr);
  const float* srow = p.S0 + b * p.ssb + h * p.ssh + R * j16;
  float sc = 0.0f;
  for (int r0 = 0; r0 < S; r0 += 4) {
    const int s = r0 + g;
    int sid = __shfl(id, s < S ? s : 0, kWave);
    sid = sid < 0 ? 0 : (sid >= p.M ? p.M - 1 : sid);   // gather-dot clamps the id into the level
    float rows[R];
    load_row_g<float, R>(srow + (int64_t)sid * D, rows);
    const float v = __fmul_rn(canon_dot<R>(qr, rows), p.scale);   // every lane of the group holds it
    const float mine = __shfl(v, (lane & 3) * 16, kWave);         // slot r0 + lane % 4 comes from group lane % 4
    if ((lane >> 2) == (r0 >> 2)) sc = mine;
  }

  bool m;
  {
#pragma clang fp contract(off)
    const float thr = base - p.rho * fabsf(base);
    m = lane < S && ok0 && sc >= thr;
  }
  const uint64_t in_probe = p.probe * p.NS >= 64 ? ~0ull : ((1ull << (p.probe * p.NS)) - 1);
  const uint64_t okb = __ballot(lane < S && ok0), mb = __ballot(m);
  const int nok = __popcll(okb & in_probe), nm = __popcll(mb & in_probe);
  const float rate = (float)nm / (float)(nok > 1 ? nok : 1);
  const int cap = p.cap_min + (int)rintf((float)(p.Wn - p.cap_min) * rate);
  m = m && back <= cap && p.neighbors != 0;
  // distinct matched ids: a matched lane counts unless an earlier matched lane holds the same id
  const uint64_t fin = __ballot(m);
  bool first = m;
  for (int s = 0; s < S; ++s) {
    const int other = __shfl(id, s, kWave);
    if (((fin >> s) & 1) && s < lane && other == id) first = false;
  }
  const int nl = __popcll(__ballot(first));

  int L = 0;
  if constexpr (HEAD) {
    const int F = p.hd_F, hid = p.hd.hid, ncls = p.hd.ncls;
    float* f = b2l + ((ncls + 3) & ~3) + wave_id() * (F + hid);
    float* hs = f + F;
    if ((int)threadIdx.x < hid) b1l[threadIdx.x] = p.hd.b1[threadIdx.x];
    if ((int)threadIdx.x < ncls) b2l[threadIdx.x] = p.hd.b2[threadIdx.x];
    // features [q, log(|q| + 1e-6), one-hot(h), ksum / max(t, 1)]; the key sum then takes this step's key
    float ss = 0.0f;
    const float tt = (float)max(t, 1);
#pragma unroll
    for (int u = 0; u < (D + kWave - 1) / kWave; ++u) {
      const int i = lane + u * kWave;
      if (i < D) {
        f[i] = fq[u];
        ss += fq[u] * fq[u];
        if (p.hd.ksum != nullptr) {
          f[D + 1 + p.H + i] = fs[u] / tt;
          if (live && p.hd.k != nullptr) p.hd.ksum[qi * D + i] = fs[u] + fk[u];
        }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) f[D] = logf(sqrtf(ss) + 1e-6f);
    wait_vmcnt_n<0>();
    __syncthreads();
    if (!live) return;
    L = p.hd.classes[budget_class(f, hs, w1l, w2l, b1l, b2l, D, p.H, F, hid, ncls, h)];
    if (lane == 0 && p.hd.lhat != nullptr) p.hd.lhat[qi] = L;
  }
  if (lane < S) {
    p.nid[qi * S + lane] = id;
    p.match[qi * S + lane] = m ? 1 : 0;
  }
  if (lane == 0) {
    p.nL[qi] = nl;
    if ((HEAD || p.lhat != nullptr) && p.n_tree != nullptr) {
      if constexpr (!HEAD) L = p.lhat[qi];
      const int half = (L + 1) / 2;
      const int need = L - nl > 0 ? L - nl : 0;
      const int least = nl < half ? 2 : 1;
      int nt = nl >= L ? 0 : (need > least ? need : least);
      p.n_tree[qi] = nt < p.wmax ? nt : p.wmax;
    }
  }
}

// ----------------------------------------------------------------------------------------- leaf store
// The decode step's store of position t's top n leaves for the next positions' neighbour pass (engine.py:103-105):
// st_leaf[b, h, t, r] = the leaf id (an invalid slot's -1 as 0), st_score = its score (0 when invalid), st_ok =
// valid, for r < n.  One thread per (b, h, r); a position outside [0, Tst) is skipped.
__global__ __launch_bounds__(256) void leaf_store_kernel(const int32_t* __restrict__ ids, const uint8_t* __restrict__ vld,
                                                         const float* __restrict__ sct, int H, int wl, int n,
                                                         const int32_t* __restrict__ t_pos, int32_t* __restrict__ st_leaf,
                                                         float* __restrict__ st_score, uint8_t* __restrict__ st_ok,
                                                         int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst,
                                                         int total) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int bh = i / n, r = i - bh * n;
  const int b = bh / H, h = bh - b * H;
  const int t = t_pos[b];
  if (t < 0 || t >= Tst) return;
  const int64_t src = (int64_t)bh * wl + r;
  const int64_t dst = b * st_sb + h * st_sh + (int64_t)t * st_st + r;
  const bool ok = vld[src] != 0;
  const int id = ids[src];
  st_leaf[dst] = id < 0 ? 0 : id;
  st_score[dst] = ok ? sct[src] : 0.0f;
  st_ok[dst] = ok ? 1 : 0;
}


// The budget head of one decode step (engine.py:89-96): per (sequence, head) the features
//   f = [q (D), log(|q| + 1e-6), one-hot(h) (H), ksum / max(t, 1) (D, with the global pool)],
// hidden = relu(W1 f + b1), logits = W2 hidden + b2, budget = classes[argmax logits] (the first maximum; a NaN
// logit counts as the maximum, as torch's argmax takes it).  Everything in float32.  A workgroup of eight
// wavefronts serves eight (b, h): it first copies the weights (W1 transposed, F x hid; W2; b1; b2) into LDS with
// all its loads in flight, then each wavefront puts its features in its LDS row, lane j forms hidden units j,
// j + 64, ... (consecutive LDS words across the lanes, the feature a broadcast), and each logit is a wave sum.
// The one-hot term adds W1's column D + 1 + h, the product with the other zero features being exact zeros.
// With `k` the running key sum then takes this step's key (ksum += k), after its read: the sum of keys
// 0 .. t-1 feeds the head at t.
constexpr int kBhWaves = 8, kBhMaxF = 1024, kBhMaxHid = 256, kBhMaxCls = 64, kBhMaxW = 24576;

template <typename T>
__global__ __launch_bounds__(kBhWaves * kWave) void budget_head_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, float* __restrict__ ksum, const T* __restrict__ k, int64_t ksb,
    int64_t ksh, const int32_t* __restrict__ t_pos, const float* __restrict__ w1t, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, const int32_t* __restrict__ classes, int B, int H,
    int D, int F, int hid, int ncls, int32_t* __restrict__ lhat) {
  extern __shared__ float bh_lds[];
  const int nw = F * hid, n2 = ncls * hid;
  float* wl = bh_lds;                                   // W1 transposed, F x hid
  float* w2l = wl + ((nw + 3) & ~3);                    // W2, ncls x hid
  float* b1l = w2l + n2;                                // b1 (hid), then b2 (ncls)
  float* b2l = b1l + hid;
  const int lane = lane_id(), w = wave_id();
  float* f = bh_lds + ((nw + 3) & ~3) + ((n2 + hid + ncls + 3) & ~3) + w * (F + hid);
  float* hs = f + F;                                    // this wavefront's features, then its hidden units
  {
    // the weights into LDS, every load issued before the first is waited for: W1 in float4 words while the
    // size allows (hid % 4 == 0 keeps the table 16-byte aligned)
    const int tid = threadIdx.x;
    if ((hid & 3) == 0) {
      const float4* src = reinterpret_cast<const float4*>(w1t);
      float4* dst = reinterpret_cast<float4*>(wl);
      const int n4 = nw >> 2;
#pragma unroll 8
      for (int i = tid; i < n4; i += kBhWaves * kWave) dst[i] = src[i];
    } else {
#pragma unroll 8
      for (int i = tid; i < nw; i += kBhWaves * kWave) wl[i] = w1t[i];
    }
#pragma unroll 4
    for (int i = tid; i < n2; i += kBhWaves * kWave) w2l[i] = w2[i];
    if (tid < hid) b1l[tid] = b1[tid];
    if (tid < ncls) b2l[tid] = b2[tid];
  }
  const int bh = blockIdx.x * kBhWaves + w;
  const bool live = bh < B * H;
  const int b = live ? bh / H : 0, h = live ? bh - b * H : 0;
  if (live) {
    const T* qr = q + b * qsb + h * qsh;
    float ss = 0.0f;
    for (int i = lane; i < D; i += kWave) {
      const float x = to_f32(qr[i]);
      f[i] = x;
      ss += x * x;
    }
    ss = wave_sum(ss);
    if (lane == 0) f[D] = logf(sqrtf(ss) + 1e-6f);
    if (ksum != nullptr) {
      const float tt = (float)max(t_pos[b], 1);
      float* kr = ksum + (int64_t)bh * D;
      float* fp = f + D + 1 + H;
      for (int i = lane; i < D; i += kWave) {
        const float s = kr[i];
        fp[i] = s / tt;
        if (k != nullptr) kr[i] = s + to_f32(k[b * ksb + h * ksh + i]);
      }
    }
  }
  __syncthreads();
  if (!live) return;
  const int best = budget_class(f, hs, wl, w2l, b1l, b2l, D, H, F, hid, ncls, h);
  if (lane == 0) lhat[bh] = classes[best];
}

}  // namespace ta

using namespace ta;

extern "C" int ta_leaf_store(const int32_t* ids, const uint8_t* vld, const float* sct, int B, int H, int wl, int n,
                             const int32_t* t_pos, int32_t* st_leaf, float* st_score, uint8_t* st_ok, int64_t st_sb,
                             int64_t st_sh, int64_t st_st, int Tst, void* stream) {
  if (B <= 0 || H <= 0 || wl < 0 || n < 0 || n > wl || Tst <= 0 || ids == nullptr || vld == nullptr ||
      sct == nullptr || t_pos == nullptr || st_leaf == nullptr || st_score == nullptr || st_ok == nullptr) {
    set_error("ta_leaf_store: bad arguments (0 <= n <= wl)");
    return TA_ERR_ARG;
  }
  const int64_t total = (int64_t)B * H * n;
  if (total == 0) return TA_OK;
  if (total > 0x7fffffff) {
    set_error("ta_leaf_store: too many slots");
    return TA_ERR_ARG;
  }
  hipLaunchKernelGGL(leaf_store_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, ids,
                     vld, sct, H, wl, n, t_pos, st_leaf, st_score, st_ok, st_sb, st_sh, st_st, Tst, (int)total);
  return check_launch("leaf_store_kernel");
}

extern "C" int ta_budget_head(const void* q, int q_dtype, int64_t qsb, int64_t qsh, float* ksum, const void* k,
                              int64_t ksb, int64_t ksh, const int32_t* t_pos, const float* w1t, const float* b1,
                              const float* w2, const float* b2, const int32_t* classes, int B, int H, int D, int hid,
                              int ncls, int32_t* lhat, void* stream) {
  const int F = D + 1 + H + (ksum != nullptr ? D : 0);
  if (B <= 0 || H <= 0 || D <= 0 || hid <= 0 || hid > kBhMaxHid || ncls <= 0 || ncls > kBhMaxCls ||
      2 * D + 1 + H > kBhMaxF || (int64_t)(F + ncls) * hid > kBhMaxW || q == nullptr || t_pos == nullptr ||
      w1t == nullptr || b1 == nullptr || w2 == nullptr || b2 == nullptr || classes == nullptr || lhat == nullptr ||
      (k != nullptr && ksum == nullptr) || (int64_t)B * H > 0x7fffffff - kBhWaves ||
      ((hid & 3) == 0 && ((uintptr_t)w1t & 15))) {
    set_error("ta_budget_head: bad arguments (hid <= 256, classes <= 64, 2 D + 1 + H <= 1024, (F + classes) * hid <= 24576, "
              "W1 16-byte aligned)");
    return TA_ERR_ARG;
  }
  const dim3 grid((unsigned)((B * H + kBhWaves - 1) / kBhWaves));
  const size_t lds = ((size_t)((F * hid + 3) & ~3) + (size_t)((ncls * hid + hid + ncls + 3) & ~3) +
                      (size_t)kBhWaves * (F + hid)) * sizeof(float);
  hipStream_t st = (hipStream_t)stream;
#define TA_BH(TT)                                                                                                  \
  hipLaunchKernelGGL(budget_head_kernel<TT>, grid, dim3(kBhWaves * kWave), lds, st, (const TT*)q, qsb, qsh, ksum,  \
                     (const TT*)k, ksb, ksh, t_pos, w1t, b1, w2, b2, classes, B, H, D, F, hid, ncls, lhat)
  switch (q_dtype) {
    case TA_F32: TA_BH(float); break;
    case TA_BF16: TA_BH(bf16_t); break;
    case TA_F16: TA_BH(f16_t); break;
    default:
      set_error("ta_budget_head: q dtype f32, bf16 or f16");
      return TA_ERR_ARG;
  }
#undef TA_BH
  return check_launch("budget_head_kernel");
}

namespace {
int neighbor_pass_impl(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, const float* S0,
                       int64_t ssb, int64_t ssh, int M, const int32_t* st_leaf, const float* st_score,
                       const uint8_t* st_ok, int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst,
                       const int32_t* tq, int64_t tq_sb, int B, int H, int Nq, int D, int nb_window,
                       int nb_store, int nb_probe, int nb_cap_min, float nb_rho, int neighbors, float scale,
                       const int32_t* lhat, int wmax, int32_t* nid, uint8_t* match, int32_t* nL,
                       int32_t* n_tree, const ta_budget_head_in* hd, void* stream) {
  if (B <= 0 || H <= 0 || Nq <= 0 || M <= 0 || nb_window <= 0 || nb_store <= 0 || nb_window * nb_store > 64 ||
      nb_probe < 0 || Tst <= 0 || (D != 16 && D != 32 && D != 64 && D != 128 && D != 256) || q == nullptr || S0 == nullptr || st_leaf == nullptr ||
      st_score == nullptr || st_ok == nullptr || tq == nullptr || nid == nullptr || match == nullptr ||
      nL == nullptr || (lhat != nullptr && n_tree == nullptr)) {
    set_error("ta_neighbor_pass: bad arguments (D 16, 32, 64, 128 or 256; nb_window * nb_store <= 64)");
    return TA_ERR_ARG;
  }
  const int R = D / 16, es = q_dtype == TA_F32 ? 4 : 2;
  if (((uintptr_t)S0 % 16) || (ssb % 4) || (ssh % 4) || ((uintptr_t)q % (R * es)) || (qsb % R) || (qsh % R) ||
      (qsn % R)) {
    set_error("ta_neighbor_pass: node sums 16-byte aligned, query rows aligned to D / 16 elements");
    return TA_ERR_ARG;
  }
  NbParams p{q, qsb, qsh, qsn, S0, ssb, ssh, M, st_leaf, st_score, st_ok, st_sb, st_sh, st_st, Tst, tq, tq_sb,
             B, H, Nq, nb_window, nb_store, nb_probe, nb_cap_min, neighbors, nb_rho, scale, lhat, wmax, nid, match,
             nL, n_tree, ta_budget_head_in{}, 0};
  size_t lds = 0;
  if (hd != nullptr) {
    // the budget head in the same launch: one query per (b, h), W1 / W2 rows whole float4 words
    const int F = D + 1 + H + (hd->ksum != nullptr ? D : 0);
    lds = ((size_t)nb_head_words(F, hd->hid, hd->ncls) + (size_t)4 * (F + hd->hid)) * sizeof(float);
    if (Nq != 1 || lhat != nullptr || n_tree == nullptr || hd->w1t == nullptr || hd->b1 == nullptr ||
        hd->w2 == nullptr || hd->b2 == nullptr || hd->classes == nullptr || hd->hid <= 0 || hd->hid > 256 ||
        (hd->hid & 3) || hd->ncls <= 0 || hd->ncls > 64 || ((uintptr_t)hd->w1t & 15) || ((uintptr_t)hd->w2 & 15) ||
        (hd->k != nullptr && hd->ksum == nullptr) || lds > 160 * 1024) {
      set_error("ta_neighbor_pass_head: one query per (b, h), no lhat, n_tree given; hid <= 256 and a multiple of "
                "4, classes <= 64, W1 and W2 16-byte aligned, weights within 160 KB of LDS");
      return TA_ERR_ARG;
    }
    p.hd = *hd;
    p.hd_F = F;
  }
  const int64_t nqry = (int64_t)B * H * Nq;
  const dim3 grid((unsigned)((nqry + 3) / 4));
  hipStream_t st = (hipStream_t)stream;
#define TA_NB(TT, DD)                                                                          \
  do {                                                                                         \
    if (hd != nullptr)                                                                         \
      hipLaunchKernelGGL((neighbor_kernel<TT, DD, true>), grid, dim3(256), lds, st, p);        \
    else                                                                                       \
      hipLaunchKernelGGL((neighbor_kernel<TT, DD, false>), grid, dim3(256), 0, st, p);         \
  } while (0)
#define TA_NB_D(TT)                          \
  switch (D) {                               \
    case 16: TA_NB(TT, 16); break;           \
    case 32: TA_NB(TT, 32); break;           \
    case 64: TA_NB(TT, 64); break;           \
    case 128: TA_NB(TT, 128); break;         \
    default: TA_NB(TT, 256); break;          \
  }
  switch (q_dtype) {
    case TA_F32: TA_NB_D(float); break;
    case TA_F16: TA_NB_D(f16_t); break;
    case TA_BF16: TA_NB_D(bf16_t); break;
    default: set_error("ta_neighbor_pass: unknown dtype"); return TA_ERR_ARG;
  }
#undef TA_NB_D
#undef TA_NB
  return check_launch("neighbor_kernel");
}
}  // namespace

extern "C" int ta_neighbor_pass(const void* q, int q_dtype, int64_t qsb, int64_t qsh, int64_t qsn, const float* S0,
                                int64_t ssb, int64_t ssh, int M, const int32_t* st_leaf, const float* st_score,
                                const uint8_t* st_ok, int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst,
                                const int32_t* tq, int64_t tq_sb, int B, int H, int Nq, int D, int nb_window,
                                int nb_store, int nb_probe, int nb_cap_min, float nb_rho, int neighbors, float scale,
                                const int32_t* lhat, int wmax, int32_t* nid, uint8_t* match, int32_t* nL,
                                int32_t* n_tree, void* stream) {
  return neighbor_pass_impl(q, q_dtype, qsb, qsh, qsn, S0, ssb, ssh, M, st_leaf, st_score, st_ok, st_sb, st_sh, st_st,
                            Tst, tq, tq_sb, B, H, Nq, D, nb_window, nb_store, nb_probe, nb_cap_min, nb_rho, neighbors,
                            scale, lhat, wmax, nid, match, nL, n_tree, nullptr, stream);
}

extern "C" int ta_neighbor_pass_head(const void* q, int q_dtype, int64_t qsb, int64_t qsh, const float* S0,
                                     int64_t ssb, int64_t ssh, int M, const int32_t* st_leaf, const float* st_score,
                                     const uint8_t* st_ok, int64_t st_sb, int64_t st_sh, int64_t st_st, int Tst,
                                     const int32_t* t_pos, int B, int H, int D, int nb_window, int nb_store,
                                     int nb_probe, int nb_cap_min, float nb_rho, int neighbors, float scale, int wmax,
                                     const ta_budget_head_in* head, int32_t* nid, uint8_t* match, int32_t* nL,
                                     int32_t* n_tree, void* stream) {
  if (head == nullptr) {
    set_error("ta_neighbor_pass_head: head missing");
    return TA_ERR_ARG;
  }
  return neighbor_pass_impl(q, q_dtype, qsb, qsh, 0, S0, ssb, ssh, M, st_leaf, st_score, st_ok, st_sb, st_sh, st_st,
                            Tst, t_pos, 1, B, H, 1, D, nb_window, nb_store, nb_probe, nb_cap_min, nb_rho, neighbors,
                            scale, nullptr, wmax, nid, match, nL, n_tree, head, stream);
}
