// Sparse softmax attention of one query over the keys it selected, shared by the attention kernels
// (attend.hip) and the persistent decode step (step.hip).
//
// Reference functions replaced: fastseg.py:50-78 (_attn_fwd), fastseg.py:134-177 (sparse_attn),
// fastseg.py:367-383 (candidate assembly + dedupe_fast), engine.py:107-119 (decode attention).
#pragma once

#include "attn.hpp"
#include "common.hpp"

namespace ta {

constexpr int kWavesPerBlock = 4;
template <typename T> struct Raw16;  // 16 bytes of T -> EPL floats
template <> struct Raw16<float> {
  static constexpr int EPL = 4;
  __device__ static void cvt(const uint4& u, float (&f)[4]) {
    f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y); f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
  }
};
template <> struct Raw16<bf16_t> {
  static constexpr int EPL = 8;
  __device__ static void cvt(const uint4& u, float (&f)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <> struct Raw16<f16_t> {
  static constexpr int EPL = 8;
  __device__ static void cvt(const uint4& u, float (&f)[8]) {
    const f16_t* h = reinterpret_cast<const f16_t*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};

// Attention of queries over their key lists.  Rows of K and V are read as 16-byte slices: LPR = D / EPL
// lanes share a row (EPL elements each) and one load instruction covers RPI = 64 / LPR consecutive keys,
// so a leaf block is read in contiguous 1 KB pieces.  A chunk is NL load instructions = KPC keys; the loads
// of the next PF chunks are in flight while one is consumed.  Scores are reduced over the LPR lanes of
// a row; every lane keeps a weighted-V accumulator for its EPL dimensions, reduced over the RPI row groups
// at the end.
//   SPLIT = false: one wavefront per query (many queries: prefill).
//   SPLIT = true: the 4 wavefronts of a workgroup share one query and interleave its chunks; their partial
//   (max, sum, accumulator) are merged in LDS.  With gsplit > 1 workgroups per query each writes its merged
//   partial to ws with stores that write through to memory, waits for them to complete and counts itself in;
//   the last to arrive reads the partials past the caches, combines them
//   (out = sum_g acc_g e^(m_g - M) / sum_g L_g e^(m_g - M)) and resets the counter.  No workgroup waits for
//   another.
// Per query: n (index in its (sequence, head) row), g (split index), b, h, qi (flat query index for the
// per-query arrays of p), qrow (the query's D elements), t (position; structural mode), idr / vr (selected
// leaf-block ids and their validity; structural mode), nv_given (number of valid ids when >= 0, else counted
// from vr), nt (budget of tree leaves), orow_base (the output row), smem_f (LDS of the workgroup).
// Paged caches: pre_leaf_pg (LDS, may be null) holds the pages of the leaf blocks idr lists and pre_static_pg
// (LDS, may be null) the page of static slot i's block (slot 0: position 0, slot i >= 1: position t - i + 1),
// read earlier by the caller; when null they are looked up in the page table here.
template <typename T, int D, bool SPLIT, bool CAND, bool PIPE = false>
__device__ __forceinline__ void attn_query(const AttnParams& p, int n, int g, int b, int h, int64_t qi, const T* qrow,
                                           int t, const int32_t* idr, const uint8_t* vr, int nv_given, int nt,
                                           T* orow_base, float* smem_f, const int32_t* pre_leaf_pg = nullptr,
                                           const int32_t* pre_static_pg = nullptr) {
  constexpr int EPL = Raw16<T>::EPL;
  constexpr int LPR = D / EPL;              // lanes per key row
  static_assert(LPR >= 1 && LPR <= kWave, "row slice layout");
  constexpr int RPI = kWave / LPR;          // key rows per load instruction
  constexpr int NL = 2;                     // load instructions per chunk (4 chunks in flight ahead)
  constexpr int KPC = NL * RPI;             // keys per chunk
  const int lane = lane_id(), w = wave_id();
  (void)n;
  (void)b;
  (void)h;
  const int wl_pad = p.cand ? 0 : attn_list_cap(p.wl, p.nb_S);
  // per wavefront: used leaf ids [wl_pad], their pages [wl_pad], static keys [32] and their pages [32]
  int32_t* s_ids = reinterpret_cast<int32_t*>(smem_f + w * attn_wave_ints(wl_pad));
  int32_t* s_row0 = s_ids + wl_pad;
  int32_t* s_ext = s_row0 + wl_pad;
  // Keys are addressed by a row index r (K at kb + r * kst, V at vb + r * vst).  Contiguous caches: r is the
  // position.  Paged caches: r = page * rpp + (position within the block), rpp = rows from one page to the next
  // (the page stride in rows), so a key costs the same arithmetic in both layouts.  row0_of(j): the row of the
  // first position of leaf block j, -1 when the block has no valid page (its keys are then skipped).
  const int32_t* ptrow = p.ptab ? p.ptab + b * p.pt_sb + h * p.pt_sh : nullptr;
  const int rpp = ptrow ? (int)(p.kps / p.kst) : 0;
  auto row0_pg = [&](int pg) -> int { return (pg >= 0 && pg < p.npages) ? pg * rpp : -1; };
  auto row0_of = [&](int j) -> int { return ptrow == nullptr ? (j << p.leaf_log2) : row0_pg(ptrow[j]); };
  const int rg = lane / LPR;               // key row of this lane inside a load instruction
  const int ds = (lane % LPR) * EPL;       // first dimension of this lane's slice

  float qv[EPL];
  load_row<T, EPL>(qrow + ds, qv);

  // key list of this query
  int N, nused = 0, lb = 0, nloc = 0, next = 0, own0 = -1;
  const int leaf = 1 << p.leaf_log2;
  if constexpr (CAND) {
    N = p.KC;
  } else {
    if (t >= p.Tk) t = -1;  // out of range: attend nothing
    int nv = nv_given;
    if (nv < 0) {
      nv = 0;
      for (int i0 = 0; i0 < p.wl; i0 += kWave) {
        const int i = i0 + lane;
        const bool v = i < p.wl && vr[i] != 0;
        nv += __popcll(__ballot(v));
      }
    }
    nused = t < 0 ? 0 : (nv < nt ? nv : (nt > 0 ? nt : 0));
    for (int i = lane; i < nused; i += kWave) {
      const int id = idr[i];
      s_ids[i] = id;
      s_row0[i] = (pre_leaf_pg != nullptr && ptrow != nullptr) ? row0_pg(pre_leaf_pg[i]) : row0_of(id);
    }
    lb = t < 0 ? 0 : (t >> p.leaf_log2) << p.leaf_log2;
    nloc = t < 0 ? 0 : t - lb + 1;
    wave_sync();
    if (p.nb_S > 0 && t >= 0) {
      // neighbour leaves: a matched slot joins when its block is complete before the own block, is not one of the
      // tree leaves and no earlier matched slot holds the same leaf (the reference's first-copy dedupe of
      // [tree | neighbour | static] positions, fastseg.py:376-381, as a set of leaf blocks)
      const bool in = lane < p.nb_S;
      const int id = in ? p.nb_id[qi * p.nb_S + lane] : -1;
      const bool cand = in && p.nb_ok[qi * p.nb_S + lane] != 0 && id >= 0;
      bool keepn = cand && id < (lb >> p.leaf_log2);
      for (int i = 0; i < nused; ++i)
        if (s_ids[i] == id) keepn = false;
      const uint64_t cm = __ballot(cand);
      for (int s2 = 0; s2 < p.nb_S; ++s2) {
        const int o = __shfl(id, s2, kWave);
        if (((cm >> s2) & 1) && s2 < lane && o == id) keepn = false;
      }
      const uint64_t km = __ballot(keepn);
      if (keepn) {
        const int slot = nused + __popcll(km & ((1ull << lane) - 1));
        s_ids[slot] = id;
        s_row0[slot] = row0_of(id);
      }
      nused += __popcll(km);
      wave_sync();
    }
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
    if (keep) {
      const int slot = __popcll(bal & ((1ull << lane) - 1));
      const int r0 = (pre_static_pg != nullptr && ptrow != nullptr) ? row0_pg(pre_static_pg[lane])
                                                                    : row0_of(pe >> p.leaf_log2);
      s_ext[slot] = r0 < 0 ? -1 : r0 + (pe & (leaf - 1));
    }
    next = __popcll(bal);
    N = nused * leaf + nloc + next;
    own0 = t < 0 ? -1 : ((pre_static_pg != nullptr && ptrow != nullptr) ? row0_pg(pre_static_pg[1])
                                                                        : row0_of(t >> p.leaf_log2));
  }
  wave_sync();

  const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.k) + b * p.ksb + h * p.ksh + ds);
  const char* vb = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.v) + b * p.vsb + h * p.vsh + ds);
  const int64_t kst_b = p.kst * (int64_t)sizeof(T), vst_b = p.vst * (int64_t)sizeof(T);
  const int nchunks = (N + KPC - 1) / KPC;
  const int nl = nused * leaf;
  const int stride = SPLIT ? p.gsplit * kWavesPerBlock : 1;
  const int first = SPLIT ? g * kWavesPerBlock + w : 0;

  // All positions of a chunk first (branch-free LDS reads in the structural mode, so no wait on memory
  // sits between the K/V loads), then its K/V loads.
  // All rows of a chunk first (branch-free LDS reads in the structural mode, so no wait on memory sits
  // between the K/V loads), then its K/V loads.
  auto fetch = [&](int c, uint4 (&kr)[NL], uint4 (&vr)[NL], bool (&ok)[NL]) {
    int row[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int key = c * KPC + i * RPI + rg;
      if constexpr (CAND) {
        const int pos = key < N ? p.cand[qi * p.KC + key] : -1;
        const int r0 = (pos >= 0 && pos < p.Tk) ? row0_of(pos >> p.leaf_log2) : -1;
        row[i] = r0 < 0 ? -1 : r0 + (pos & (leaf - 1));
      } else {
        const int kt = key < nl ? key : 0;
        const int r0 = s_row0[kt >> p.leaf_log2];
        const int leafrow = r0 < 0 ? -1 : r0 + (kt & (leaf - 1));
        const int ke = key - nl - nloc;
        const int extrow = s_ext[(ke >= 0 && ke < next) ? ke : 0];
        const int ownrow = own0 < 0 ? -1 : own0 + (key - nl);
        row[i] = key < nl ? leafrow : (key < nl + nloc ? ownrow : (key < N ? extrow : -1));
      }
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      ok[i] = row[i] >= 0;
      const int64_t r = ok[i] ? row[i] : 0;
      kr[i] = ldg16(kb + r * kst_b);
      vr[i] = ldg16(vb + r * vst_b);
    }
  };

  float m = kNegBig, l = 0.0f;
  float acc[EPL];
#pragma unroll
  for (int d = 0; d < EPL; ++d) acc[d] = 0.0f;

  auto consume = [&](const uint4 (&kr)[NL], const uint4 (&vr)[NL], const bool (&ok)[NL]) {
    float sc[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float kv[EPL];
      Raw16<T>::cvt(kr[i], kv);
      float d0 = 0.0f;
#pragma unroll
      for (int d = 0; d < EPL; ++d) d0 = fmaf(qv[d], kv[d], d0);
      sc[i] = d0;
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) sc[i] = group_sum<LPR>(sc[i]);
    // running max per row group (its LPR lanes see the same scores); the groups merge at the end
    float cm = kNegBig;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      sc[i] = ok[i] ? sc[i] * p.scale : kNegBig;
      cm = fmaxf(cm, sc[i]);
    }
    const float mn = fmaxf(m, cm);
    {
      const float alpha = __expf(m - mn);
#pragma unroll
      for (int d = 0; d < EPL; ++d) acc[d] *= alpha;
      l *= alpha;
    }
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const float pw = ok[i] ? __expf(sc[i] - mn) : 0.0f;
      lsum += pw;
      float vv[EPL];
      Raw16<T>::cvt(vr[i], vv);
#pragma unroll
      for (int d = 0; d < EPL; ++d) acc[d] = fmaf(pw, vv[d], acc[d]);
    }
    if (lane % LPR == 0) l += lsum;
    m = mn;
  };

  {
    constexpr int PF = 4;   // chunks in flight per wavefront
    uint4 kq[PF][NL], vq[PF][NL];
    bool okq[PF][NL];
    if constexpr (PIPE) {
      // Several workgroups per query (few queries, each wavefront's chain of round trips is the time): slot j is
      // consumed, then refilled with the chunk PF steps later, the loop unrolled over the slots so that no
      // register set is copied (a copy of registers whose loads are in flight waits for those loads, which
      // makes every chunk a full round trip).  Every fetch is issued, past the last chunk too (its keys are
      // invalid: row 0 is read and nothing is used), so every path has the same loads in flight and the wait
      // before a slot's use covers that slot only.  Measured at config 5: 0.690 against 0.711-0.718 ms/step.
#pragma unroll
      for (int j = 0; j < PF; ++j) fetch(first + j * stride, kq[j], vq[j], okq[j]);
      for (int c0 = first; c0 < nchunks; c0 += PF * stride) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
          const int c = c0 + j * stride;
          if (c < nchunks) consume(kq[j], vq[j], okq[j]);
          fetch(c + PF * stride, kq[j], vq[j], okq[j]);
        }
      }
    } else {
      // Otherwise (one workgroup per query: many queries streaming together, HBM the limit): the next chunk
      // requested before each one is consumed and the register sets shifted, which waits for the requests in
      // flight at the end of every step; measured faster here than the copy-free loop above (config 4's layer
      // attention 61-63 against 65.5 us with cold caches) and than 8 loads one chunk ahead (49.9 against 46.9 us).
#pragma unroll
      for (int j = 0; j < PF; ++j)
        if (first + j * stride < nchunks) fetch(first + j * stride, kq[j], vq[j], okq[j]);
      int c = first;
      while (c < nchunks) {
        const int cn = c + PF * stride;
        uint4 kn[NL], vn[NL];
        bool okn[NL];
        if (cn < nchunks) fetch(cn, kn, vn, okn);
        consume(kq[0], vq[0], okq[0]);
#pragma unroll
        for (int j = 0; j + 1 < PF; ++j)
#pragma unroll
          for (int i = 0; i < NL; ++i) {
            kq[j][i] = kq[j + 1][i]; vq[j][i] = vq[j + 1][i]; okq[j][i] = okq[j + 1][i];
          }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          kq[PF - 1][i] = kn[i]; vq[PF - 1][i] = vn[i]; okq[PF - 1][i] = okn[i];
        }
        c += stride;
      }
    }
  }

  // bring the row groups to the wavefront's max, then sum them
  {
    const float Mw = wave_max(m);
    const float f = __expf(m - Mw);
    l *= f;
#pragma unroll
    for (int d = 0; d < EPL; ++d) acc[d] *= f;
    m = Mw;
  }
  float L = wave_sum(l);
  // sum the accumulators of the RPI row groups: afterwards lanes 0..LPR-1 hold the full dims
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1) {
#pragma unroll
    for (int d = 0; d < EPL; ++d) acc[d] += __shfl_xor(acc[d], o, kWave);
  }
  if constexpr (SPLIT) {
    // merge the 4 wavefronts of the workgroup through LDS
    float* red = smem_f + kWavesPerBlock * attn_wave_ints(wl_pad);   // [4][D + 2]
    if (rg == 0) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) red[w * (D + 2) + 2 + ds + e] = acc[e];
    }
    if (lane == 0) {
      red[w * (D + 2)] = m;
      red[w * (D + 2) + 1] = L;
    }
    __syncthreads();
    if (w != 0) return;
    float M = kNegBig;
#pragma unroll
    for (int s = 0; s < kWavesPerBlock; ++s)
      if (red[s * (D + 2) + 1] > 0.0f) M = fmaxf(M, red[s * (D + 2)]);
    float Lt = 0.0f;
    float sc[kWavesPerBlock];
#pragma unroll
    for (int s = 0; s < kWavesPerBlock; ++s) {
      const float Ls = red[s * (D + 2) + 1];
      sc[s] = Ls > 0.0f ? __expf(red[s * (D + 2)] - M) : 0.0f;
      Lt += Ls * sc[s];
    }
    if (p.gsplit > 1) {
      float* part = p.ws + (qi * p.gsplit + g) * (D + 2);
      for (int d = lane; d < D; d += kWave) {
        float a = 0.0f;
#pragma unroll
        for (int s = 0; s < kWavesPerBlock; ++s) a += red[s * (D + 2) + 2 + d] * sc[s];
        __hip_atomic_store(part + 2 + d, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) {
        __hip_atomic_store(part, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part + 1, Lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (g == 0 && p.keys) p.keys[qi] = (float)N;
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the partial has reached memory
      int last = 0;
      if (lane == 0)
        last = __hip_atomic_fetch_add(p.cnt + qi, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(p.gsplit - 1);
      if (!__shfl(last, 0, kWave)) return;
      // last workgroup of this query: lane s holds partial s's (max, sum); gsplit <= 64
      const float* base = p.ws + qi * p.gsplit * (D + 2);
      float ms = kNegBig, Ls = 0.0f;
      if (lane < p.gsplit) {
        ms = __hip_atomic_load(base + lane * (D + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        Ls = __hip_atomic_load(base + lane * (D + 2) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const float Mq = wave_max(Ls > 0.0f ? ms : kNegBig);
      const float fac = Ls > 0.0f ? __expf(ms - Mq) : 0.0f;
      const float Lq = wave_sum(Ls * fac);
      const float inv = Lq > 0.0f ? 1.0f / Lq : 0.0f;
      float* s_fac = reinterpret_cast<float*>(s_ext);   // the static-key list is no longer needed
      s_fac[lane] = fac;
      wave_sync();
      T* orow = orow_base;
      for (int d = lane; d < D; d += kWave) {
        float a = 0.0f;
        for (int s0 = 0; s0 < p.gsplit; s0 += 8) {
          float pv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            pv[i] = s0 + i < p.gsplit ? __hip_atomic_load(base + (s0 + i) * (D + 2) + 2 + d, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (s0 + i < p.gsplit) a += pv[i] * s_fac[s0 + i];
        }
        orow[d] = from_f32<T>(a * inv);
      }
      if (lane == 0) {
        if (p.lse) p.lse[qi] = Lq > 0.0f ? Mq + __logf(Lq) : kNegBig;
        __hip_atomic_store(p.cnt + qi, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // ready for the next call
      }
      return;
    }
    const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
    T* orow = orow_base;
    for (int d = lane; d < D; d += kWave) {
      float a = 0.0f;
#pragma unroll
      for (int s = 0; s < kWavesPerBlock; ++s) a += red[s * (D + 2) + 2 + d] * sc[s];
      orow[d] = from_f32<T>(a * inv);
    }
    if (lane == 0) {
      if (p.lse) p.lse[qi] = Lt > 0.0f ? M + __logf(Lt) : kNegBig;
      if (p.keys) p.keys[qi] = (float)N;
    }
  } else {
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (rg == 0) {
      T* orow = orow_base + ds;
#pragma unroll
      for (int e = 0; e < EPL; ++e) orow[e] = from_f32<T>(acc[e] * inv);
    }
    if (lane == 0) {
      if (p.lse) p.lse[qi] = L > 0.0f ? m + __logf(L) : kNegBig;
      if (p.keys) p.keys[qi] = (float)N;
    }
  }
}


}  // namespace ta
