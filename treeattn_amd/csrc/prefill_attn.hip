// Prefill sparse attention on gfx950 matrix cores (v_mfma_f32_32x32x16_bf16 / _f16): block-sparse flash
// attention over the leaf blocks a tile of queries selected.
//
// A workgroup takes 128 consecutive queries of one (b, h), 32 per wavefront.  It marks in LDS, per leaf block
// and wavefront, which of the wavefront's queries use the block (a selected leaf block, or the query's own
// block) and which need it only for a static key (the sink, position 0, or one of the last Lw positions), and
// lists the blocks any query marked, in ascending order.  The workgroup walks the listed blocks' 32-key tiles
// together: each tile's K rows and V^T (as key pairs) are staged once in LDS for the four wavefronts, in two
// stages, with the global loads of a tile issued two tiles ahead (the workgroup's threads share them, so a
// thread holds four 16-byte pieces per tile).  A wavefront skips a tile none of its queries uses; otherwise it
// forms the transposed scores S^T = K Q^T (keys x queries), masks each (query, key) to the query's key set --
// key <= t and (block used by the query, or key = 0, or key > t - Lw) -- updates the running softmax of each
// query and accumulates O^T += V^T P^T.  The rows of the K operand are the tile's keys in the order with bits
// 2 and 3 of the row index exchanged, which puts the probabilities of each query in exactly the lanes and
// registers the B operand of the second product needs, and leaves every query's statistics (running max, sum)
// in its own lane.
//
// Keys per query are those of the vector kernel's structural mode (the reference's candidate assembly and
// dedupe, fastseg.py:367-383, then sparse_attn, fastseg.py:134-177), each key counted once.
#include "attn.hpp"

namespace ta {

typedef __bf16 pa_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pa_f16x8 __attribute__((ext_vector_type(8)));
typedef float pa_f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
__device__ __forceinline__ pa_f32x16 pa_mfma(const uint4& a, const uint4& b, pa_f32x16 c);
template <>
__device__ __forceinline__ pa_f32x16 pa_mfma<bf16_t>(const uint4& a, const uint4& b, pa_f32x16 c) {
  pa_bf16x8 av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ pa_f32x16 pa_mfma<f16_t>(const uint4& a, const uint4& b, pa_f32x16 c) {
  pa_f16x8 av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
}

template <typename T> __device__ __forceinline__ uint16_t pa_bits(float x);
template <> __device__ __forceinline__ uint16_t pa_bits<bf16_t>(float x) { return bf16_from(x).bits; }
template <> __device__ __forceinline__ uint16_t pa_bits<f16_t>(float x) {
  const f16_t h = (f16_t)x;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

constexpr int kPaQ = 128;         // queries per workgroup (32 per wavefront)
constexpr int kPaWaves = 4;
constexpr int kPaVW = 20;         // row stride (32-bit words) of the V^T tile: 16 key pairs + 4 (16-byte rows)
constexpr float kPaSlack = 8.0f;  // running-max slack of the lazy softmax rescaling (log2 units)
constexpr float kPaMaxInit = -1e20f;

// LDS of prefill_attn_kernel: two stages of [K tile (32 rows of D + 8 elements) | V^T tile (D rows of kPaVW
// words)], reused at the end for the four wavefronts' output tiles (32 rows of D + 8 elements each); then the
// per-(block, wavefront) masks and the block list (nbk-sized, dynamic).
__host__ __device__ constexpr int pa_kt_bytes(int D) { return 32 * (D + 8) * 2; }
__host__ __device__ constexpr int pa_stage_bytes(int D) { return pa_kt_bytes(D) + D * kPaVW * 4; }
__host__ __device__ constexpr int pa_lds_fixed(int D) {
  return 2 * pa_stage_bytes(D) > kPaWaves * pa_kt_bytes(D) ? 2 * pa_stage_bytes(D) : kPaWaves * pa_kt_bytes(D);
}

// Two probabilities as a packed pair of T (hardware round-to-nearest-even conversion).
template <typename T> __device__ __forceinline__ uint32_t pa_pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pa_pack2<bf16_t>(float a, float b) {
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  uint16_t ux, uy;
  __builtin_memcpy(&ux, &x, 2);
  __builtin_memcpy(&uy, &y, 2);
  return (uint32_t)ux | ((uint32_t)uy << 16);
}
template <> __device__ __forceinline__ uint32_t pa_pack2<f16_t>(float a, float b) {
  return (uint32_t)pa_bits<f16_t>(a) | ((uint32_t)pa_bits<f16_t>(b) << 16);
}

// A tile's global pieces held by one thread between its loads and its LDS writes: one or two 16-byte pieces of K
// rows, and two V rows' 16-byte pieces (one key pair, one 8-dimension column chunk).
struct PaRegs {
  uint4 k0, k1;   // k1 used when LPK == 2 (D = 128)
  uint4 v0, v1;
};

template <typename T, int D, int LEAF_LOG2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attn_kernel(AttnParams p, int nbk) {
  constexpr int LEAF = 1 << LEAF_LOG2;
  constexpr int KS = D / 16;        // k-steps of S^T = K Q^T
  constexpr int MT = D / 32;        // 32-dim row tiles of O^T
  constexpr int KT = LEAF / 32;     // 32-key tiles per block
  constexpr int CPR = D / 8;        // 16-byte chunks per key row
  constexpr int KROW = D + 8;       // K tile row stride (elements)
  constexpr int LPK = 32 * CPR / 256;   // K pieces per thread and tile
  constexpr int NVP = 16 * CPR;         // V pieces (key pair, chunk) per tile
  static_assert((LPK == 1 || LPK == 2) && 32 * CPR % 256 == 0 && NVP <= 256, "tile pieces per thread");
  extern __shared__ __align__(16) unsigned char pa_smem[];
  uint32_t* bmask = reinterpret_cast<uint32_t*>(pa_smem + pa_lds_fixed(D));   // [nbk][4] queries using block
  uint32_t* smask = bmask + kPaWaves * nbk;                                    // [nbk][4] with a static key in it
  uint16_t* blist = reinterpret_cast<uint16_t*>(smask + kPaWaves * nbk);       // [nbk] marked blocks, ascending
  __shared__ int s_t[kPaQ], s_nused[kPaQ], s_nv[kPaQ];
  __shared__ int s_wtot[kPaWaves];

  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  // Workgroups are dealt to the 8 XCDs round robin (workgroup L to XCD L % 8).  XCD x takes a contiguous
  // range of (b, h, tile) indices, so the tiles of one (b, h) run together on one XCD and share its L2
  // for the K/V blocks; the tiles of a (b, h) go latest position first (they have the most blocks).
  int bh, tile;
  {
    const int G = gridDim.x, L = blockIdx.x;
    const int x = L & 7, r = L >> 3;
    const int base = G >> 3, rem = G & 7;
    const int lam = x * base + (x < rem ? x : rem) + r;
    const int ntq = (p.Nq + kPaQ - 1) / kPaQ;
    bh = lam / ntq;
    tile = ntq - 1 - (lam - bh * ntq);
  }
  const int n0 = tile * kPaQ;
  const int b = bh / p.H, h = bh % p.H;
  const int nq = p.Nq - n0 < kPaQ ? p.Nq - n0 : kPaQ;

  for (int i = tid; i < 2 * kPaWaves * nbk; i += 256) bmask[i] = 0u;
  int tq_own = -1, nt_own = 0;
  if (tid < nq) {
    tq_own = p.tq[b * p.tq_sb + n0 + tid];
    nt_own = p.n_tree ? p.n_tree[(int64_t)bh * p.Nq + n0 + tid] : p.wl;
  }
  if (tid < kPaQ) s_nv[tid] = 0;
  __syncthreads();
  // the tile's (query, slot) entries are contiguous: count the valid ones per query (loads batched)
  const int ne = nq * p.wl;
  const int64_t ebase = ((int64_t)bh * p.Nq + n0) * p.wl;
  constexpr int EB = 4;
  for (int e0 = 0; e0 < ne; e0 += 256 * EB) {
    uint8_t vv[EB];
    // unconditional loads (clamped index), so the EB requests are in flight together
#pragma unroll
    for (int j = 0; j < EB; ++j) {
      const int e = e0 + tid + 256 * j;
      vv[j] = *(const TA_GLOBAL uint8_t*)(p.vld + ebase + (e < ne ? e : ne - 1));
    }
#pragma unroll
    for (int j = 0; j < EB; ++j)
      if (e0 + tid + 256 * j >= ne) vv[j] = 0;
#pragma unroll
    for (int j = 0; j < EB; ++j)
      if (vv[j]) atomicAdd(&s_nv[(e0 + tid + 256 * j) / p.wl], 1);
  }
  __syncthreads();
  if (tid < kPaQ) {
    int t = -1, nused = 0;
    if (tid < nq) {
      t = tq_own >= p.Tk || tq_own < 0 ? -1 : tq_own;
      const int nv = s_nv[tid];
      nused = t < 0 ? 0 : (nv < nt_own ? nv : (nt_own > 0 ? nt_own : 0));
    }
    s_t[tid] = t;
    s_nused[tid] = nused;
  }
  __syncthreads();
  // mark the blocks: selected leaf blocks and own blocks (full use, keys <= t), static-key blocks; word
  // 4 u + v holds the bits of wavefront v's 32 queries
  for (int e0 = 0; e0 < ne; e0 += 256 * EB) {
    int uu[EB];
#pragma unroll
    for (int j = 0; j < EB; ++j) {
      const int e = e0 + tid + 256 * j;
      uu[j] = *(const TA_GLOBAL int32_t*)(p.ids + ebase + (e < ne ? e : ne - 1));
    }
#pragma unroll
    for (int j = 0; j < EB; ++j) {
      const int e = e0 + tid + 256 * j;
      bool use = false;
      if (e < ne) {
        const int q = e / p.wl;
        use = e - q * p.wl < s_nused[q];
      }
      if (!use) uu[j] = -1;
    }
#pragma unroll
    for (int j = 0; j < EB; ++j) {
      const int u = uu[j];
      if (u >= 0 && u < nbk) {
        const int q = (e0 + tid + 256 * j) / p.wl;
        atomicOr(&bmask[kPaWaves * u + (q >> 5)], 1u << (q & 31));
      }
    }
  }
  if (tid < nq) {
    const int t = s_t[tid];
    if (t >= 0) {
      const int own = t >> LEAF_LOG2;
      const uint32_t bit = 1u << (tid & 31);
      const int wv = tid >> 5;
      atomicOr(&bmask[kPaWaves * own + wv], bit);
      atomicOr(&smask[wv], bit);
      const int lb = own << LEAF_LOG2;
      if (lb > 0 && t - p.Lw + 1 < lb) atomicOr(&smask[kPaWaves * (own - 1) + wv], bit);
    }
  }
  __syncthreads();
  // ascending list of marked blocks: thread tid scans [tid * per, (tid + 1) * per)
  auto marked = [&](int u) {
    uint32_t a = 0u;
#pragma unroll
    for (int v = 0; v < kPaWaves; ++v) a |= bmask[kPaWaves * u + v] | smask[kPaWaves * u + v];
    return a != 0u;
  };
  const int per = (nbk + 255) / 256;
  int cnt = 0;
  for (int i = 0; i < per; ++i) {
    const int u = tid * per + i;
    if (u < nbk && marked(u)) ++cnt;
  }
  // exclusive prefix of the counts over the workgroup (wavefront scans, then the wavefront totals)
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == kWave - 1) s_wtot[w] = incl;
  __syncthreads();
  int off = incl - cnt, U = 0;
#pragma unroll
  for (int i = 0; i < kPaWaves; ++i) {
    if (i < w) off += s_wtot[i];
    U += s_wtot[i];
  }
  for (int i = 0; i < per; ++i) {
    const int u = tid * per + i;
    if (u < nbk && marked(u)) blist[off++] = (uint16_t)u;
  }
  __syncthreads();

  // ---- main loop: the workgroup walks the listed blocks' tiles; wavefront w scores its queries 32 w ..
  const int c = lane & 31, hh = lane >> 5;
  const int qi = 32 * w + c;
  const int tc = s_t[qi];
  const bool qok = qi < nq && tc >= 0;
  uint4 qb[KS];   // B operand of S^T: query qi, dims 16s + 8hh .. + 8
  {
    const T* qr = reinterpret_cast<const T*>(p.q) + b * p.qsb + h * p.qsh + (int64_t)(n0 + (qi < nq ? qi : 0)) * p.qsn +
                  8 * hh;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = qi < nq ? *reinterpret_cast<const uint4*>(qr + 16 * s) : make_uint4(0, 0, 0, 0);
  }
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.ksb + h * p.ksh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.vsb + h * p.vsh;
  const float sl2 = p.scale * 1.4426950408889634f;                     // scores in log2 units
  // A-operand row rho of S^T holds key pi(rho) = rho with bits 2 and 3 exchanged
  const int rho = lane & 31;
  const int krow = (rho & ~12) | ((rho & 4) << 1) | ((rho & 8) >> 1);

  // running max in log2 units; it starts far above the masked score kNegBig, so a masked key always gets
  // probability 2^(kNegBig - m) = 0, and far below any real score, which replaces it on first sight
  float m = kPaMaxInit, l = 0.0f;
  int kcount = 0;
  pa_f32x16 o[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[mt][i] = 0.0f;

  const int nit = U * KT;
  // row offsets in elements fit 32 bits (checked on the host); keys past the sequence read its last row and
  // are masked
  const int kst = (int)p.kst, vst = (int)p.vst, tlast = p.Tk - 1;
  // this thread's pieces: K row tid / CPR + 8 j (chunk tid % CPR); V key pair vp / CPR, chunk vp % CPR
  const int kr0 = tid / CPR, kc0 = tid % CPR;
  const int vp = tid % NVP, vkp = vp / CPR, vdc = vp % CPR;
  auto tile_key0 = [&](int it) __attribute__((always_inline)) {
    const int itc = it < nit ? it : nit - 1;
    return ((int)blist[itc / KT] << LEAF_LOG2) + (itc % KT) * 32;
  };
  auto gload = [&](int it) __attribute__((always_inline)) {
    PaRegs r;
    const int key0 = tile_key0(it);
    r.k0 = *reinterpret_cast<const uint4*>(kbase + (uint32_t)(min(key0 + kr0, tlast) * kst + 8 * kc0));
    if constexpr (LPK == 2)
      r.k1 = *reinterpret_cast<const uint4*>(kbase + (uint32_t)(min(key0 + kr0 + 256 / CPR, tlast) * kst + 8 * kc0));
    const int p0 = key0 + 2 * vkp;
    r.v0 = *reinterpret_cast<const uint4*>(vbase + (uint32_t)(min(p0, tlast) * vst + 8 * vdc));
    r.v1 = *reinterpret_cast<const uint4*>(vbase + (uint32_t)(min(p0 + 1, tlast) * vst + 8 * vdc));
    return r;
  };
  auto stage_k = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<T*>(pa_smem + sb * pa_stage_bytes(D)); };
  auto stage_vt = [&](int sb) __attribute__((always_inline)) { return reinterpret_cast<uint32_t*>(pa_smem + sb * pa_stage_bytes(D) + pa_kt_bytes(D)); };
  auto lwrite = [&](const PaRegs r, int sb) __attribute__((always_inline)) {
    T* kt = stage_k(sb);
    *reinterpret_cast<uint4*>(kt + kr0 * KROW + 8 * kc0) = r.k0;
    if constexpr (LPK == 2) *reinterpret_cast<uint4*>(kt + (kr0 + 256 / CPR) * KROW + 8 * kc0) = r.k1;
    if (tid < NVP) {
      // V^T as key pairs: word (d, kp) = (V[2 kp][d], V[2 kp + 1][d])
      uint32_t* vt = stage_vt(sb);
      // components by name (a pointer into the registers would put them in scratch memory)
      const uint32_t a[4] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w};
      const uint32_t bq[4] = {r.v1.x, r.v1.y, r.v1.z, r.v1.w};
#pragma unroll
      for (int m2 = 0; m2 < 4; ++m2) {
        vt[(8 * vdc + 2 * m2) * kPaVW + vkp] = __builtin_amdgcn_perm(bq[m2], a[m2], 0x05040100u);
        vt[(8 * vdc + 2 * m2 + 1) * kPaVW + vkp] = __builtin_amdgcn_perm(bq[m2], a[m2], 0x07060302u);
      }
    }
  };
  auto compute = [&](int it, int sb) __attribute__((always_inline)) {
    if (it >= nit) return;
    const int u = blist[it / KT];
    const int key0 = (u << LEAF_LOG2) + (it % KT) * 32;
    const bool use = ((bmask[kPaWaves * u + w] >> c) & 1u) != 0u;
    // mask: register i holds key key0 + 16 (i / 8) + 8 hh + i % 8 for query qi.  A tile is wholly in
    // (a used block ending at or before t) or wholly out for a query unless it holds the query's position
    // or a static key; when that holds for every query of the wavefront no per-key test is needed.
    const bool full = qok && use && key0 + 31 <= tc;
    const bool stat = qok && key0 <= tc && (key0 == 0 || key0 + 31 > tc - p.Lw);
    const bool none = !qok || key0 > tc || (!use && !stat);
    if (__all(none)) return;   // no query of this wavefront takes a key of the tile
    const T* kt = stage_k(sb);
    uint4 ka[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) ka[s] = *reinterpret_cast<const uint4*>(kt + krow * KROW + 16 * s + 8 * hh);
    pa_f32x16 st;
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) st = pa_mfma<T>(ka[s], qb[s], st);
    float pv[16];
    if (__all(full || none)) {
      const float f = full ? sl2 : 0.0f, z = full ? 0.0f : kNegBig;
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = fmaf(st[i], f, z);
      kcount += full ? 16 : 0;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int pos = key0 + 16 * (i >> 3) + 8 * hh + (i & 7);
        const bool inc = qok && pos <= tc && (use || pos == 0 || pos > tc - p.Lw);
        pv[i] = inc ? st[i] * sl2 : kNegBig;
        kcount += inc;
      }
    }
    float mx = pv[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, pv[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    // lazy rescaling: keep the running max until some query's tile max exceeds it by more than kPaSlack
    // (probabilities then stay below 2^kPaSlack); l and O share the max, so the result is the same
    if (__any(mx > m + kPaSlack)) {
      const float mn = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][i] *= alpha;
      m = mn;
    }
    uint4 pb[2];
    {
      uint32_t wds[8];
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = __builtin_amdgcn_exp2f(pv[i] - m);       // masked keys: 2^(-1e30) = 0
        const float p1 = __builtin_amdgcn_exp2f(pv[i + 1] - m);
        l += p0 + p1;
        wds[i >> 1] = pa_pack2<T>(p0, p1);
      }
      pb[0] = make_uint4(wds[0], wds[1], wds[2], wds[3]);
      pb[1] = make_uint4(wds[4], wds[5], wds[6], wds[7]);
    }
    const uint32_t* vt = stage_vt(sb);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint4 va = *reinterpret_cast<const uint4*>(vt + (32 * mt + rho) * kPaVW + 8 * s2 + 4 * hh);
        o[mt] = pa_mfma<T>(va, pb[s2], o[mt]);
      }
    }
  };
  if (nit > 0) {
    // tiles it and it + 1 are in registers (A, B) or LDS; each half-pass requests tile it + 2, scores the
    // stage of tile it and writes tile it + 1 (loaded a half-pass earlier) into the other stage
    PaRegs ra = gload(0);
    PaRegs rb = gload(1);
    lwrite(ra, 0);
    lds_barrier();
    for (int it = 0; it < nit; it += 2) {
      ra = gload(it + 2);
      compute(it, 0);
      lwrite(rb, 1);
      lds_barrier();
      rb = gload(it + 3);
      compute(it + 1, 1);
      lwrite(ra, 0);
      lds_barrier();
    }
  }

  // ---- each wavefront writes its 32 queries (halves of a lane pair hold disjoint keys of the same query)
  l += __shfl_xor(l, 32, kWave);
  kcount += __shfl_xor(kcount, 32, kWave);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  uint16_t* ot = reinterpret_cast<uint16_t*>(pa_smem) + w * 32 * KROW;   // [32][D + 8], this wavefront's
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      ot[c * KROW + 32 * mt + 8 * (i >> 2) + 4 * hh + (i & 3)] = pa_bits<T>(o[mt][i] * inv);
  if (hh == 0 && qi < nq) {
    const int64_t gi = (int64_t)bh * p.Nq + n0 + qi;
    if (p.lse) p.lse[gi] = l > 0.0f ? (m + __log2f(l)) * 0.6931471805599453f : kNegBig;
    if (p.keys) p.keys[gi] = (float)kcount;
  }
  wave_sync();
  const int nw = nq - 32 * w < 0 ? 0 : (nq - 32 * w > 32 ? 32 : nq - 32 * w);
  for (int e = lane; e < nw * CPR; e += kWave) {
    const int r = e / CPR, dc = e - r * CPR;
    T* orow = reinterpret_cast<T*>(p.out) + b * p.osb + h * p.osh + (int64_t)(n0 + 32 * w + r) * p.osn;
    *reinterpret_cast<uint4*>(orow + 8 * dc) = *reinterpret_cast<const uint4*>(ot + r * KROW + 8 * dc);
  }
}

}  // namespace ta

using namespace ta;

int ta::prefill_attn_mfma(const AttnParams& p, int B, int dtype, int D, hipStream_t st) {
  if (p.cand || p.gsplit != 1 || (dtype != TA_BF16 && dtype != TA_F16) || (D != 64 && D != 128) ||
      p.leaf_log2 < 5 || p.leaf_log2 > 7 || p.Lw > (1 << p.leaf_log2) || p.Nq <= 0 || p.wl > 1024)
    return TA_ERR_UNSUPPORTED;
  const int nbk = (p.Tk + (1 << p.leaf_log2) - 1) >> p.leaf_log2;
  if (nbk > 65535) return TA_ERR_UNSUPPORTED;
  const size_t lds = (size_t)pa_lds_fixed(D) + (size_t)nbk * (2 * kPaWaves * 4 + 2) + 16;
  if (lds > 96 * 1024) return TA_ERR_UNSUPPORTED;
  if ((p.osn * 2) % 16 || (p.osh * 2) % 16 || (p.osb * 2) % 16 || (uintptr_t)p.out % 16) return TA_ERR_UNSUPPORTED;
  // 32-bit row offsets within one (b, h)
  if (p.kst <= 0 || p.vst <= 0 || (int64_t)p.Tk * p.kst >= (int64_t)1 << 31 || (int64_t)p.Tk * p.vst >= (int64_t)1 << 31)
    return TA_ERR_UNSUPPORTED;
  const int64_t nwg = (int64_t)((p.Nq + kPaQ - 1) / kPaQ) * B * p.H;
  if (nwg > 0x7fffffff) return TA_ERR_UNSUPPORTED;
  dim3 grid((unsigned)nwg);
  const dim3 blk(kPaWaves * kWave);
#define TA_PA(T, DD, LL) hipLaunchKernelGGL((prefill_attn_kernel<T, DD, LL>), grid, blk, lds, st, p, nbk)
#define TA_PA_L(T, DD)                        \
  if (p.leaf_log2 == 5) TA_PA(T, DD, 5);      \
  else if (p.leaf_log2 == 6) TA_PA(T, DD, 6); \
  else TA_PA(T, DD, 7);
  if (dtype == TA_BF16) {
    if (D == 64) { TA_PA_L(bf16_t, 64) } else { TA_PA_L(bf16_t, 128) }
  } else {
    if (D == 64) { TA_PA_L(f16_t, 64) } else { TA_PA_L(f16_t, 128) }
  }
#undef TA_PA_L
#undef TA_PA
  return check_launch("prefill_attn_kernel");
}
