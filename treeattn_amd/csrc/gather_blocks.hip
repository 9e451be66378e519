// Leaf-block gather-dot on gfx950 MFMA: out[b,h,n, c*block + j] = scale * q[b,h,n] . K[b,h, blk[b,h,n,c]*block + j].
//
// Block-major: a workgroup takes Q consecutive queries of one (b, h) (512 at D = 64, 128 at D = 128: as many as
// the LDS copy of their rows allows) and turns their (query, slot) pairs into
// per-block lists, so every score the matrix cores compute belongs to a pair that selected the block.
//
//  * Set-up: the workgroup's query rows are copied into LDS (every piece requested before the first is stored);
//    its pairs (at most Q * 16, their block ids all requested before they are counted) are sorted by block
//    id with a counting sort in LDS (a count per block, one scan giving each block its list offset and its
//    number of chunks, then each pair placed with an LDS atomic).  A chunk is up to 128 pairs that selected the
//    same block; an item is a chunk and one 32-key tile of its block.
//  * The wavefronts take contiguous runs of chunks.  For an item a wavefront requests the key tile once (from
//    global memory; the head's keys stay in the XCD's L2) as the MFMA A operand and runs the chunk's 32-pair
//    sub-chunks against it: their query rows from LDS as the B operand, S^T = K_tile . Q^T with
//    v_mfma_f32_32x32x16 (lane (p, hh) holds keys 8 i + 4 hh + r of pair p).  One tile read serving up to 128
//    pairs is what keeps the L2 traffic of the tiles well below the scores' (a 32-pair chunk read a 4 KB tile
//    for 4 KB of scores).  The 32 x 32 scores pass through the wavefront's own LDS tile so that each store
//    instruction writes eight pairs' 128-byte runs of consecutive keys (whole lines).
//  * The key tile of item i + 2 is requested before item i's stores, with three register sets in rotation
//    (the loop runs three items per pass): the vector-memory counter counts stores too, so a wait for a key tile
//    then covers only stores issued at least two items earlier, and the stores drain while later items compute.
//    Stores go through a buffer resource over the workgroup's output rows; lanes past a sub-chunk's count get an
//    offset past its end, which the hardware drops, so every store is issued unconditionally.
//
// The products of bf16 / f16 values are exact in float32 and the sum over D is taken by the MFMA, so scores
// agree with a sequential float32 sum to a few ulps (not bit for bit).  Each output column of an MFMA depends only
// on its own operand column, so a pair's scores do not depend on which pairs share its chunk.
#include "common.hpp"

namespace ta {

typedef __bf16 bf16x8_g __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_g __attribute__((ext_vector_type(8)));
typedef float f32x16_g __attribute__((ext_vector_type(16)));
typedef unsigned int gd_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGdMaxBlocks = 8192;      // blocks per (b, h) (M / block): the per-block counts (+2) fit the LDS union
constexpr int kGdMaxSlots = 16;         // selected blocks per query

template <typename T>
__device__ __forceinline__ f32x16_g mfma32(const uint4& a, const uint4& b, f32x16_g c);
template <>
__device__ __forceinline__ f32x16_g mfma32<bf16_t>(const uint4& a, const uint4& b, f32x16_g c) {
  bf16x8_g av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16_g mfma32<f16_t>(const uint4& a, const uint4& b, f32x16_g c) {
  f16x8_g av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, c, 0, 0, 0);
}

constexpr int kGpWaves = 8;
constexpr int kGpThreads = kGpWaves * kWave;
// Queries per workgroup: as many as the LDS copy of their rows allows (512 rows of D = 64, 128 of D = 128).
// More queries per workgroup means more pairs per block, so each key tile read from the L2 serves more chunks.
template <int D> struct GpShape {
  static constexpr int Q = D == 64 ? 512 : 128;
  static constexpr int MaxPairs = Q * kGdMaxSlots;
};
constexpr int kGpRow = 36;                                 // staging row stride in floats (32 + 4 of padding)
constexpr int kGpStage = 32 * kGpRow;                      // floats per wavefront staging tile

template <typename T, int D, int BLOCK>
__global__ __launch_bounds__(kGpThreads) void gather_pairs_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qsn, const T* __restrict__ K, int64_t ksb,
    int64_t ksh, int64_t ksn, const int32_t* __restrict__ blk, int H, int N, int nblocks, int NB, int ntile,
    float scale, float* __restrict__ out) {
  constexpr int Q = GpShape<D>::Q, MaxPairs = GpShape<D>::MaxPairs;
  constexpr int KS = D / 16;         // MFMA k-steps
  constexpr int KT = BLOCK / 32;     // 32-key tiles per block
  constexpr int kUnion = (kGdMaxBlocks + 2 > kGpWaves * kGpStage ? kGdMaxBlocks + 2 : kGpWaves * kGpStage);
  static_assert(MaxPairs % kGpThreads == 0, "pairs per thread");
  // counts / offsets per block during the sort, then the wavefronts' staging tiles
  __shared__ __attribute__((aligned(16))) uint32_t uni[kUnion];
  __shared__ uint16_t plist[MaxPairs];      // (query << 4 | slot), grouped by block
  __shared__ uint32_t chunk[MaxPairs];      // list << 18 | start << 5 (the count: up to the next start)
  __shared__ uint32_t wsum[kGpWaves];
  __shared__ uint32_t s_tot;
  __shared__ __attribute__((aligned(16))) T qs[Q * (D + 8)];   // the workgroup's query rows

  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  // XCD-aware order: workgroup x runs on XCD x % 8; the tiles of one (b, h) go to one XCD so its L2 holds that
  // head's keys and queries
  const int G = gridDim.x, x = blockIdx.x;
  const int base = G / 8, rem = G % 8, xcd = x % 8;
  const int lam = xcd * base + (xcd < rem ? xcd : rem) + x / 8;
  const int bh = lam / ntile;
  const int n0 = (lam - bh * ntile) * Q;
  const int b = bh / H, h = bh - b * H;
  const int nq = N - n0 < Q ? N - n0 : Q;
  const int npairs = nq * NB;

  {
    // every 16-byte piece of the workgroup's query rows requested before any is stored (a load-store pair per
    // piece in a loop would wait for each load in turn)
    constexpr int CPR = D / 8;
    constexpr int NQL = Q * CPR / kGpThreads;
    static_assert(Q * CPR % kGpThreads == 0, "query pieces per thread");
    const T* qb0 = q + b * qsb + h * qsh + (int64_t)n0 * qsn;
    uint4 piece[NQL];
#pragma unroll
    for (int k = 0; k < NQL; ++k) {
      const int e = tid + k * kGpThreads;
      const int r = e / CPR, cc = e - r * CPR;
      piece[k] = ldg16(qb0 + (int64_t)(r < nq ? r : nq - 1) * qsn + 8 * cc);
    }
#pragma unroll
    for (int k = 0; k < NQL; ++k) {
      const int e = tid + k * kGpThreads;
      const int r = e / CPR, cc = e - r * CPR;
      if (r < nq) *reinterpret_cast<uint4*>(qs + r * (D + 8) + 8 * cc) = piece[k];
    }
  }
  // 1. counts per block.  The reference clamps every key position into [0, M - 1] (cand = blk * block + j,
  // fastseg.py:121): a negative id's keys are all row 0 and an id past the end all row M - 1, so those pairs go
  // to two extra lists, nblocks and nblocks + 1
  const int nlist = nblocks + 2;
  for (int i = tid; i < nlist; i += kGpThreads) uni[i] = 0u;
  __syncthreads();
  constexpr int PPT = MaxPairs / kGpThreads;
  int pid[PPT];
  const int32_t* brow = blk + ((int64_t)bh * N + n0) * NB;
  // all of this thread's block ids requested first, then counted (a load then an LDS atomic per pair in one loop
  // would wait for each load in turn)
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int pi = tid + k * kGpThreads;
    pid[k] = *(const TA_GLOBAL int32_t*)(brow + (pi < npairs ? pi : 0));
  }
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int pi = tid + k * kGpThreads;
    int v = -1;
    if (pi < npairs) {
      v = pid[k];
      v = v < 0 ? nblocks : (v >= nblocks ? nblocks + 1 : v);
      atomicAdd(&uni[v], 1u);
    }
    pid[k] = v;
  }
  __syncthreads();
  // 2. one scan over the blocks of (chunks << 16 | count): each thread takes E consecutive blocks
  const int E = (nlist + kGpThreads - 1) / kGpThreads;
  const int j0 = tid * E;
  uint32_t loc = 0;
  for (int e = 0; e < E; ++e) {
    const int j = j0 + e;
    if (j < nlist) {
      const uint32_t c = uni[j];
      loc += (((c + 127u) >> 7) << 16) | c;
    }
  }
  uint32_t inc = loc;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t y = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += y;
  }
  if (lane == kWave - 1) wsum[w] = inc;
  __syncthreads();
  uint32_t wpre = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kGpWaves; ++i) {
    const uint32_t s = wsum[i];
    wpre += i < w ? s : 0u;
    tot += s;
  }
  uint32_t run = wpre + inc - loc;    // exclusive prefix of this thread's first block
  for (int e = 0; e < E; ++e) {
    const int j = j0 + e;
    if (j < nlist) {
      const uint32_t c = uni[j];
      const uint32_t st = run & 0xffffu, cs = run >> 16;
      for (uint32_t k = 0; 128u * k < c; ++k) chunk[cs + k] = ((uint32_t)j << 18) | ((st + 128u * k) << 5);
      uni[j] = st;    // becomes the running fill position
      run += (((c + 127u) >> 7) << 16) | c;
    }
  }
  if (tid == 0) s_tot = tot;
  __syncthreads();
  // 3. place every pair in its block's list
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int pi = tid + k * kGpThreads;
    if (pid[k] >= 0) {
      const uint32_t pos = atomicAdd(&uni[pid[k]], 1u);
      const int nl = pi / NB, sl = pi - nl * NB;
      plist[pos] = (uint16_t)((nl << 4) | sl);
    }
  }
  __syncthreads();   // lists complete; uni is now the staging area
  const int nchunk = (int)(s_tot >> 16);
  const int c0 = (int)(((int64_t)nchunk * w) / kGpWaves), c1 = (int)(((int64_t)nchunk * (w + 1)) / kGpWaves);

  float* stg = reinterpret_cast<float*>(uni) + w * kGpStage;
  const int p = lane & 31, hh = lane >> 5;
  const T* kbase = K + b * ksb + h * ksh + 8 * hh;
  float* obase = out + ((int64_t)bh * N + n0) * NB * BLOCK;
  // stores through a buffer resource over the workgroup's output rows: a lane past the chunk's count gets an
  // offset past the end, which the hardware drops, so every store is issued unconditionally
  const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(obase, 0, nq * NB * BLOCK * 4, 0x00020000);
  const int rP = lane >> 3, rc = lane & 7;
  // item i = (chunk c0 + i / KT, key tile i % KT); a chunk's pairs run from its start to the next chunk's (the
  // chunks partition the block-sorted list in order)
  const int nit = (c1 - c0) * KT;
  auto item_chunk = [&](int i) { return c0 + i / KT; };
  auto item_kt = [&](int i) { return i % KT; };
  auto cstart = [&](int c) { return c < nchunk ? (int)((chunk[c] >> 5) & 0x1fffu) : npairs; };
  auto kload = [&](int i, uint4 (&kk)[KS]) {
    const int cc = item_chunk(i), kt = item_kt(i);
    const int c = cc < c1 ? cc : c1 - 1;
    const int j = (int)(chunk[c] >> 18);
    const int64_t row = j < nblocks ? (int64_t)j * BLOCK + 32 * kt + p : (j == nblocks ? 0 : (int64_t)nblocks * BLOCK - 1);
    const T* kr = kbase + row * ksn;
#pragma unroll
    for (int s = 0; s < KS; ++s) kk[s] = ldg16(kr + 16 * s);
  };
  // one item: scores from the K tile in cur, the next item's tile requested into nxt, then the stores; the
  // loop runs two items per pass with the two register sets alternating (an odd count is padded by an item
  // whose stores are all dropped), so no register copy waits for a load issued in the same pass
  // item i with its key tile in ck; the key tile of item i + 2 is requested into nk before this item's stores, so
  // a wait for a tile covers only stores issued at least two items earlier
  // item i from its key tile in ck: the chunk's pairs in 32-pair sub-chunks, each scored, transposed and stored;
  // the key tile of item i + 2 is requested into nk first
  auto item = [&](int i, const uint4 (&ck)[KS], uint4 (&nk)[KS]) {
    const int iv = i < nit ? i : nit - 1;
    const int cc = item_chunk(iv), kt = item_kt(iv);
    const int c = cc < c1 ? cc : c1 - 1;
    const int st = cstart(c);
    const int cnt = (i < nit && cc < c1) ? cstart(c + 1) - st : 0;
    kload(iv + 2 < nit ? iv + 2 : nit - 1, nk);
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const int sc = cnt - 32 * sb < 0 ? 0 : (cnt - 32 * sb > 32 ? 32 : cnt - 32 * sb);
      if (sb > 0 && sc == 0) continue;   // past the chunk's pairs
      const int s0 = sc > 0 ? st + 32 * sb : st;
      const int code = plist[s0 + (p < sc ? p : 0)];
      const uint4* qr = reinterpret_cast<const uint4*>(qs + (code >> 4) * (D + 8)) + hh;
      uint4 qb[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) qb[s] = qr[2 * s];
      f32x16_g acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mfma32<T>(ck[s], qb[s], acc);
      int orow[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int P = 8 * u + rP;
        const int cd = plist[s0 + (P < sc ? P : 0)];
        const int o = (((cd >> 4) * NB + (cd & 15)) * BLOCK + 4 * rc + 32 * kt) * 4;
        orow[u] = P < sc ? o : 0x7fffff00;
      }
#pragma unroll
      for (int a2 = 0; a2 < 4; ++a2) {
        const float4 v = make_float4(acc[4 * a2] * scale, acc[4 * a2 + 1] * scale, acc[4 * a2 + 2] * scale,
                                     acc[4 * a2 + 3] * scale);
        *reinterpret_cast<float4*>(stg + p * kGpRow + 8 * a2 + 4 * hh) = v;
      }
      wave_sync();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 v = *reinterpret_cast<const float4*>(stg + (8 * u + rP) * kGpRow + 4 * rc);
        gd_u32x4 vv = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(vv, orsrc, orow[u], 0, 0);
      }
      wave_sync();
    }
  };
  uint4 k0[KS], k1[KS], k2[KS];
  if (nit > 0) {
    // three register sets in rotation; the first item is peeled so that every way into the loop ends with a
    // tile request followed by stores
    kload(0, k0);
    kload(nit > 1 ? 1 : 0, k1);
    item(0, k0, k2);
    for (int i = 1; i < nit; i += 3) {
      item(i, k1, k0);
      item(i + 1, k2, k1);
      item(i + 2, k0, k2);
    }
  }
}

}  // namespace ta

using namespace ta;

// Fast path of ta_gather_dot_blocks (bf16/f16, D in {64, 128}, block in {32, 64, 128}); returns
// TA_ERR_UNSUPPORTED for other shapes so the caller uses the canonical-order kernel.
int ta::gather_blocks_mfma(const void* q, const void* K, int dtype, int64_t qsb, int64_t qsh, int64_t qsn,
                           int64_t ksb, int64_t ksh, int64_t ksn, const int32_t* blk, int B, int H, int N, int M,
                           int NB, int block, int D, float scale, float* out, void* stream) {
  if ((dtype != TA_BF16 && dtype != TA_F16) || (D != 64 && D != 128) || (block != 32 && block != 64 && block != 128) ||
      NB > kGdMaxSlots || M / block > kGdMaxBlocks || M % block || NB <= 0 || M <= 0)
    return TA_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)K | (uintptr_t)out) % 16 || (qsb | qsh | qsn | ksb | ksh | ksn) % 8)
    return TA_ERR_UNSUPPORTED;
  if (N == 0) return TA_OK;
  hipStream_t st = (hipStream_t)stream;
  const int nblocks = M / block;
  const int qpw = D == 64 ? GpShape<64>::Q : GpShape<128>::Q;
  const int ntp = (N + qpw - 1) / qpw;
  const int64_t nwp = (int64_t)ntp * B * H;
  if (nwp > 0x7fffffff) return TA_ERR_UNSUPPORTED;
#define TA_GP(T, DD, BL)                                                                                        \
  hipLaunchKernelGGL((gather_pairs_kernel<T, DD, BL>), dim3((unsigned)nwp), dim3(kGpThreads), 0, st,           \
                     (const T*)q, qsb, qsh, qsn, (const T*)K, ksb, ksh, ksn, blk, H, N, nblocks, NB, ntp, scale, out)
#define TA_GP_BL(T, DD)                  \
  if (block == 32) TA_GP(T, DD, 32);     \
  else if (block == 64) TA_GP(T, DD, 64); \
  else TA_GP(T, DD, 128);
  if (dtype == TA_BF16) {
    if (D == 64) { TA_GP_BL(bf16_t, 64) } else { TA_GP_BL(bf16_t, 128) }
  } else {
    if (D == 64) { TA_GP_BL(f16_t, 64) } else { TA_GP_BL(f16_t, 128) }
  }
#undef TA_GP_BL
#undef TA_GP
  return check_launch("gather_pairs_kernel");
}
