// Leaf-block gather-dot on gfx950 MFMA: out[b,h,n, c*block + j] = scale * q[b,h,n] . K[b,h, blk[b,h,n,c]*block + j].
//
// A workgroup takes 128 consecutive queries of one (b, h) and runs five wavefronts: four consumers, each
// owning 32 of the queries, and one producer.
//
//  * Set-up: each consumer lane holds the NB block ids of its query in registers and marks them in an LDS
//    bitmap of the head's blocks; wavefront 0 lists the marked blocks in ascending order.  The work is a
//    list of items, one per (distinct block, 32-key tile), walked in stages of NI items.
//  * Producer: copies the K tiles of stage s + NBUF - 1 straight into an LDS ring buffer with
//    global_load_lds_dwordx4 (no registers), waits for stage s + 1 to have landed and joins the stage
//    barrier.  It issues loads only, so its vmcnt waits never cover a store.
//  * Consumers: every consumer takes every item of the stage for its own 32 queries.  Each lane compares its
//    query's block ids with the stage's blocks (a mask of the slots that selected each); a block none of
//    the 32 queries selected is skipped.  Otherwise the consumer computes the transposed scores
//    S^T = K_tile . Q_tile^T with v_mfma_f32_32x32x16 (the tile from LDS as the A operand, the queries in
//    registers as the B operand).  In that result lane (q, h) holds, in each group of four accumulator
//    registers, four consecutive keys of its own query q, so it writes them straight to its output row with
//    one 16-byte store per group (the two lanes of a query fill 32 bytes per store, a 128-byte run per four
//    stores).  Stores go through a buffer resource whose range is the consumer's rows: the stores of
//    queries that did not select the block get an offset past the end and are dropped, so there is no
//    branch per store.  Consumers issue no loads from global memory inside the loop, so no wait of theirs
//    covers the stores: the stores drain while the next stages compute.
//
// Each K tile is read from global memory once per 128 queries.  It is stored in the ring with its 16-byte
// chunks permuted per row (chunk c of row r at position c ^ (r & 7)) so the B-operand reads are free of bank
// conflicts.  The products of bf16 / f16 values are exact in float32 and the sum over D is taken by the MFMA,
// so scores agree with a sequential float32 sum to a few ulps (not bit for bit).  The kernel is bound by the
// float32 output writes.
#include "common.hpp"

namespace ta {

typedef __bf16 bf16x8_g __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_g __attribute__((ext_vector_type(8)));
typedef float f32x16_g __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kGdMaxBlocks = 8192;      // blocks per (b, h) the bitmap can mark (M / block); ids fit 16 bits
constexpr int kGdMaxSlots = 16;         // selected blocks per query
constexpr int kGdCons = 7;              // consumer wavefronts (with the producer, 8 per workgroup)
constexpr int kGdQ = 32 * kGdCons;      // queries per workgroup
constexpr int kGdThreads = (kGdCons + 1) * kWave;
constexpr int kGdMaxDistinct = kGdQ * kGdMaxSlots < kGdMaxBlocks ? kGdQ * kGdMaxSlots : kGdMaxBlocks;

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

// s_waitcnt vmcnt(N) with the LDS and export counters left alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Exclusive prefix sum over one wavefront; returns the lane's exclusive prefix, total in *tot.
__device__ __forceinline__ int wave_exscan(int v, int* tot) {
  const int lane = lane_id();
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  *tot = __shfl(x, kWave - 1, kWave);
  return x - v;
}

typedef unsigned int gd_u32x4 __attribute__((ext_vector_type(4)));

// Ring geometry per head dimension: NI items per stage, NBUF stages in the ring.
template <int D> struct GdRing;
template <> struct GdRing<64> { static constexpr int NI = 4, NBUF = 3; };
template <> struct GdRing<128> { static constexpr int NI = 2, NBUF = 3; };

template <typename T, int D, int BLOCK>
__global__ __launch_bounds__(kGdThreads) void gather_blocks_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, int64_t qsn, const T* __restrict__ K, int64_t ksb,
    int64_t ksh, int64_t ksn, const int32_t* __restrict__ blk, int H, int N, int nblocks, int NB, int ntile,
    float scale, float* __restrict__ out) {
  constexpr int NI = GdRing<D>::NI, NBUF = GdRing<D>::NBUF;
  constexpr int KS = D / 16;                 // MFMA k-steps
  constexpr int KT = BLOCK / 32;             // 32-key tiles per block
  constexpr int CPR = D / 8;                 // 16-byte chunks per key row
  constexpr int RPL = kWave / CPR;           // key rows per 64-lane copy
  constexpr int LPI = 32 / RPL;              // copies per item (tile of 32 rows)
  constexpr int LPS = LPI * NI;              // copies per stage
  constexpr int TILE4 = 32 * CPR;            // uint4 per K tile
  constexpr int NWORDS = kGdMaxBlocks / 32;
  static_assert(LPS * (NBUF - 2) < 64, "outstanding copies exceed vmcnt");
  static_assert(NBUF * NI * TILE4 * 4 >= NWORDS, "the bitmap must fit in the ring");
  __shared__ uint4 ring[NBUF * NI * TILE4];
  __shared__ uint16_t ublk[kGdMaxDistinct];        // distinct blocks, ascending
  constexpr int NBS = NI >= KT ? NI / KT : 1;     // blocks per stage
  __shared__ int s_nu;                             // number of distinct blocks

  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  // XCD-aware order: workgroup x runs on XCD x % 8; consecutive logical indices (tiles of one (b, h)) are
  // given to one XCD so its L2 holds that head's keys.  Within a head the longest tiles go first.
  const int G = gridDim.x, x = blockIdx.x;
  const int base = G / 8, rem = G % 8, xcd = x % 8;
  const int lam = xcd * base + (xcd < rem ? xcd : rem) + x / 8;
  const int bh = lam / ntile;
  const int n0 = (ntile - 1 - (lam - bh * ntile)) * kGdQ;
  const int b = bh / H, h = bh - b * H;
  const int nq = N - n0 < kGdQ ? N - n0 : kGdQ;
  const int nwords = (nblocks + 31) / 32;

  // consumers: their 32 queries as the MFMA A operand (lane -> query lane % 32, dims 16 s + 8 (lane / 32) ..)
  // and the block ids of query lane % 32 (-1 for slots past NB and rows past the last query, whose scores
  // are never written out; their A rows repeat the first query)
  const int rq = 32 * w + (lane & 31), hh = lane >> 5;
  const bool qok = rq < nq;
  uint4 qa[KS];
  int ids[kGdMaxSlots];
  uint32_t* used = reinterpret_cast<uint32_t*>(ring);          // NWORDS: bitmap of selected blocks
  for (int i = tid; i < NWORDS; i += kGdThreads) used[i] = 0u;
  if (w < kGdCons) {
    const T* qr = q + b * qsb + h * qsh + (int64_t)(n0 + (qok ? rq : 0)) * qsn + 8 * hh;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = *reinterpret_cast<const uint4*>(qr + 16 * s);
    const int32_t* brow = blk + ((int64_t)bh * N + n0 + (qok ? rq : 0)) * NB;
#pragma unroll
    for (int s = 0; s < kGdMaxSlots; ++s) ids[s] = brow[s < NB ? s : 0];
#pragma unroll
    for (int s = 0; s < kGdMaxSlots; ++s) {
      const int v = ids[s] < 0 ? 0 : (ids[s] >= nblocks ? nblocks - 1 : ids[s]);
      ids[s] = (qok && s < NB) ? v : -1;
    }
  }
  __syncthreads();
  // the ids packed two per register (16 bits each, 0xffff for an unused slot; block ids are below 8192)
  uint32_t ids2[kGdMaxSlots / 2];
  if (w < kGdCons) {
    if (hh == 0) {
#pragma unroll
      for (int s = 0; s < kGdMaxSlots; ++s)
        if (ids[s] >= 0) atomicOr(&used[ids[s] >> 5], 1u << (ids[s] & 31));
    }
#pragma unroll
    for (int s = 0; s < kGdMaxSlots / 2; ++s)
      ids2[s] = ((uint32_t)ids[2 * s] & 0xffffu) | ((uint32_t)ids[2 * s + 1] << 16);
  }
  __syncthreads();
  // wavefront 0 lists the marked blocks: lane l owns words 4l .. 4l + 3
  if (w == 0) {
    int c[4], s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int wd = 4 * lane + k;
      c[k] = wd < nwords ? __popc(used[wd]) : 0;
      s += c[k];
    }
    int tot;
    int pre = wave_exscan(s, &tot);
    if (lane == 0) s_nu = tot;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int wd = 4 * lane + k;
      if (wd < nwords) {
        uint32_t bits = used[wd];
        int p = pre;
        while (bits) {
          ublk[p++] = (uint16_t)(32 * wd + __ffs(bits) - 1);
          bits &= bits - 1;
        }
      }
      pre += c[k];
    }
  }
  __syncthreads();   // the bitmap (in the ring) is dead from here; ublk complete
  const int nu = s_nu;
  const int nitems = nu * KT;
  const int S = (nitems + NI - 1) / NI;

  if (w == kGdCons) {
    // ---------------------------------------------------------------- producer
    const T* kb = K + b * ksb + h * ksh;
    const int prow = lane / CPR, pc = lane % CPR;
    auto issue = [&](int st) {
      uint4* dst0 = ring + (st % NBUF) * NI * TILE4;
#pragma unroll
      for (int c = 0; c < NI; ++c) {
        int item = st * NI + c;
        item = item < nitems ? item : nitems - 1;
        const int cb = item / KT, kt = item - cb * KT;
        const int64_t row0 = (int64_t)ublk[cb] * BLOCK + kt * 32;
#pragma unroll
        for (int j = 0; j < LPI; ++j) {
          const int row = j * RPL + prow;
          const T* src = kb + (row0 + row) * ksn + 8 * (pc ^ (row & 7));
          __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(dst0 + c * TILE4 + j * kWave), 16, 0, 0);
        }
      }
    };
    for (int st = 0; st < NBUF - 1; ++st)
      if (st < S) issue(st);
    // stage 0 landed: the copies issued after it (stages 1 .. NBUF - 2) may still be in flight
    {
      const int later = (S - 1 < NBUF - 2 ? S - 1 : NBUF - 2);
      if (NBUF >= 4 && later >= 2) wait_vmcnt<(NBUF >= 4 ? 2 * LPS : 0)>();
      else if (NBUF >= 3 && later >= 1) wait_vmcnt<(NBUF >= 3 ? LPS : 0)>();
      else wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    for (int s = 0; s < S; ++s) {
      if (s + NBUF - 1 < S) issue(s + NBUF - 1);
      // stage s + 1 landed; stages s + 2 .. s + NBUF - 1 may be in flight
      const int hi = (s + NBUF - 1 < S - 1 ? s + NBUF - 1 : S - 1);
      const int later = hi - (s + 1);
      if (NBUF >= 4 && later >= 2) wait_vmcnt<(NBUF >= 4 ? 2 * LPS : 0)>();
      else if (NBUF >= 3 && later >= 1) wait_vmcnt<(NBUF >= 3 ? LPS : 0)>();
      else wait_vmcnt<0>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
  } else {
    // ---------------------------------------------------------------- consumers
    const int q = lane & 31;   // this lane's query (row of the workgroup's tile: 32 w + q)
    // stores go through a buffer resource over this consumer's valid rows: an offset past its end (a query
    // that did not select the block) is dropped by the hardware, so every store is one instruction without
    // a branch
    const int rstride = NB * BLOCK;                                   // floats per query row
    const int qv = nq - 32 * w < 0 ? 0 : (nq - 32 * w > 32 ? 32 : nq - 32 * w);
    const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
        out + ((int64_t)bh * N + n0 + 32 * w) * rstride, 0, qv * rstride * 4, 0x00020000);
    const int lane_off = (q * rstride + 4 * hh) * 4;                 // bytes
    // transposed scores of item c of the stage in ring buffer rb: S^T = K_tile . Q^T with the tile as the A
    // operand, so accumulator register i of lane (q, hh) holds key 8 (i / 4) + 4 hh + i % 4 of query q:
    // every group of four registers is four consecutive keys of the lane's own query
    auto stage_scores = [&](int c, int rb) -> f32x16_g {
      const uint4* slot = ring + (rb * NI + c) * TILE4;
      uint4 kbv[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kbv[ks] = slot[q * CPR + ((2 * ks + hh) ^ (q & 7))];
      f32x16_g acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc = mfma32<T>(kbv[ks], qa[ks], acc);
      return acc;
    };
    __syncthreads();   // stage 0 landed
    for (int s = 0; s < S; ++s) {
      const int it0 = s * NI;
      const int cb0 = it0 / KT;
      // slot masks of the stage's blocks for this lane's query
      uint32_t any = 0, mk[NBS];
#pragma unroll
      for (int j = 0; j < NBS; ++j) {
        const int cb = cb0 + j;
        const int u = cb < nu ? (int)ublk[cb] : 0xfffe;   // never equal to an id (unused slots hold 0xffff)
        const uint32_t u2 = ((uint32_t)u & 0xffffu) * 0x10001u;
        uint32_t m = 0;
#pragma unroll
        for (int k = 0; k < kGdMaxSlots / 2; ++k) {
          const uint32_t d = ids2[k] ^ u2;
          m |= ((d & 0xffffu) == 0u ? 1u : 0u) << (2 * k);
          m |= ((d >> 16) == 0u ? 1u : 0u) << (2 * k + 1);
        }
        mk[j] = m;
        if (__any(m != 0)) any |= 1u << j;
      }
      // scores and stores of the stage's items, one at a time; an item none of this consumer's queries
      // selected (or past the end) is skipped
#pragma unroll
      for (int c = 0; c < NI; ++c) {
        const int item = it0 + c;
        const int j = NI >= KT ? c / KT : 0;
        if (item >= nitems || !((any >> j) & 1u)) continue;
        const f32x16_g acc = stage_scores(c, s % NBUF);
        const uint32_t m = mk[j];
        const int ob = lane_off + (item % KT) * 128;
        const int off = m ? ob + (__ffs(m) - 1) * BLOCK * 4 : 0x7fffffff;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          gd_u32x4 v = {__float_as_uint(acc[4 * a] * scale), __float_as_uint(acc[4 * a + 1] * scale),
                        __float_as_uint(acc[4 * a + 2] * scale), __float_as_uint(acc[4 * a + 3] * scale)};
          __builtin_amdgcn_raw_buffer_store_b128(v, orsrc, off + 32 * a, 0, 0);
        }
        // a query that selected this block in more than one slot: write the remaining slots
        uint32_t more = m & (m - 1);
        if (__any(more != 0)) {
          while (more) {
            const int o2 = ob + (__ffs(more) - 1) * BLOCK * 4;
            more &= more - 1;
#pragma unroll
            for (int a = 0; a < 4; ++a) {
              gd_u32x4 v = {__float_as_uint(acc[4 * a] * scale), __float_as_uint(acc[4 * a + 1] * scale),
                            __float_as_uint(acc[4 * a + 2] * scale), __float_as_uint(acc[4 * a + 3] * scale)};
              __builtin_amdgcn_raw_buffer_store_b128(v, orsrc, o2 + 32 * a, 0, 0);
            }
          }
        }
      }
      __syncthreads();
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
  const int ntile = (N + kGdQ - 1) / kGdQ;
  const int64_t nwg = (int64_t)ntile * B * H;
  if (nwg > 0x7fffffff) return TA_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int nblocks = M / block;
#define TA_GB(T, DD, BL)                                                                                        \
  hipLaunchKernelGGL((gather_blocks_kernel<T, DD, BL>), dim3((unsigned)nwg), dim3(kGdThreads), 0, st,          \
                     (const T*)q, qsb, qsh, qsn, (const T*)K, ksb, ksh, ksn, blk, H, N, nblocks, NB, ntile,      \
                     scale, out)
#define TA_GB_BL(T, DD)                  \
  if (block == 32) TA_GB(T, DD, 32);     \
  else if (block == 64) TA_GB(T, DD, 64); \
  else TA_GB(T, DD, 128);
  if (dtype == TA_BF16) {
    if (D == 64) { TA_GB_BL(bf16_t, 64) } else { TA_GB_BL(bf16_t, 128) }
  } else {
    if (D == 64) { TA_GB_BL(f16_t, 64) } else { TA_GB_BL(f16_t, 128) }
  }
#undef TA_GB_BL
#undef TA_GB
  return check_launch("gather_blocks_kernel");
}
