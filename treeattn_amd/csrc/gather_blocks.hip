// Leaf-block gather-dot on gfx950 MFMA: out[b,h,n, c*block + j] = scale * q[b,h,n] . K[b,h, blk[b,h,n,c]*block + j].
//
// A workgroup (4 wavefronts) takes 32 consecutive queries of one (b, h).  It marks the distinct blocks its
// queries selected, and each wavefront takes every fourth of them: for each 32-key tile of the block it
// computes the 32 x 32 scores Q_tile . K_tile^T with v_mfma_f32_32x32x16_bf16 (D/16 k-steps), stages them in
// its LDS slot, and the (query, slot) entries that selected the block are compacted and written 8 lanes per
// entry, each a contiguous 128-byte run of that query's 32 scores.  The K tile of the next (block, tile) is loaded before the current
// one is written out.  The products of bf16 values are exact in float32; the sum over D is taken by the MFMA, so
// scores agree with a sequential float32 sum to a few ulps (not bit for bit).  The kernel is bound by the
// float32 output writes.
#include "common.hpp"

namespace ta {

typedef __bf16 bf16x8_g __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_g __attribute__((ext_vector_type(8)));
typedef float f32x16_g __attribute__((ext_vector_type(16)));

constexpr int kGdMaxBlocks = 8192;      // distinct blocks per (b, h) the bitmap can mark (M / block)
constexpr int kGdMaxSlots = 16;         // selected blocks per query (entries held 8 per lane)

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

template <typename T, int D, int BLOCK>
__global__ __launch_bounds__(256) void gather_blocks_kernel(const T* __restrict__ q, int64_t qsb, int64_t qsh,
                                                            int64_t qsn, const T* __restrict__ K, int64_t ksb,
                                                            int64_t ksh, int64_t ksn, const int32_t* __restrict__ blk,
                                                            int H, int N, int nblocks, int NB, float scale,
                                                            float* __restrict__ out) {
  constexpr int KS = D / 16;           // MFMA k-steps
  constexpr int KT = BLOCK / 32;       // 32-key tiles per block
  constexpr int EPL = 32 * kGdMaxSlots / kWave;   // (query, slot) entries per lane
  __shared__ uint32_t used[kGdMaxBlocks / 32];
  __shared__ float s_tile[4][32][33];
  __shared__ int32_t s_hit[4][32 * kGdMaxSlots];
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int n0 = blockIdx.x * 32;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int nq = N - n0 < 32 ? N - n0 : 32;
  const int ne = nq * NB;
  const int nwords = (nblocks + 31) / 32;

  for (int i = tid; i < nwords; i += 256) used[i] = 0u;
  __syncthreads();
  // every wavefront keeps all (query, slot) entries of the tile: entry e = lane + 64 i
  const int32_t* brow = blk + ((int64_t)bh * N + n0) * NB;
  int ev[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + kWave * i;
    int v = -1;
    if (e < ne) {
      v = brow[e];
      v = v < 0 ? 0 : (v >= nblocks ? nblocks - 1 : v);
      if (w == (i & 3)) atomicOr(&used[v >> 5], 1u << (v & 31));
    }
    ev[i] = v;
  }
  __syncthreads();

  // query tile as the MFMA A operand: lane -> row lane % 32, dims 16*ks + 8*(lane/32) .. +8
  const int rq = lane & 31;
  const int kh = (lane >> 5) * 8;
  uint4 qa[KS];
  {
    const bool ok = rq < nq;
    const T* qr = q + b * qsb + h * qsh + (int64_t)(n0 + (ok ? rq : 0)) * qsn + kh;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = ok ? *reinterpret_cast<const uint4*>(qr + 16 * s) : make_uint4(0, 0, 0, 0);
  }
  const T* kbase = K + b * ksb + h * ksh + kh;
  float* obase = out + ((int64_t)bh * N + n0) * (int64_t)NB * BLOCK;

  // the marked blocks, wavefront w taking every fourth; the K tile of the next (block, tile) is loaded
  // before the current one is written out
  auto next_item = [&](int& word, uint32_t& bits, int& seen) -> int {
    while (true) {
      while (bits == 0u) {
        if (++word >= nwords) return -1;
        bits = used[word];
      }
      const int bit = __ffs(bits) - 1;
      bits &= bits - 1;
      if ((seen++ & 3) == w) return word * 32 + bit;
    }
  };
  int word = 0, seen = 0;
  uint32_t bits = nwords > 0 ? used[0] : 0u;
  int u = next_item(word, bits, seen);
  uint4 kb[KS];
  int kt = 0;
  if (u >= 0) {
    const T* kr = kbase + (int64_t)(u * BLOCK + rq) * ksn;
#pragma unroll
    for (int s = 0; s < KS; ++s) kb[s] = *reinterpret_cast<const uint4*>(kr + 16 * s);
  }
  while (u >= 0) {
    f32x16_g acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma32<T>(qa[s], kb[s], acc);
    // advance to the next (block, tile) and start its loads
    const int cu = u, ckt = kt;
    if (++kt == KT) {
      kt = 0;
      u = next_item(word, bits, seen);
    }
    if (u >= 0) {
      const T* kr = kbase + (int64_t)(u * BLOCK + kt * 32 + rq) * ksn;
#pragma unroll
      for (int s = 0; s < KS; ++s) kb[s] = *reinterpret_cast<const uint4*>(kr + 16 * s);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) s_tile[w][8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)][lane & 31] = acc[i] * scale;
    wave_sync();
    // entries that selected block cu, compacted; then 8 lanes per entry write its 32 scores (128 bytes)
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const bool hit = ev[i] == cu;
      const uint64_t bal = __ballot(hit);
      if (hit) s_hit[w][cnt + __popcll(bal & ((1ull << lane) - 1))] = lane + kWave * i;
      cnt += __popcll(bal);
    }
    wave_sync();
    for (int p0 = 0; p0 < cnt; p0 += 8) {
      const int p = p0 + (lane >> 3);
      if (p < cnt) {
        const int e = s_hit[w][p];
        const int qq = e / NB, slot = e - qq * NB;
        const int j = lane & 7;
        const float* src = &s_tile[w][qq][4 * j];
        *reinterpret_cast<float4*>(obase + ((int64_t)qq * NB + slot) * BLOCK + ckt * 32 + 4 * j) =
            make_float4(src[0], src[1], src[2], src[3]);
      }
    }
    wave_sync();
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
  dim3 grid((N + 31) / 32, B * H);
  hipStream_t st = (hipStream_t)stream;
  const int nblocks = M / block;
#define TA_GB(T, DD, BL)                                                                                          \
  hipLaunchKernelGGL((gather_blocks_kernel<T, DD, BL>), grid, dim3(256), 0, st, (const T*)q, qsb, qsh, qsn,      \
                     (const T*)K, ksb, ksh, ksn, blk, H, N, nblocks, NB, scale, out)
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
