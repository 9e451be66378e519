// Row-block matrix product tile on gfx950 MFMA (v_mfma_f32_32x32x16_bf16), shared by the standalone
// product kernel (gemm.hip) and the persistent decode step (step.hip):
//
//   Y[M, N] = epilogue( prologue(X)[M, K] . W[N, K]^T ),  bf16 in and out, float32 accumulation.
//   prologue: LayerNorm over K without bias (engine.py:14-15; model.py:12-18) when a LayerNorm weight is given.
//   epilogue: none | GELU (erf form, model.py:30) | residual add R + (.) (model.py:42-44).
// Rounding follows the unfused op chain in bf16: the LayerNorm output, the product and the GELU output are
// each rounded to bf16, the residual sum is taken in float32 of the two bf16 values and rounded.
//
// A workgroup of four wavefronts computes one 32 x 32 output tile over a range of K (a split).  The K blocks
// of 64 are dealt to eight streams (stream v takes blocks v, v + 8, v + 16, ...); wavefront w runs streams w
// and w + 4, each into its own accumulator, and the eight partial tiles are summed in stream order.
// X is staged in LDS a round (up to 16 blocks) at a time with direct global-to-LDS copies (no registers,
// every copy in flight at once) in the layout [block][row][64], the 16-byte pieces of row r stored at
// position piece ^ (r % 8) so that the MFMA operand reads of 32 rows are free of bank conflicts.  A lane
// feeds row lane % 32 of X and of W (output column); lanes 0-31 take k0..k0+31 of a block, lanes 32-63
// k0+32..k0+63; MFMA j of the block takes elements 8j..8j+7 of each lane's run, the same k for X and W.
// W of the first round can be loaded into registers before X is available (mm_load_w), which the decode
// step uses to fetch weights while the producing tasks still run.  LayerNorm statistics come from the staged
// rows (when one round holds all of K) or from a pass over X (8 threads per row, fixed order); the staged
// rows are then normalised in place before the products.
//
// With splits > 1 the K blocks are divided among that many workgroups per tile: each writes its float32
// partial tile with stores that write through to memory, waits for them, and counts itself in with a
// device-scope atomic; the last to arrive sums the partials in split order (independent of arrival order),
// applies the epilogue and resets the counter.
//
// FRESH = true: X and R were written by other workgroups of the running kernel -- they are read past the
// caches.  WT = true: Y is written through (so other workgroups of the running kernel may read it the same
// way); by default WT = FRESH.
#pragma once

#include "common.hpp"

#ifndef TA_MARK
#define TA_MARK(i) \
  do {             \
  } while (0)
#endif

namespace ta {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum { EPI_NONE = 0, EPI_GELU = 1, EPI_RESIDUAL = 2 };

constexpr int kMmThreads = 256;                    // four wavefronts
constexpr int kMmStreams = 8;                      // K-block streams
constexpr int kMmSlots = 2;                        // blocks per stream and round
constexpr int kMmRound = kMmStreams * kMmSlots;    // 16 blocks (1024 of K) per round
constexpr int kMmRedBytes = kMmStreams * 32 * 33 * 4;
constexpr int kMmTailBytes = 64 * 4 + 16;          // mean, rstd, last
constexpr int kNtLnMaxK = 896;                     // narrow tiles with the LayerNorm prologue: K up to this

// LDS of a tile whose splits span at most `kblocks` K blocks: X (4 KB per block of a round) and the
// LayerNorm weight of the round (128 B per block, plus the slack of a whole last copy), aliased by the
// partial tiles once the products are done; then the row statistics.
__host__ __device__ constexpr int mm_lds_main(int kblocks) {
  return (kblocks < kMmRound ? kblocks : kMmRound) * 4224 + 1024 > kMmRedBytes
             ? (kblocks < kMmRound ? kblocks : kMmRound) * 4224 + 1024
             : kMmRedBytes;
}
__host__ __device__ constexpr int mm_lds_bytes(int kblocks) { return mm_lds_main(kblocks) + kMmTailBytes; }

struct MmArgs {
  const bf16_t* X;
  int64_t ldx;
  const bf16_t* W;
  int64_t ldw;
  bf16_t* Y;
  int64_t ldy;
  const bf16_t* R;
  int64_t ldr;
  const bf16_t* gam;   // LayerNorm weight (the prologue is on when the template flag LN is set)
  float eps;
  int M, N, K;
  int splits;          // workgroups per tile along K
  int tiles;           // output tiles of the product (partials are indexed split * tiles + tile)
  float* part;         // splits * tiles * 1024 floats when splits > 1
  uint32_t* cnt;       // per-tile arrival counters when splits > 1 (zero between calls)
};

// W of the first round for the two streams of this wavefront.
struct MmPre {
  uint4 w[2][kMmSlots][4];
};

// ----------------------------------------------------------------------------------------- helpers
template <bool FRESH>
__device__ __forceinline__ uint4 mm_ld16(const void* p) {
  if constexpr (FRESH) return ldg16_dc(p);
  else return ldg16(p);
}

__device__ __forceinline__ float mm_bf16_round(float x) { return to_f32(bf16_from(x)); }

__device__ __forceinline__ uint32_t mm_pack2(float a, float b) { return bf16_pack2(a, b); }

// Blocks [blk0, blk0 + nblk) of split s.
__host__ __device__ __forceinline__ void mm_split_range(int K, int splits, int s, int& blk0, int& nblk) {
  const int nb = K / 64;
  const int per = (nb + splits - 1) / splits;
  blk0 = s * per;
  const int blk1 = blk0 + per < nb ? blk0 + per : nb;
  nblk = blk1 > blk0 ? blk1 - blk0 : 0;
}

// W blocks of round `round` for stream v of this lane (row n0 + lane % 32).
__device__ __forceinline__ void mm_load_w_stream(const MmArgs& a, int n0, int blk0, int nblk, int round, int v,
                                                 uint4 (&wb)[kMmSlots][4]) {
  const int lane = lane_id();
  const int rl = lane & 31, kh = (lane >> 5) * 32;
  const bool wok = n0 + rl < a.N;
  const bf16_t* wr = a.W + (int64_t)(n0 + (wok ? rl : 0)) * a.ldw + (int64_t)blk0 * 64 + kh;
#pragma unroll
  for (int i = 0; i < kMmSlots; ++i) {
    const int blk = round * kMmRound + v + kMmStreams * i;
    const bool ok = wok && blk < nblk;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wb[i][j] = ok ? ldg16(wr + (int64_t)blk * 64 + 8 * j) : make_uint4(0, 0, 0, 0);
  }
}

// W of the first round for this wavefront's two streams as exactly kMmWLoads load instructions per lane,
// whatever the shape: a block past the split reads block 0 again and a column past N reads column n0 (neither
// feeds an output that is kept), so that a wait on the memory counter can count them.
constexpr int kMmWLoads = 2 * kMmSlots * 4;
__device__ __forceinline__ void mm_load_w_all(const MmArgs& a, int n0, int nblk0, int blk0, MmPre& pre) {
  const int lane = lane_id(), w = wave_id();
  const int rl = lane & 31, kh = (lane >> 5) * 32;
  const bf16_t* wr = a.W + (int64_t)(n0 + (n0 + rl < a.N ? rl : 0)) * a.ldw + (int64_t)blk0 * 64 + kh;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < kMmSlots; ++i) {
      const int blk = w + 4 * s + kMmStreams * i;
      const int b = blk < nblk0 ? blk : 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) pre.w[s][i][j] = ldg16(wr + (int64_t)b * 64 + 8 * j);
    }
}

// Issue the loads of W's first round for this wavefront's two streams.
__device__ __forceinline__ void mm_load_w(const MmArgs& a, int tn, int split, MmPre& pre) {
  int blk0, nblk;
  mm_split_range(a.K, a.splits, split, blk0, nblk);
  const int w = wave_id();
  mm_load_w_stream(a, tn * 32, blk0, nblk, 0, w, pre.w[0]);
  mm_load_w_stream(a, tn * 32, blk0, nblk, 0, w + 4, pre.w[1]);
}

// Best (value, column) of a row: larger value, or equal value at a smaller column; NaN never wins.
__device__ __forceinline__ void mm_better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Order-preserving 64-bit key of (value, column) for an atomic maximum: larger value first, then smaller
// column.  0 is below every key (no candidate).
__device__ __forceinline__ uint64_t mm_argmax_key(float v, int col) {
  uint32_t u = __float_as_uint(v + 0.0f);
  u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
  return ((uint64_t)u << 32) | (uint32_t)(0x7FFFFFFF - col);
}

// LayerNorm row statistics from the sums of x and x^2 over n elements: written once, with contraction off, so
// that every kernel normalising rows computes the same bits.
__device__ __forceinline__ void mm_stats(float s, float s2, int n, float eps, float& mean, float& rstd) {
#pragma clang fp contract(off)
  mean = s / (float)n;
  rstd = rsqrtf(fmaxf(s2 / (float)n - mean * mean, 0.0f) + eps);
}

// The epilogue of one output element: the float32 product rounded to bf16, then GELU (erf form, model.py:30)
// of that value rounded again, or the residual (a bf16 value as float32) plus it rounded.
template <int EPI>
__device__ __forceinline__ bf16_t mm_epilogue(float acc, float res) {
  float v = mm_bf16_round(acc);
  if constexpr (EPI == EPI_GELU) v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
  if constexpr (EPI == EPI_RESIDUAL) v = res + v;
  return bf16_from(v);
}

__device__ __forceinline__ void mm_add8(uint4 u, float& s, float& s2) {
  const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float f0 = __uint_as_float(wd[e] << 16), f1 = __uint_as_float(wd[e] & 0xffff0000u);
    s += f0;
    s2 = fmaf(f0, f0, s2);
    s += f1;
    s2 = fmaf(f1, f1, s2);
  }
}

// Yn[r] = LN(Y[r]) (weight gam, no bias) for rows r < M of N columns, the arithmetic of mm_tile's prologue:
// 8 threads per row, thread `part` sums piece `part` (8 elements) of every 64-column block in block order,
// then the xor tree over the 8 threads; each element (y - mean) * rstd * g rounded to bf16.  256 threads.
// FRESH: Y was written by other workgroups of the running kernel.
template <bool FRESH>
__device__ __forceinline__ void mm_rows_ln(const bf16_t* Y, int64_t ldy, int M, int N, const bf16_t* gam, float eps,
                                           bf16_t* Yn, int64_t ldyn) {
  const int tid = threadIdx.x;
  for (int r0 = 0; r0 < M; r0 += kMmThreads / 8) {
    const int r = r0 + (tid >> 3), part = tid & 7;
    const bool ok = r < M;
    const bf16_t* yr = Y + (int64_t)(ok ? r : 0) * ldy + 8 * part;
    float s = 0.0f, s2 = 0.0f;
    for (int k0 = 0; k0 < N; k0 += 64 * 8) {
      uint4 u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) u[i] = k0 + 64 * i < N ? mm_ld16<FRESH>(yr + k0 + 64 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + 64 * i < N) mm_add8(u[i], s, s2);
    }
    s = group_sum<8>(s);
    s2 = group_sum<8>(s2);
    float mean, rstd;
    mm_stats(s, s2, N, eps, mean, rstd);
    if (!ok) continue;
    bf16_t* yn = Yn + (int64_t)r * ldyn + 8 * part;
    for (int k = 0; k < N; k += 64) {
      const uint4 xu = mm_ld16<FRESH>(yr + k);
      const uint4 gu = ldg16(gam + k + 8 * part);
      const uint32_t xw[4] = {xu.x, xu.y, xu.z, xu.w}, gw[4] = {gu.x, gu.y, gu.z, gu.w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float f0 = __uint_as_float(xw[e] << 16), f1 = __uint_as_float(xw[e] & 0xffff0000u);
        const float g0 = __uint_as_float(gw[e] << 16), g1 = __uint_as_float(gw[e] & 0xffff0000u);
        o[e] = mm_pack2((f0 - mean) * rstd * g0, (f1 - mean) * rstd * g1);
      }
      *(TA_GLOBAL u32x4_t*)(yn + k) = u32x4_t{o[0], o[1], o[2], o[3]};
    }
  }
}

// X rows m0..m0+31 of blocks [blk0, blk0 + rn) -> LDS xs ([rn][32][64], 16-byte pieces of a row swizzled
// by the row), and the LayerNorm weight of those blocks -> gs; one copy = 8 rows of one block, lane -> (row,
// piece).  Unrolled, so that no copy waits for another.  FRESH: cache policy sc1 (device scope, as the
// device-coherent loads).
template <bool LN, bool FRESH>
__device__ __forceinline__ void mm_stage(const MmArgs& a, bf16_t* xs, bf16_t* gs, int m0, int blk0, int rn) {
  const int lane = lane_id(), w = wave_id();
  const int prow = lane >> 3, pc = (lane & 7) ^ prow;
#pragma unroll
  for (int i = 0; i < kMmRound; ++i) {
    const int c = w + 4 * i;
    if (c >= rn * 4) break;
    const int blk = c >> 2, row = (c & 3) * 8 + prow;
    const int gm = m0 + row < a.M ? m0 + row : a.M - 1;
    const bf16_t* src = a.X + (int64_t)gm * a.ldx + (int64_t)(blk0 + blk) * 64 + 8 * pc;
    if constexpr (FRESH)
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(xs + (size_t)c * 512), 16, 0, 16);
    else
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(xs + (size_t)c * 512), 16, 0, 0);
  }
  if constexpr (LN) {
    // rn * 8 pieces of 16 bytes (a copy's surplus lanes read piece 0)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = w + 4 * i;
      if (c * 64 >= rn * 8) break;
      const int piece = c * 64 + lane;
      const bf16_t* src = a.gam + (int64_t)blk0 * 64 + 8 * (piece < rn * 8 ? piece : 0);
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(gs + (size_t)c * 512), 16, 0, 0);
    }
  }
}

// One 16-byte piece of a row normalised: (x - mean) * rstd * g, rounded to bf16.
__device__ __forceinline__ uint4 mm_ln_piece(uint4 xu, uint4 gu, float mean, float rstd) {
  const uint32_t gw[4] = {gu.x, gu.y, gu.z, gu.w};
  const uint32_t xw[4] = {xu.x, xu.y, xu.z, xu.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float f0 = __uint_as_float(xw[e] << 16), f1 = __uint_as_float(xw[e] & 0xffff0000u);
    const float g0 = __uint_as_float(gw[e] << 16), g1 = __uint_as_float(gw[e] & 0xffff0000u);
    o[e] = mm_pack2((f0 - mean) * rstd * g0, (f1 - mean) * rstd * g1);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// LayerNorm in place of the rn staged blocks that hold all of K (statistics from the staged rows).  Thread
// (r, part) owns piece `part` of row r in every block: it sums them for the statistics (the row's 8 threads
// then combine their sums), keeps them in registers and writes them back normalised.
__device__ __forceinline__ void mm_ln_staged(bf16_t* xs, const bf16_t* gs, int rn, int K, float eps) {
  const int tid = threadIdx.x;
  const int r = tid >> 3, part = tid & 7;
  const int phys = 8 * (part ^ (r & 7));   // where piece `part` of row r sits in a staged block
  const bf16_t* gp = gs + 8 * part;
  uint4 xv[kMmRound];   // every read issued before the first sum (a block past the round reads block 0)
#pragma unroll
  for (int blk = 0; blk < kMmRound; ++blk)
    xv[blk] = *reinterpret_cast<const uint4*>(xs + (size_t)((blk < rn ? blk : 0) * 32 + r) * 64 + phys);
  float s = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int blk = 0; blk < kMmRound; ++blk)
    if (blk < rn) mm_add8(xv[blk], s, s2);
  s = group_sum<8>(s);
  s2 = group_sum<8>(s2);
  float mean, rstd;
  mm_stats(s, s2, K, eps, mean, rstd);
  // four blocks at a time: their weight pieces read together, then the transforms, then the stores
#pragma unroll
  for (int b4 = 0; b4 < kMmRound; b4 += 4) {
    if (b4 >= rn) break;
    uint4 gv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) gv[i] = *reinterpret_cast<const uint4*>(gp + (b4 + i < rn ? b4 + i : 0) * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (b4 + i < rn)
        *reinterpret_cast<uint4*>(xs + (size_t)((b4 + i) * 32 + r) * 64 + phys) = mm_ln_piece(xv[b4 + i], gv[i], mean, rstd);
  }
}

// The products of the rn staged blocks with W (wb: this wavefront's two streams of K blocks), accumulated
// into acc in a fixed order.
__device__ __forceinline__ void mm_products(const bf16_t* xs, int rn, const MmPre& wb, f32x16 (&acc)[2]) {
  const int lane = lane_id(), w = wave_id();
  const int rl = lane & 31;
  const int ph = (lane >> 5) * 4;   // first 16-byte piece of this lane's half of a block row
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int v = w + 4 * s;
#pragma unroll
    for (int i = 0; i < kMmSlots; ++i) {
      const int lb = v + kMmStreams * i;   // block within the round
      if (lb >= rn) break;
      const bf16_t* xrow = xs + (size_t)(lb * 32 + rl) * 64;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 xa = *reinterpret_cast<const uint4*>(xrow + 8 * ((ph + j) ^ (rl & 7)));
        bf16x8 av, bv;
        __builtin_memcpy(&av, &xa, 16);
        __builtin_memcpy(&bv, &wb.w[s][i][j], 16);
        acc[s] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc[s], 0, 0, 0);
      }
    }
  }
}

// The tile (tn, tm) of split `split`, tile index `tile` among a.tiles.  pre holds W's first round (from
// mm_load_w).  lds: mm_lds_bytes(blocks of the split) bytes of LDS, 16-byte aligned.  ARGMAX: also fold each
// row's best (value, column) over the tile's columns -- of the bf16 outputs -- into amax[row] with an atomic
// maximum of mm_argmax_key.  Returns true when this workgroup wrote the tile's output (always without
// splits; the last to arrive with splits).
// WLATE: pre is not used; W's first round is loaded here, right after the copies of X's first round are
// issued, and only the copies are waited for before the LayerNorm, so the statistics and the transform of
// the staged rows run while W is still arriving.
template <bool LN, int EPI, bool FRESH, bool ARGMAX = false, bool WT = FRESH, bool WLATE = false>
__device__ __forceinline__ bool mm_tile(const MmArgs& a, int tn, int tm, int split, int tile, const MmPre& pre,
                                        char* lds, uint64_t* amax = nullptr) {
  const int tid = threadIdx.x;
  const int lane = lane_id(), w = wave_id();
  const int n0 = tn * 32, m0 = tm * 32;
  int blk0, nblk;
  mm_split_range(a.K, a.splits, split, blk0, nblk);
  const int nround = (nblk + kMmRound - 1) / kMmRound;
  const int rblk = nblk < kMmRound ? nblk : kMmRound;   // blocks staged per round
  bf16_t* xs = reinterpret_cast<bf16_t*>(lds);                   // [rblk][32][64]
  bf16_t* gs = xs + rblk * 2048;                                 // [rblk * 64] (+ slack)
  float* red = reinterpret_cast<float*>(lds);                    // [8][32][33], after the products
  float* s_mean = reinterpret_cast<float*>(lds + mm_lds_main(nblk));
  float* s_rstd = s_mean + 32;
  uint32_t* s_last = reinterpret_cast<uint32_t*>(s_rstd + 32);
  constexpr int EPT = 1024 / kMmThreads;                         // epilogue elements per thread

  // residual values of the epilogue, fetched now (they do not depend on the product)
  float rres[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) rres[k] = 0.0f;
  if constexpr (EPI == EPI_RESIDUAL) {
    uint16_t rb[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * kMmThreads;
      const int gm = m0 + (e >> 5), gn = n0 + (e & 31);
      const bf16_t* p = a.R + (int64_t)(gm < a.M ? gm : 0) * a.ldr + (gn < a.N ? gn : 0);
      if constexpr (FRESH) rb[k] = ldg2_dc(p);
      else rb[k] = *(const TA_GLOBAL uint16_t*)p;
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) rres[k] = __uint_as_float((uint32_t)rb[k] << 16);
  }

  // LayerNorm statistics over all of K: from the staged rows when one round holds all of K, else from a pass
  // over X first (8 threads per row)
  const bool stats_staged = nround == 1 && nblk == a.K / 64;
  if (LN && !stats_staged) {
    const int r = tid >> 3, part = tid & 7;
    float s = 0.0f, s2 = 0.0f;
    const bf16_t* xr = a.X + (int64_t)(m0 + r < a.M ? m0 + r : a.M - 1) * a.ldx;
    for (int k0 = part * 8; k0 < a.K; k0 += 64 * 8) {
      uint4 u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        u[i] = k0 + 64 * i < a.K ? mm_ld16<FRESH>(xr + k0 + 64 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) mm_add8(u[i], s, s2);
    }
    s = group_sum<8>(s);
    s2 = group_sum<8>(s2);
    if (part == 0) {
      float mean, rstd;
      mm_stats(s, s2, a.K, a.eps, mean, rstd);
      s_mean[r] = mean;
      s_rstd[r] = rstd;
    }
  }

  f32x16 acc[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[s][i] = 0.0f;

  auto stage = [&](int rb0, int rn) { mm_stage<LN, FRESH>(a, xs, gs, m0, blk0 + rb0, rn); };

  // statistics (when they come from the staged rows) and the LayerNorm of the staged rows, in place
  auto normalise = [&](int rn) {
    if constexpr (LN) {
      const int r = tid >> 3, part = tid & 7;
      const int phys = 8 * (part ^ (r & 7));   // where piece `part` of row r sits in a staged block
      const bf16_t* gp = gs + 8 * part;
      if (stats_staged) {
        mm_ln_staged(xs, gs, rn, a.K, a.eps);
      } else {
        // statistics from the pass over X
        const float mean = s_mean[r], rstd = s_rstd[r];
#pragma unroll 4
        for (int blk = 0; blk < rn; ++blk) {
          uint4* xp = reinterpret_cast<uint4*>(xs + (size_t)(blk * 32 + r) * 64 + phys);
          *xp = mm_ln_piece(*xp, *reinterpret_cast<const uint4*>(gp + blk * 64), mean, rstd);
        }
      }
      lds_barrier();
    }
    TA_MARK(2);
  };

  auto products = [&](int rn, const MmPre& wb) { mm_products(xs, rn, wb, acc); };

  // round 0; its W registers are used where they were loaded (no copies, which would wait for the loads)
  {
    const int rn = nblk < kMmRound ? nblk : kMmRound;
    stage(0, rn);
    if constexpr (WLATE) {
      MmPre wl;
      asm volatile("" ::: "memory");   // W's loads are issued after the copies, so they are counted last
      mm_load_w_all(a, n0, rn, blk0, wl);
      wait_vmcnt_n<kMmWLoads>();       // the copies (and the residual loads before them) have landed
      lds_barrier();                   // (W stays in flight through the LayerNorm)
      TA_MARK(0);
      normalise(rn);
      products(rn, wl);
    } else {
      wait_vmcnt_n<0>();
      __syncthreads();
      TA_MARK(0);
      normalise(rn);
      products(rn, pre);
    }
  }
  for (int round = 1; round < nround; ++round) {
    const int rb0 = round * kMmRound;
    const int rn = nblk - rb0 < kMmRound ? nblk - rb0 : kMmRound;
    __syncthreads();   // the previous round's rows have been read
    stage(rb0, rn);
    wait_vmcnt_n<0>();
    __syncthreads();
    normalise(rn);
    MmPre wb;
    mm_load_w_stream(a, n0, blk0, nblk, round, w, wb.w[0]);
    mm_load_w_stream(a, n0, blk0, nblk, round, w + 4, wb.w[1]);
    products(rn, wb);
  }
  __syncthreads();   // every wavefront is done with the staged rows; the partial tiles take their place
  // 32x32 MFMA output layout: lane -> column lane % 32; register i -> row 8(i/4) + 4(lane/32) + i%4
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int v = w + 4 * s;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      red[(v * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * 33 + (lane & 31)] = acc[s][i];
  }
  __syncthreads();
  TA_MARK(3);

  if (a.splits > 1) {
    float* mine = a.part + ((int64_t)split * a.tiles + tile) * 1024;
    for (int e = tid; e < 1024; e += kMmThreads) {
      const int r = e >> 5, c = e & 31;
      float v = red[r * 33 + c];
#pragma unroll
      for (int s = 1; s < kMmStreams; ++s) v += red[(s * 32 + r) * 33 + c];
      stgf_dc(&mine[e], v);   // written through
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wavefront's stores have completed
    __syncthreads();
    if (tid == 0)
      *s_last = __hip_atomic_fetch_add((TA_GLOBAL uint32_t*)&a.cnt[tile], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.splits - 1);
    __syncthreads();
    if (!*s_last) return false;
  }
  // epilogue: thread tid takes column tid % 32 of rows tid / 32 + 8k
  float vals[EPT];
  if (a.splits > 1) {
    // the partials of every split, all loads in flight before the sums (in split order)
    const int64_t stride = (int64_t)a.tiles * 1024;
    const float* p = a.part + (int64_t)tile * 1024 + tid;
#pragma unroll
    for (int k = 0; k < EPT; ++k) vals[k] = 0.0f;
    for (int s0 = 0; s0 < a.splits; s0 += 4) {
      float pv[4][EPT];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int k = 0; k < EPT; ++k)
          pv[s][k] = s0 + s < a.splits ? ldgf_dc(p + (s0 + s) * stride + k * kMmThreads) : 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int k = 0; k < EPT; ++k)
          if (s0 + s < a.splits) vals[k] = (s0 + s == 0) ? pv[s][k] : vals[k] + pv[s][k];
    }
  } else {
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * kMmThreads;
      const int r = e >> 5, c = e & 31;
      float v = red[r * 33 + c];
#pragma unroll
      for (int s = 1; s < kMmStreams; ++s) v += red[(s * 32 + r) * 33 + c];
      vals[k] = v;
    }
  }
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + k * kMmThreads;
    const int r = e >> 5, c = e & 31;
    const int gm = m0 + r, gn = n0 + c;
    const bool in = gm < a.M && gn < a.N;
    const bf16_t o = mm_epilogue<EPI>(vals[k], rres[k]);
    if (in) {
      bf16_t* y = a.Y + (int64_t)gm * a.ldy + gn;
      if constexpr (WT) stg2_dc(y, o.bits);
      else *(TA_GLOBAL uint16_t*)y = o.bits;
    }
    if constexpr (ARGMAX) {
      // the row's best over the tile's 32 columns (lanes 0-31 or 32-63 of this wavefront hold one row)
      float bv = in ? to_f32(o) : -INFINITY;
      int bi = in ? gn : 0x7FFFFFFF;
      if (bv != bv) {   // NaN never wins
        bv = -INFINITY;
        bi = 0x7FFFFFFF;
      }
#pragma unroll
      for (int o2 = 1; o2 < 32; o2 <<= 1) {
        const float v2 = __shfl_xor(bv, o2, kWave);
        const int i2 = __shfl_xor(bi, o2, kWave);
        mm_better(bv, bi, v2, i2);
      }
      if (c == 0 && gm < a.M && bi != 0x7FFFFFFF)
        __hip_atomic_fetch_max((TA_GLOBAL uint64_t*)&amax[gm], mm_argmax_key(bv, bi), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (a.splits > 1 && tid == 0)   // ready for the next call
    __hip_atomic_store((TA_GLOBAL uint32_t*)&a.cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  TA_MARK(4);
  return true;
}

}  // namespace ta
