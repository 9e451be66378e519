// Row-block matrix product for the decode step of the model around the attention: a few rows (the
// sequences of a decode batch) times a weight matrix, with the LayerNorm before it and the GELU or the
// residual add after it fused in, on gfx950 MFMA (v_mfma_f32_32x32x16_bf16).
//
//   Y[M, N] = epilogue( prologue(X)[M, K] . W[N, K]^T ),  bf16 in and out, float32 accumulation.
//   prologue: LayerNorm over K without bias (engine.py:14-15; model.py:12-18) when ln_w is given.
//   epilogue: none | GELU (erf form, model.py:30) | residual add R + (.) (model.py:42-44).
// Rounding follows the unfused op chain in bf16: the LayerNorm output, the product and the GELU output are
// each rounded to bf16, the residual sum is taken in float32 of the two bf16 values and rounded.
//
// One workgroup computes a 32 x 32 output tile over a range of K; its eight wavefronts split that range in
// blocks of 64, each issuing the loads of up to four blocks before its first product, and their partial tiles
// are summed in LDS in a fixed order.  With `splits` > 1 the K blocks are divided among that many workgroups
// per tile (a few rows give too few tiles to occupy the chip): each writes its float32 partial tile to the
// workspace and counts itself in with a device-scope atomic; the last to arrive sums the partials in split
// order (so the result does not depend on arrival order), applies the epilogue and resets the counter.
// A lane reads 64 contiguous bytes of one X row and one W row per block: lanes 0-31 rows 0-31 at k0..k0+31,
// lanes 32-63 the same rows at k0+32..k0+63; MFMA j of the block takes elements 8j..8j+7 of each lane's run,
// the same k positions for X and W.
#include "common.hpp"

namespace ta {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum { EPI_NONE = 0, EPI_GELU = 1, EPI_RESIDUAL = 2 };

__device__ __forceinline__ float bf16_round(float x) { return to_f32(bf16_from(x)); }

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)bf16_from(a).bits | ((uint32_t)bf16_from(b).bits << 16);
}

constexpr int kRowmmWaves = 8;   // wavefronts per workgroup, each taking up to kRowmmBlk K-blocks at once
constexpr int kRowmmBlk = 4;

template <bool LN, int EPI>
__global__ __launch_bounds__(kRowmmWaves * 64) void rowmm_kernel(const bf16_t* __restrict__ X, int64_t ldx,
                                                                const bf16_t* __restrict__ W, int64_t ldw, bf16_t* Y,
                                                                int64_t ldy, const bf16_t* R, int64_t ldr,
                                                                const bf16_t* __restrict__ gam, float eps, int M, int N,
                                                                int K, int splits, float* __restrict__ part,
                                                                uint32_t* __restrict__ cnt) {
  constexpr int NT = kRowmmWaves * 64;
  __shared__ float s_mean[32], s_rstd[32];
  __shared__ float red[kRowmmWaves][32][33];
  const int tid = threadIdx.x;
  const int lane = lane_id(), w = wave_id();
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  // this workgroup's K blocks [blk0, blk1)
  const int nblk_all = K / 64;
  const int per = (nblk_all + splits - 1) / splits;
  const int blk0 = blockIdx.z * per;
  const int blk1 = blk0 + per < nblk_all ? blk0 + per : nblk_all;
  const int nblk = blk1 - blk0;
  // LayerNorm statistics from the X blocks the wavefronts load for the product when one round of loads
  // covers all of K; otherwise a separate pass over the rows first
  const bool stats_from_blocks = splits == 1 && nblk <= kRowmmWaves * kRowmmBlk;

  // the residual tile of the epilogue, loaded up front
  constexpr int EPT = 1024 / NT;   // epilogue elements per thread
  float rres[EPT];
  if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * NT;
      const int gm = m0 + (e >> 5), gn = n0 + (e & 31);
      rres[k] = (gm < M && gn < N) ? to_f32(R[(int64_t)gm * ldr + gn]) : 0.0f;
    }
  }

  if (LN && !stats_from_blocks) {
    // row statistics in one pass (sum and sum of squares), TPR threads per row
    constexpr int TPR = NT / 32;
    const int r = tid / TPR, part = tid % TPR;
    const bool ok = m0 + r < M;
    const bf16_t* xr = X + (int64_t)(m0 + r) * ldx;
    float s = 0.0f, s2 = 0.0f;
    if (ok)
      for (int k = part * 8; k < K; k += TPR * 8) {
        float f[8];
        load_row<bf16_t, 8>(xr + k, f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          s += f[i];
          s2 = fmaf(f[i], f[i], s2);
        }
      }
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) {
      s += __shfl_xor(s, o, kWave);
      s2 += __shfl_xor(s2, o, kWave);
    }
    if (part == 0) {
      const float mean = s / (float)K;
      const float var = fmaxf(s2 / (float)K - mean * mean, 0.0f);
      s_mean[r] = mean;
      s_rstd[r] = rsqrtf(var + eps);
    }
    __syncthreads();
  }

  const int rl = lane & 31;      // row of X and row of W (output column) this lane feeds
  const int kh = (lane >> 5) * 32;
  const bool xok = m0 + rl < M;
  const bool wok = n0 + rl < N;
  const bf16_t* xr = X + (int64_t)(m0 + (xok ? rl : 0)) * ldx + kh;
  const bf16_t* wr = W + (int64_t)(n0 + (wok ? rl : 0)) * ldw + kh;
  float mean = 0.0f, rstd = 0.0f;
  if (LN && !stats_from_blocks) {
    mean = s_mean[rl];
    rstd = s_rstd[rl];
  }
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  xr += blk0 * 64;
  wr += blk0 * 64;
  const bf16_t* gk = LN ? gam + blk0 * 64 : gam;
  for (int base = 0; base < nblk; base += kRowmmWaves * kRowmmBlk) {
    uint4 xa[kRowmmBlk][4], wb[kRowmmBlk][4], ga[LN ? kRowmmBlk : 1][4];
#pragma unroll
    for (int i = 0; i < kRowmmBlk; ++i) {
      const int blk = base + w + kRowmmWaves * i;
      const bool bok = blk < nblk;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wb[i][j] = (bok && wok) ? *reinterpret_cast<const uint4*>(wr + blk * 64 + 8 * j) : make_uint4(0, 0, 0, 0);
        xa[i][j] = (bok && xok) ? *reinterpret_cast<const uint4*>(xr + blk * 64 + 8 * j) : make_uint4(0, 0, 0, 0);
        if constexpr (LN)
          ga[i][j] = bok ? *reinterpret_cast<const uint4*>(gk + blk * 64 + kh + 8 * j) : make_uint4(0, 0, 0, 0);
      }
    }
    if (LN && stats_from_blocks) {
      // lanes rl and rl + 32 hold the two halves of row rl of each of this wavefront's blocks
      float sx = 0.0f, sxx = 0.0f;
#pragma unroll
      for (int i = 0; i < kRowmmBlk; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float f[8];
          const bf16_t* xe = reinterpret_cast<const bf16_t*>(&xa[i][j]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            f[e] = to_f32(xe[e]);
            sx += f[e];
            sxx = fmaf(f[e], f[e], sxx);
          }
        }
      }
      sx += __shfl_xor(sx, 32, kWave);
      sxx += __shfl_xor(sxx, 32, kWave);
      if (lane < 32) {
        red[w][0][lane] = sx;
        red[w][1][lane] = sxx;
      }
      __syncthreads();
      float ts = 0.0f, tss = 0.0f;
#pragma unroll
      for (int v = 0; v < kRowmmWaves; ++v) {
        ts += red[v][0][rl];
        tss += red[v][1][rl];
      }
      mean = ts / (float)K;
      rstd = rsqrtf(fmaxf(tss / (float)K - mean * mean, 0.0f) + eps);
      __syncthreads();   // red is reused for the output tile
    }
#pragma unroll
    for (int i = 0; i < kRowmmBlk; ++i) {
      const int blk = base + w + kRowmmWaves * i;
      if (blk >= nblk) break;
      if constexpr (LN) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float f[8], gg[8];
          const bf16_t* xe = reinterpret_cast<const bf16_t*>(&xa[i][j]);
          const bf16_t* ge = reinterpret_cast<const bf16_t*>(&ga[i][j]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            f[e] = to_f32(xe[e]);
            gg[e] = to_f32(ge[e]);
          }
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack2((f[2 * e] - mean) * rstd * gg[2 * e], (f[2 * e + 1] - mean) * rstd * gg[2 * e + 1]);
          xa[i][j] = xok ? make_uint4(o[0], o[1], o[2], o[3]) : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x8 av, bv;
        __builtin_memcpy(&av, &xa[i][j], 16);
        __builtin_memcpy(&bv, &wb[i][j], 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
      }
    }
  }
  // output layout of the 32x32 MFMA tile: lane -> column lane % 32; register i -> row 8(i/4) + 4(lane/32) + i%4
#pragma unroll
  for (int i = 0; i < 16; ++i) red[w][8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)][lane & 31] = acc[i];
  __syncthreads();
  const int tile = blockIdx.y * gridDim.x + blockIdx.x;
  if (splits > 1) {
    // partial tile -> workspace; the last workgroup of the tile to arrive goes on to the epilogue
    float* mine = part + ((int64_t)blockIdx.z * gridDim.x * gridDim.y + tile) * 1024;
    for (int e = tid; e < 1024; e += NT) {
      const int r = e >> 5, c = e & 31;
      float v = red[0][r][c];
#pragma unroll
      for (int s = 1; s < kRowmmWaves; ++s) v += red[s][r][c];
      __hip_atomic_store(&mine[e], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);   // written through
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wavefront's stores have completed
    __syncthreads();
    __shared__ uint32_t s_last;
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
               (uint32_t)(splits - 1);
    __syncthreads();
    if (!s_last) return;
  }
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + k * NT;
    const int r = e >> 5, c = e & 31;
    const int gm = m0 + r, gn = n0 + c;
    if (gm < M && gn < N) {
      float v;
      if (splits > 1) {
        const int64_t stride = (int64_t)gridDim.x * gridDim.y * 1024;
        const float* p = part + (int64_t)tile * 1024 + e;
        v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);   // bypassing the caches
        for (int s = 1; s < splits; ++s)
          v += __hip_atomic_load(p + s * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      } else {
        v = red[0][r][c];
#pragma unroll
        for (int s = 1; s < kRowmmWaves; ++s) v += red[s][r][c];
      }
      v = bf16_round(v);
      if constexpr (EPI == EPI_GELU) v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
      if constexpr (EPI == EPI_RESIDUAL) v = rres[k] + v;
      Y[(int64_t)gm * ldy + gn] = bf16_from(v);
    }
  }
  if (splits > 1 && tid == 0)   // ready for the next call
    __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace ta

using namespace ta;

namespace {

constexpr int64_t kRowmmCountBytes = 4096;   // tile counters at the head of the workspace

int64_t rowmm_tiles(int M, int N) { return (int64_t)((N + 31) / 32) * ((M + 31) / 32); }

int rowmm_splits(int K, int splits) {
  const int nblk = K / 64;
  if (splits < 1) splits = 1;
  if (splits > nblk) splits = nblk;
  const int per = (nblk + splits - 1) / splits;
  return (nblk + per - 1) / per;   // no empty split
}

}  // namespace

extern "C" int64_t ta_rowmm_workspace_size(int M, int N, int K, int splits) {
  if (M <= 0 || N <= 0 || K < 64) return 0;
  const int s = rowmm_splits(K, splits);
  if (s <= 1) return 0;
  return kRowmmCountBytes + (int64_t)s * rowmm_tiles(M, N) * 1024 * 4;
}

extern "C" int ta_rowmm(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                        const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                        int epilogue, int splits, void* ws, int64_t ws_bytes, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || ldx < K || ldw < K || ldy < N ||
      (epilogue == EPI_RESIDUAL && (R == nullptr || ldr < N)) || epilogue < 0 || epilogue > 2) {
    set_error("ta_rowmm: bad sizes (K must be a multiple of 64)");
    return TA_ERR_ARG;
  }
  if (((uintptr_t)X | (uintptr_t)W) % 16 || (ldx * 2) % 16 || (ldw * 2) % 16 ||
      (ln_w != nullptr && (uintptr_t)ln_w % 16)) {
    set_error("ta_rowmm: X, W and the LayerNorm weight must be 16-byte aligned with 16-byte row strides");
    return TA_ERR_ARG;
  }
  const int S = rowmm_splits(K, splits);
  float* part = nullptr;
  uint32_t* cnt = nullptr;
  if (S > 1) {
    if (rowmm_tiles(M, N) * 4 > kRowmmCountBytes) {
      set_error("ta_rowmm: too many output tiles for a split product (at most 1024)");
      return TA_ERR_UNSUPPORTED;
    }
    if (ws == nullptr || ws_bytes < ta_rowmm_workspace_size(M, N, K, splits) || (uintptr_t)ws % 256) {
      set_error("ta_rowmm: workspace missing, too small or not 256-byte aligned");
      return TA_ERR_WORKSPACE;
    }
    cnt = (uint32_t*)ws;
    part = (float*)((char*)ws + kRowmmCountBytes);
  }
  dim3 grid((N + 31) / 32, (M + 31) / 32, S);
  hipStream_t st = (hipStream_t)stream;
  const bf16_t* x = (const bf16_t*)X;
  const bf16_t* w = (const bf16_t*)W;
  bf16_t* y = (bf16_t*)Y;
  const bf16_t* r = (const bf16_t*)R;
  const bf16_t* g = (const bf16_t*)ln_w;
#define TA_LAUNCH(LNF, E)                                                                                   \
  hipLaunchKernelGGL((rowmm_kernel<LNF, E>), grid, dim3(kRowmmWaves * 64), 0, st, x, ldx, w, ldw, y, ldy, r, ldr, g, ln_eps, M, \
                     N, K, S, part, cnt)
  if (ln_w) {
    if (epilogue == EPI_NONE) TA_LAUNCH(true, EPI_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(true, EPI_GELU);
    else TA_LAUNCH(true, EPI_RESIDUAL);
  } else {
    if (epilogue == EPI_NONE) TA_LAUNCH(false, EPI_NONE);
    else if (epilogue == EPI_GELU) TA_LAUNCH(false, EPI_GELU);
    else TA_LAUNCH(false, EPI_RESIDUAL);
  }
#undef TA_LAUNCH
  return check_launch("rowmm_kernel");
}
