// float32 row products of a decode step for a few rows (the float32 decoder's step, engine.py:168-177:
// F.linear(ln_1(x), c_attn), x + F.linear(y, c_proj), F.gelu(F.linear(ln_2(x), c_fc)), x + F.linear(h, c_mlp),
// F.linear(ln_f(x), wte)), each product with its LayerNorm prologue and its epilogue in one launch.
//
// One wavefront per output column n: it holds W's row n (lane l: elements l, l + 64, ...) in registers, and for
// each input row m the row's elements the same way; the LayerNorm statistics of the row (mean, then the mean
// of the squared deviations, both reduced over the wavefront) are taken by every wavefront that reads the row,
// the normalised element is (x - mean) * rstd * w_ln, the dot product is the lanes' partial sums reduced over the
// wavefront, and lane 0 applies the epilogue and writes Y[m, n].  At batch 1 a product is a few round trips
// (the rows and W's row requested together), not bandwidth.
//
// The bf16 form (the bf16 decoder's products for one or two rows, where the matrix-core tiles of ta_rowmm compute
// 31 or 30 idle rows of every 32) keeps ta_rowmm's arithmetic at every rounding point: the LayerNorm statistics
// from the float32 sums of x and x^2 (mm_stats), the normalised row rounded to bf16 (mm_ln_piece), float32
// products of bf16 values (exact) summed in float32, and mm_epilogue (the sum rounded to bf16, then GELU or the
// residual, rounded again).  Only the order of the float32 sums differs from ta_rowmm's, so the two agree to the
// last bf16 bit in most outputs and within one bf16 unit in the rest.  A lane holds 16-byte pieces (8 elements)
// l, l + 64, ... of a row.
#include "rowmm_tile.hpp"

namespace ta {

constexpr int kRvWaves = 4;                    // wavefronts (output columns) per workgroup
constexpr int kRvMaxK = 2048;                  // input width
constexpr int kRvMaxM = 8;                     // rows

// P: elements of a row per lane (8, 16 or 32: the smallest that holds K)
template <int EPI, bool LN, int P>
__global__ __launch_bounds__(kRvWaves * kWave) void rowvec_f32_kernel(
    const float* __restrict__ X, int64_t ldx, const float* __restrict__ W, int64_t ldw, const float* __restrict__ lnw,
    float eps, const float* R, int64_t ldr, float* Y, int64_t ldy, int M, int N, int K) {
  const int lane = lane_id();
  const int n = blockIdx.x * kRvWaves + wave_id();
  if (n >= N) return;   // a whole wavefront leaves; no barrier follows
  const float* wr = W + (int64_t)n * ldw;
  float wv[P], gv[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int k = i * kWave + lane;
    wv[i] = k < K ? wr[k] : 0.0f;
    if constexpr (LN) gv[i] = k < K ? lnw[k] : 0.0f;
  }
  for (int m = 0; m < M; ++m) {
    const float* xr = X + (int64_t)m * ldx;
    float xv[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int k = i * kWave + lane;
      xv[i] = k < K ? xr[k] : 0.0f;
    }
    if constexpr (LN) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < P; ++i) s += xv[i];
      const float mean = wave_sum(s) / (float)K;
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const float d = i * kWave + lane < K ? xv[i] - mean : 0.0f;
        v += d * d;
      }
      const float rstd = rsqrtf(wave_sum(v) / (float)K + eps);
#pragma unroll
      for (int i = 0; i < P; ++i) xv[i] = (xv[i] - mean) * rstd * gv[i];
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) acc += xv[i] * wv[i];
    acc = wave_sum(acc);
    if (lane == 0) {
      float y = acc;
      if constexpr (EPI == 1) y = 0.5f * y * (1.0f + erff(y * 0.70710678118654752f));   // exact GELU
      if constexpr (EPI == 2) y = R[(int64_t)m * ldr + n] + y;                              // residual
      Y[(int64_t)m * ldy + n] = y;
    }
  }
}

// PP: 16-byte pieces of a row per lane (1 to 8: the smallest that holds K / 8 pieces)
constexpr int kRvMaxKb = 4096;
template <int EPI, bool LN, int PP>
__global__ __launch_bounds__(kRvWaves * kWave) void rowvec_bf16_kernel(
    const bf16_t* __restrict__ X, int64_t ldx, const bf16_t* __restrict__ W, int64_t ldw,
    const bf16_t* __restrict__ lnw, float eps, const bf16_t* R, int64_t ldr, bf16_t* Y, int64_t ldy, int M, int N,
    int K) {
  const int lane = lane_id();
  const int n = blockIdx.x * kRvWaves + wave_id();
  if (n >= N) return;   // a whole wavefront leaves; no barrier follows
  const int np = K / 8;   // pieces of a row
  const bf16_t* wr = W + (int64_t)n * ldw;
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  uint4 wv[PP], gv[PP];
#pragma unroll
  for (int i = 0; i < PP; ++i) {
    const int pc = i * kWave + lane;
    wv[i] = pc < np ? ldg16(wr + 8 * pc) : zero;
    if constexpr (LN) gv[i] = pc < np ? ldg16(lnw + 8 * pc) : zero;
  }
  for (int m = 0; m < M; ++m) {
    const bf16_t* xr = X + (int64_t)m * ldx;
    uint4 xv[PP];
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const int pc = i * kWave + lane;
      xv[i] = pc < np ? ldg16(xr + 8 * pc) : zero;   // zero pieces add nothing to the sums
    }
    if constexpr (LN) {
      float s = 0.0f, s2 = 0.0f;
#pragma unroll
      for (int i = 0; i < PP; ++i) mm_add8(xv[i], s, s2);
      float mean, rstd;
      mm_stats(wave_sum(s), wave_sum(s2), K, eps, mean, rstd);
#pragma unroll
      for (int i = 0; i < PP; ++i) xv[i] = mm_ln_piece(xv[i], gv[i], mean, rstd);   // zero weights: zero pieces
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const uint32_t xw[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = fmaf(__uint_as_float(xw[e] << 16), __uint_as_float(ww[e] << 16), acc);
        acc = fmaf(__uint_as_float(xw[e] & 0xffff0000u), __uint_as_float(ww[e] & 0xffff0000u), acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const float res = EPI == EPI_RESIDUAL ? to_f32(R[(int64_t)m * ldr + n]) : 0.0f;
      Y[(int64_t)m * ldy + n] = mm_epilogue<EPI>(acc, res);
    }
  }
}

}  // namespace ta

using namespace ta;

extern "C" int ta_rowvec_f32(const float* X, int64_t ldx, const float* W, int64_t ldw, float* Y, int64_t ldy,
                             const float* R, int64_t ldr, const float* ln_w, float ln_eps, int M, int N, int K,
                             int epilogue, void* stream) {
  if (X == nullptr || W == nullptr || Y == nullptr || M < 1 || M > kRvMaxM || N < 1 || K < 1 || K > kRvMaxK ||
      ldx < K || ldw < K || ldy < N || epilogue < 0 || epilogue > 2 || (epilogue == 2 && (R == nullptr || ldr < N)) ||
      (ln_w != nullptr && !(ln_eps >= 0.0f))) {
    set_error("ta_rowvec_f32: bad arguments (1 <= M <= 8 rows, K <= 2048, strides at least the row widths, "
              "epilogue 0 / 1 (GELU) / 2 (residual, R given))");
    return TA_ERR_ARG;
  }
  const float* Xe = X + (int64_t)(M - 1) * ldx;   // X and Y (or R and Y) may coincide only element for element
  const float* Ye = Y + (int64_t)(M - 1) * ldy + N;
  if (X < Ye && Y < Xe + K) {
    set_error("ta_rowvec_f32: X and Y overlap");
    return TA_ERR_ARG;
  }
  const unsigned grid = (unsigned)((N + kRvWaves - 1) / kRvWaves);
  hipStream_t st = (hipStream_t)stream;
#define TA_RV(E, LNB, PP)                                                                                          \
  hipLaunchKernelGGL((rowvec_f32_kernel<E, LNB, PP>), dim3(grid), dim3(kRvWaves * kWave), 0, st, X, ldx, W, ldw, \
                     ln_w, ln_eps, R, ldr, Y, ldy, M, N, K)
#define TA_RV_P(E, LNB)                 \
  if (K <= 8 * kWave) TA_RV(E, LNB, 8);   \
  else if (K <= 16 * kWave) TA_RV(E, LNB, 16); \
  else TA_RV(E, LNB, 32);
  if (ln_w != nullptr) {
    if (epilogue == 0) { TA_RV_P(0, true) }
    else if (epilogue == 1) { TA_RV_P(1, true) }
    else { TA_RV_P(2, true) }
  } else {
    if (epilogue == 0) { TA_RV_P(0, false) }
    else if (epilogue == 1) { TA_RV_P(1, false) }
    else { TA_RV_P(2, false) }
  }
#undef TA_RV_P
#undef TA_RV
  return check_launch("ta_rowvec_f32");
}

extern "C" int ta_rowvec_bf16(const void* X, int64_t ldx, const void* W, int64_t ldw, void* Y, int64_t ldy,
                              const void* R, int64_t ldr, const void* ln_w, float ln_eps, int M, int N, int K,
                              int epilogue, void* stream) {
  if (X == nullptr || W == nullptr || Y == nullptr || M < 1 || M > kRvMaxM || N < 1 || K < 8 || K > kRvMaxKb ||
      K % 8 || ldx < K || ldw < K || ldy < N || ldx % 8 || ldw % 8 || epilogue < 0 || epilogue > 2 ||
      (epilogue == 2 && (R == nullptr || ldr < N)) || (ln_w != nullptr && !(ln_eps >= 0.0f)) ||
      ((uintptr_t)X | (uintptr_t)W | (uintptr_t)ln_w) % 16) {
    set_error("ta_rowvec_bf16: bad arguments (1 <= M <= 8 rows, K a multiple of 8 up to 4096, X, W and ln_w "
              "16-byte aligned with row strides a multiple of 8 elements, epilogue 0 / 1 (GELU) / 2 (residual, R "
              "given))");
    return TA_ERR_ARG;
  }
  const bf16_t* Xb = (const bf16_t*)X;
  bf16_t* Yb = (bf16_t*)Y;
  if (Xb < Yb + (int64_t)(M - 1) * ldy + N && Yb < Xb + (int64_t)(M - 1) * ldx + K) {
    set_error("ta_rowvec_bf16: X and Y overlap");
    return TA_ERR_ARG;
  }
  const unsigned grid = (unsigned)((N + kRvWaves - 1) / kRvWaves);
  hipStream_t st = (hipStream_t)stream;
  const int pp = (K / 8 + kWave - 1) / kWave;
#define TA_RB(E, LNB, PP)                                                                                        \
  hipLaunchKernelGGL((rowvec_bf16_kernel<E, LNB, PP>), dim3(grid), dim3(kRvWaves * kWave), 0, st, Xb, ldx,      \
                     (const bf16_t*)W, ldw, (const bf16_t*)ln_w, ln_eps, (const bf16_t*)R, ldr, Yb, ldy, M, N, K)
#define TA_RB_P(E, LNB)                 \
  if (pp <= 2) TA_RB(E, LNB, 2);        \
  else if (pp <= 4) TA_RB(E, LNB, 4);   \
  else TA_RB(E, LNB, 8);
  if (ln_w != nullptr) {
    if (epilogue == 0) { TA_RB_P(EPI_NONE, true) }
    else if (epilogue == 1) { TA_RB_P(EPI_GELU, true) }
    else { TA_RB_P(EPI_RESIDUAL, true) }
  } else {
    if (epilogue == 0) { TA_RB_P(EPI_NONE, false) }
    else if (epilogue == 1) { TA_RB_P(EPI_GELU, false) }
    else { TA_RB_P(EPI_RESIDUAL, false) }
  }
#undef TA_RB_P
#undef TA_RB
  return check_launch("ta_rowvec_bf16");
}
