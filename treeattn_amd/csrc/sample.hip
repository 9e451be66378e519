// Greedy token choice for the decode loop: row-wise argmax (first index among equal maxima), one
// workgroup per row.  Replaces logits.argmax(-1) of the reference's greedy loop (phase2.py:51-66) so a
// captured decode step holds no library reduction.
#include <type_traits>

#include "common.hpp"
#include "rowmm_tile.hpp"

namespace ta {

// (value, index) pairs: a is kept over b when larger, or equal with a smaller index
__device__ __forceinline__ void better_of(float& v, int64_t& i, float v2, int64_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Every thread issues all its loads (16-byte runs of the row, up to kArgmaxRuns in flight) before comparing;
// then the wavefronts reduce with shuffles and the workgroup through LDS.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxRuns = 8;

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const T* __restrict__ x, int64_t n,
                                                                    int64_t stride, int vec,
                                                                    int64_t* __restrict__ out) {
  constexpr int EPR = 16 / (int)sizeof(T);   // elements per 16-byte run
  __shared__ float s_val[kArgmaxThreads / kWave];
  __shared__ int64_t s_idx[kArgmaxThreads / kWave];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * stride;
  float best = -INFINITY;
  int64_t bi = n;  // sentinel: larger than any index
  if (vec) {
    const int64_t nruns = n / EPR;
    for (int64_t r0 = 0; r0 < nruns; r0 += (int64_t)kArgmaxThreads * kArgmaxRuns) {
      uint4 u[kArgmaxRuns];
#pragma unroll
      for (int k = 0; k < kArgmaxRuns; ++k) {
        const int64_t r = r0 + threadIdx.x + (int64_t)k * kArgmaxThreads;
        u[k] = r < nruns ? reinterpret_cast<const uint4*>(xr)[r] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < kArgmaxRuns; ++k) {
        const int64_t r = r0 + threadIdx.x + (int64_t)k * kArgmaxThreads;
        if (r < nruns) {
          const T* e = reinterpret_cast<const T*>(&u[k]);
#pragma unroll
          for (int m = 0; m < EPR; ++m) better_of(best, bi, to_f32(e[m]), r * EPR + m);
        }
      }
    }
  } else {
    for (int64_t i0 = 0; i0 < n; i0 += (int64_t)kArgmaxThreads * kArgmaxRuns) {
      float v[kArgmaxRuns];
#pragma unroll
      for (int k = 0; k < kArgmaxRuns; ++k) {
        const int64_t i = i0 + threadIdx.x + (int64_t)k * kArgmaxThreads;
        v[k] = i < n ? to_f32(xr[i]) : -INFINITY;
      }
#pragma unroll
      for (int k = 0; k < kArgmaxRuns; ++k) {
        const int64_t i = i0 + threadIdx.x + (int64_t)k * kArgmaxThreads;
        if (i < n) better_of(best, bi, v[k], i);
      }
    }
  }
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) {
    const float v2 = __shfl_xor(best, o, kWave);
    const int64_t i2 = __shfl_xor(bi, o, kWave);
    better_of(best, bi, v2, i2);
  }
  if (lane_id() == 0) {
    s_val[wave_id()] = best;
    s_idx[wave_id()] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) better_of(best, bi, s_val[w], s_idx[w]);
    out[row] = bi < n ? bi : 0;
  }
}

// The decode step's first op: x[b] = wte[tok[b]] + wpe[t[b]] rounded to the element type (as the
// reference's bf16 sum does), the positions as int32 for the later kernels, and optionally t[b] += 1 for
// the next step.  One workgroup per sequence; token and position clamped to the tables.  With ln_w (bf16,
// C a multiple of 64 and at most kEmbedLnMax): x_ln[b] = LN(x[b]) for the first layer's product, the
// arithmetic of the row products' LayerNorm (mm_rows_ln).
constexpr int kEmbedLnMax = 4096;

template <typename T>
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ tok, int64_t* tpos, int advance,
                                                    const T* __restrict__ wte, int64_t ldw, const T* __restrict__ wpe,
                                                    int64_t ldp, int C, int64_t V, int64_t P, T* __restrict__ x,
                                                    int64_t ldx, int32_t* __restrict__ pos32, const T* ln_w,
                                                    float eps, T* x_ln, int64_t ldxl) {
  const int b = blockIdx.x;
  int64_t tk = tok[b], t = tpos[b];
  tk = tk < 0 ? 0 : (tk >= V ? V - 1 : tk);
  const int64_t tc = t < 0 ? 0 : (t >= P ? P - 1 : t);
  const T* er = wte + tk * ldw;
  const T* pr = wpe + tc * ldp;
  T* xr = x + (int64_t)b * ldx;
  for (int c = threadIdx.x; c < C; c += blockDim.x) xr[c] = from_f32<T>(to_f32(er[c]) + to_f32(pr[c]));
  if constexpr (sizeof(T) == 2 && !std::is_same<T, f16_t>::value) {
    if (ln_w) {
      // the row as stored, then its LayerNorm: threads 0-7 take pieces 0-7 of every 64-column block
      __shared__ __align__(16) bf16_t srow[kEmbedLnMax];
      __shared__ float s_stat[2];
      for (int c = threadIdx.x; c < C; c += blockDim.x) srow[c] = xr[c];
      __syncthreads();
      if (threadIdx.x < 8) {
        float s = 0.0f, s2 = 0.0f;
        for (int k = 0; k < C; k += 64) mm_add8(*reinterpret_cast<const uint4*>(srow + k + 8 * threadIdx.x), s, s2);
        s = group_sum<8>(s);
        s2 = group_sum<8>(s2);
        if (threadIdx.x == 0) mm_stats(s, s2, C, eps, s_stat[0], s_stat[1]);
      }
      __syncthreads();
      const float mean = s_stat[0], rstd = s_stat[1];
      for (int k = 8 * threadIdx.x; k < C; k += 8 * blockDim.x) {
        const uint4 xu = *reinterpret_cast<const uint4*>(srow + k);
        const uint4 gu = *reinterpret_cast<const uint4*>(ln_w + k);
        const uint32_t xw[4] = {xu.x, xu.y, xu.z, xu.w}, gw[4] = {gu.x, gu.y, gu.z, gu.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f0 = __uint_as_float(xw[e] << 16), f1 = __uint_as_float(xw[e] & 0xffff0000u);
          const float g0 = __uint_as_float(gw[e] << 16), g1 = __uint_as_float(gw[e] & 0xffff0000u);
          o[e] = mm_pack2((f0 - mean) * rstd * g0, (f1 - mean) * rstd * g1);
        }
        *reinterpret_cast<uint4*>(x_ln + (int64_t)b * ldxl + k) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  __syncthreads();   // every thread has read tpos[b] before it may change
  if (threadIdx.x == 0) {
    pos32[b] = (int32_t)t;
    if (advance) tpos[b] = t + 1;
  }
}

// out[i] = bf16(in[i]) with the library's rounding (bf16_from), 4 per thread.
__global__ __launch_bounds__(256) void bf16_round_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                         int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i + 4 <= n) {
    const float4 v = *reinterpret_cast<const float4*>(in + i);
    *reinterpret_cast<uint2*>(out + i) = make_uint2(bf16_pack2(v.x, v.y), bf16_pack2(v.z, v.w));
  } else {
    for (int64_t j = i; j < n; ++j) out[j] = bf16_from(in[j]).bits;
  }
}

}  // namespace ta

using namespace ta;

extern "C" int ta_bf16_from_f32(const float* in, uint16_t* out, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (in == nullptr || out == nullptr || (uintptr_t)in % 16 || (uintptr_t)out % 8))) {
    set_error("ta_bf16_from_f32: bad arguments (in 16-byte and out 8-byte aligned)");
    return TA_ERR_ARG;
  }
  if (n == 0) return TA_OK;
  const int64_t blocks = (n + 1023) / 1024;
  hipLaunchKernelGGL(bf16_round_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, in, out, n);
  return check_launch("bf16_round_kernel");
}

extern "C" int ta_embed(const int64_t* tok, int64_t* tpos, int advance, const void* wte, int64_t ldw, const void* wpe,
                        int64_t ldp, int dtype, int B, int C, int64_t V, int64_t P, void* x, int64_t ldx,
                        int32_t* pos32, const void* ln_w, float ln_eps, void* x_ln, int64_t ld_xln, void* stream) {
  if (B <= 0 || C <= 0 || V <= 0 || P <= 0 || ldw < C || ldp < C || ldx < C) {
    set_error("ta_embed: bad sizes");
    return TA_ERR_ARG;
  }
  if (ln_w && (dtype != TA_BF16 || C % 64 || C > kEmbedLnMax || x_ln == nullptr || ld_xln < C ||
               (uintptr_t)ln_w % 16 || (uintptr_t)x_ln % 16 || (ld_xln * 2) % 16)) {
    set_error("ta_embed: the LayerNorm output needs bf16, C a multiple of 64 up to 4096 and 16-byte alignment");
    return TA_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL((embed_kernel<float>), dim3(B), dim3(256), 0, st, tok, tpos, advance, (const float*)wte, ldw,
                         (const float*)wpe, ldp, C, V, P, (float*)x, ldx, pos32, (const float*)nullptr, ln_eps,
                         (float*)nullptr, ld_xln);
      break;
    case TA_F16:
      hipLaunchKernelGGL((embed_kernel<f16_t>), dim3(B), dim3(256), 0, st, tok, tpos, advance, (const f16_t*)wte, ldw,
                         (const f16_t*)wpe, ldp, C, V, P, (f16_t*)x, ldx, pos32, (const f16_t*)nullptr, ln_eps,
                         (f16_t*)nullptr, ld_xln);
      break;
    case TA_BF16:
      hipLaunchKernelGGL((embed_kernel<bf16_t>), dim3(B), dim3(256), 0, st, tok, tpos, advance, (const bf16_t*)wte,
                         ldw, (const bf16_t*)wpe, ldp, C, V, P, (bf16_t*)x, ldx, pos32, (const bf16_t*)ln_w, ln_eps,
                         (bf16_t*)x_ln, ld_xln);
      break;
    default:
      set_error("unknown dtype");
      return TA_ERR_ARG;
  }
  return check_launch("embed_kernel");
}

extern "C" int ta_argmax_rows(const void* x, int dtype, int64_t rows, int64_t n, int64_t stride, int64_t* out,
                              void* stream) {
  if (rows < 0 || n <= 0 || stride < n) {
    set_error("ta_argmax_rows: bad sizes");
    return TA_ERR_ARG;
  }
  if (rows == 0) return TA_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)rows);
  const int esz = dtype == TA_F32 ? 4 : 2;
  // 16-byte runs when every row starts 16-byte aligned and holds whole runs
  const int vec = ((uintptr_t)x % 16 == 0 && (stride * esz) % 16 == 0 && (n * esz) % 16 == 0) ? 1 : 0;
  const dim3 blk(kArgmaxThreads);
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL((argmax_rows_kernel<float>), grid, blk, 0, st, (const float*)x, n, stride, vec, out);
      break;
    case TA_F16:
      hipLaunchKernelGGL((argmax_rows_kernel<f16_t>), grid, blk, 0, st, (const f16_t*)x, n, stride, vec, out);
      break;
    case TA_BF16:
      hipLaunchKernelGGL((argmax_rows_kernel<bf16_t>), grid, blk, 0, st, (const bf16_t*)x, n, stride, vec, out);
      break;
    default:
      set_error("unknown dtype");
      return TA_ERR_ARG;
  }
  return check_launch("argmax_rows_kernel");
}
