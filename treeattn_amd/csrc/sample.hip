// Greedy token choice for the decode loop: row-wise argmax (first index among equal maxima), one
// workgroup per row.  Replaces logits.argmax(-1) of the reference's greedy loop (phase2.py:51-66) so a
// captured decode step holds no library reduction.
#include "common.hpp"

namespace ta {

template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T* __restrict__ x, int64_t n, int64_t stride,
                                                          int64_t* __restrict__ out) {
  __shared__ float s_val[1024];
  __shared__ int64_t s_idx[1024];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * stride;
  float best = -INFINITY;
  int64_t bi = n;  // sentinel: larger than any index
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = to_f32(xr[i]);
    if (v > best || (v == best && i < bi)) {
      best = v;
      bi = i;
    }
  }
  s_val[threadIdx.x] = best;
  s_idx[threadIdx.x] = bi;
  __syncthreads();
  for (int o = blockDim.x / 2; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) {
      const float v = s_val[threadIdx.x + o];
      const int64_t j = s_idx[threadIdx.x + o];
      if (v > s_val[threadIdx.x] || (v == s_val[threadIdx.x] && j < s_idx[threadIdx.x])) {
        s_val[threadIdx.x] = v;
        s_idx[threadIdx.x] = j;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[row] = s_idx[0] < n ? s_idx[0] : 0;
}

}  // namespace ta

using namespace ta;

extern "C" int ta_argmax_rows(const void* x, int dtype, int64_t rows, int64_t n, int64_t stride, int64_t* out,
                              void* stream) {
  if (rows < 0 || n <= 0 || stride < n) {
    set_error("ta_argmax_rows: bad sizes");
    return TA_ERR_ARG;
  }
  if (rows == 0) return TA_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)rows);
  switch (dtype) {
    case TA_F32:
      hipLaunchKernelGGL((argmax_rows_kernel<float>), grid, dim3(1024), 0, st, (const float*)x, n, stride, out);
      break;
    case TA_F16:
      hipLaunchKernelGGL((argmax_rows_kernel<f16_t>), grid, dim3(1024), 0, st, (const f16_t*)x, n, stride, out);
      break;
    case TA_BF16:
      hipLaunchKernelGGL((argmax_rows_kernel<bf16_t>), grid, dim3(1024), 0, st, (const bf16_t*)x, n, stride, out);
      break;
    default:
      set_error("unknown dtype");
      return TA_ERR_ARG;
  }
  return check_launch("argmax_rows_kernel");
}
