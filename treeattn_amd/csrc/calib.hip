// Calibration kernel for the measurement legs (no counterpart in the reference): the dense bf16 matrix-core
// throughput this GPU sustains, to set beside the vendor's figure when a kernel's MFMA utilisation is
// reported.  Every wavefront runs `iters` rounds of four independent v_mfma_f32_32x32x16_bf16 chains on
// register operands (no memory traffic in the loop); 32 * 32 * 16 * 2 flops per instruction.
#include "common.hpp"

namespace ta {

typedef __bf16 cal_bf16x8 __attribute__((ext_vector_type(8)));
typedef float cal_f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* out) {
  const int lane = lane_id();
  cal_bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (lane + i));
    b[i] = (__bf16)(0.002f * (lane - i));
  }
  cal_f32x16 c0, c1, c2, c3;
#pragma unroll
  for (int i = 0; i < 16; ++i) c0[i] = c1[i] = c2[i] = c3[i] = 0.0f;
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (s == 1234.5f) out[blockIdx.x] = s;   // keeps the chains live; never true for these operands
}

}  // namespace ta

using namespace ta;

// Runs wgs workgroups of four wavefronts, each wavefront 4 * iters MFMA instructions of 32768 flops.
extern "C" int ta_mfma_peak(int wgs, int iters, float* out, void* stream) {
  if (wgs <= 0 || iters <= 0 || out == nullptr) {
    set_error("ta_mfma_peak: bad arguments");
    return TA_ERR_ARG;
  }
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(wgs), dim3(256), 0, (hipStream_t)stream, iters, out);
  return check_launch("mfma_peak_kernel");
}
