// Phase marks.  A kernel marks its phases with TA_DMARK(i) (i < 16); in the library build a mark is nothing.  A
// tracing build of one source (python -m treeattn_amd.phase_trace compiles it with -DTA_TRACE into its own
// library) turns each mark into a store, by the workgroup's first thread, of the 100 MHz real-time counter
// (s_memrealtime) into that source's trace buffer: 16 words per workgroup for the first 4096 workgroups of a
// launch, the grid flattened x-fastest.  The source then exports ta_trace_read and ta_trace_clear
// (TA_TRACE_EXPORTS at its end).
#pragma once

#ifdef TA_TRACE
#include <hip/hip_runtime.h>
namespace ta {
static __device__ unsigned long long ta_trace_buf[4096 * 16];
}  // namespace ta
#define TA_DMARK(i)                                                                          \
  do {                                                                                       \
    const unsigned int wg_ = blockIdx.y * gridDim.x + blockIdx.x;                            \
    if (threadIdx.x == 0 && wg_ < 4096)                                                      \
      ::ta::ta_trace_buf[wg_ * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                 \
  } while (0)
#define TA_TRACE_EXPORTS                                                                     \
  extern "C" int ta_trace_read(unsigned long long* host) {                                   \
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(::ta::ta_trace_buf),                    \
                                    sizeof(::ta::ta_trace_buf), 0, hipMemcpyDeviceToHost);   \
  }                                                                                          \
  extern "C" int ta_trace_clear() {                                                          \
    static unsigned long long z[4096 * 16];                                                  \
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(::ta::ta_trace_buf), z, sizeof(z), 0,           \
                                  hipMemcpyHostToDevice);                                    \
  }
#else
#define TA_DMARK(i) \
  do {              \
  } while (0)
#define TA_TRACE_EXPORTS
#endif
