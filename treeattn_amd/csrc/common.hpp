// Shared device helpers for the gfx950 kernels of the segment-tree attention library.
//
// Element types, vector loads of a row slice into fp32 registers, wavefront (64-lane) reductions and the
// canonical fp32 dot product used wherever a score decides a selection.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/treeattn.h"

namespace ta {

constexpr int kWave = 64;
constexpr int kMaxLevels = 32;

// ----------------------------------------------------------------------------------------- element types
struct bf16_t { uint16_t bits; };
using f16_t = _Float16;

template <int DT> struct ElemOf;
template <> struct ElemOf<TA_F32> { using T = float; };
template <> struct ElemOf<TA_F16> { using T = f16_t; };
template <> struct ElemOf<TA_BF16> { using T = bf16_t; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(((uint32_t)x.bits) << 16); }

// float -> bf16, round to nearest even (gfx950's v_cvt_pk_bf16_f32; NaN stays NaN)
__device__ __forceinline__ bf16_t bf16_from(float f) {
  bf16_t r;
  r.bits = __builtin_bit_cast(uint16_t, (__bf16)f);
  return r;
}

// two floats -> two bf16 (a in the low half), one conversion instruction
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack2(float a, float b) {
  const bf16x2_t v = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return (f16_t)x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return bf16_from(x); }

// Load N consecutive elements of type T starting at p (aligned to N * sizeof(T) bytes, at most 16 bytes
// per instruction) into fp32 registers.
template <typename T, int N>
__device__ __forceinline__ void load_row(const T* __restrict__ p, float (&out)[N]) {
  constexpr int kBytes = N * (int)sizeof(T);
  constexpr int kChunk = kBytes >= 16 ? 16 : kBytes;
  constexpr int kPer = kChunk / (int)sizeof(T);
  static_assert(kBytes % kChunk == 0, "row slice must be a whole number of chunks");
#pragma unroll
  for (int c = 0; c < N / kPer; ++c) {
    if constexpr (kChunk == 16) {
      uint4 u = *reinterpret_cast<const uint4*>(p + c * kPer);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(e[i]);
    } else if constexpr (kChunk == 8) {
      uint2 u = *reinterpret_cast<const uint2*>(p + c * kPer);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(e[i]);
    } else if constexpr (kChunk == 4) {
      uint32_t u = *reinterpret_cast<const uint32_t*>(p + c * kPer);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(e[i]);
    } else {
      uint16_t u = *reinterpret_cast<const uint16_t*>(p + c * kPer);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(e[i]);
    }
  }
}

// ----------------------------------------------------------------------------------------- address spaces
// Pointers that reach a function through memory (a plan in device memory, a non-inlined call) are generic;
// loads through them become flat instructions, which count against the LDS counter too and so make every
// LDS access wait for them.  These helpers state that the address is device memory.
#define TA_GLOBAL __attribute__((address_space(1)))
typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ldg16(const void* p) {
  const u32x4_t v = *(const TA_GLOBAL u32x4_t*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Device-coherent loads and stores ("dc": device scope, coherent across the XCDs' L2 caches), for data that
// other workgroups of the running kernel write or read.
__device__ __forceinline__ uint64_t ldg8_dc(const void* p) {
  return __hip_atomic_load((TA_GLOBAL uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ldg16_dc(const void* p) {
  const uint64_t a = ldg8_dc(p), b = ldg8_dc((const char*)p + 8);
  return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}
__device__ __forceinline__ uint32_t ldg4_dc(const void* p) {
  return __hip_atomic_load((TA_GLOBAL uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint16_t ldg2_dc(const void* p) {
  return __hip_atomic_load((TA_GLOBAL uint16_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldgf_dc(const float* p) {
  return __hip_atomic_load((TA_GLOBAL float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stg8_dc(void* p, uint64_t v) {
  __hip_atomic_store((TA_GLOBAL uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stg4_dc(void* p, uint32_t v) {
  __hip_atomic_store((TA_GLOBAL uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stg2_dc(void* p, uint16_t v) {
  __hip_atomic_store((TA_GLOBAL uint16_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stgf_dc(float* p, float v) {
  __hip_atomic_store((TA_GLOBAL float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// load_row from device memory (see load_row)
template <typename T, int N>
__device__ __forceinline__ void load_row_g(const T* p, float (&out)[N]) {
  constexpr int kBytes = N * (int)sizeof(T);
  if constexpr (kBytes % 16 == 0) {
    constexpr int kPer = 16 / (int)sizeof(T);
#pragma unroll
    for (int c = 0; c < N / kPer; ++c) {
      const uint4 u = ldg16(p + c * kPer);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < kPer; ++i) out[c * kPer + i] = to_f32(e[i]);
    }
  } else {
    load_row<T, N>(p, out);
  }
}

// s_waitcnt vmcnt(N) with the LDS and export counters left alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt_n() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for LDS traffic only: this wavefront's LDS operations complete, then s_barrier.  Unlike
// __syncthreads() (whose workgroup-scope release fence waits for every outstanding memory load as well) it
// leaves global loads in flight, so they can overlap the LDS work that follows; data copied into LDS by
// global_load_lds must be waited for with wait_vmcnt_n before it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ----------------------------------------------------------------------------------------- wave helpers
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x / kWave); }

// Order LDS traffic between lanes of one wavefront (the wave's own LDS region; no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G a power of two up to 64); every lane of a group gets the sum.
// Quad permutes pair lanes within quads; after them the value repeats every 4 lanes, so mirroring each
// half-row (lane j <-> 7 - j) pairs the two quads of an 8-lane group, and mirroring the row (j <-> 15 - j)
// the two halves of a 16-lane group.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (G >= 2) x += dpp_f<0xB1>(x);    // quad_perm [1,0,3,2]
  if constexpr (G >= 4) x += dpp_f<0x4E>(x);    // quad_perm [2,3,0,1]
  if constexpr (G >= 8) x += dpp_f<0x141>(x);   // row_half_mirror
  if constexpr (G >= 16) x += dpp_f<0x140>(x);  // row_mirror
  if constexpr (G >= 32) x += __shfl_xor(x, 16, kWave);
  if constexpr (G >= 64) x += __shfl_xor(x, 32, kWave);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// ----------------------------------------------------------------------------------------- host helpers
void set_error(const std::string& msg);
int check_launch(const char* what);
// The current device's compute-unit count and LDS bytes per compute unit (queried once per device; 0 if the
// query fails).
int device_cus();
int device_lds_per_cu();
int gather_blocks_mfma(const void* q, const void* K, int dtype, int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb,
                       int64_t ksh, int64_t ksn, const int32_t* blk, int B, int H, int N, int M, int NB, int block, int D,
                       float scale, float* out, void* stream);

}  // namespace ta
