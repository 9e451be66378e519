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

// float -> bf16, round to nearest even (NaN kept quiet)
__device__ __forceinline__ bf16_t bf16_from(float f) {
  uint32_t u = __float_as_uint(f);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = (uint16_t)((u >> 16) | 0x40u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = (uint16_t)(u >> 16);
  }
  return r;
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

// ----------------------------------------------------------------------------------------- wave helpers
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x / kWave); }

// Order LDS traffic between lanes of one wavefront (the wave's own LDS region; no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
int gather_blocks_mfma(const void* q, const void* K, int dtype, int64_t qsb, int64_t qsh, int64_t qsn, int64_t ksb,
                       int64_t ksh, int64_t ksn, const int32_t* blk, int B, int H, int N, int M, int NB, int block, int D,
                       float scale, float* out, void* stream);

}  // namespace ta
