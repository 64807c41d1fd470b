// device_common.h -- small device helpers shared by the decode kernels.
//
// Wavefront is 64 lanes (CDNA4).  All reductions are deterministic: fixed
// butterfly order, no float atomics.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define TALOS_WAVE 64

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, TALOS_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, TALOS_WAVE));
  return v;
}

// Sum over a block of `nwaves` waves through LDS scratch (>= nwaves floats).
// Every thread receives the total.  Contains two __syncthreads().
__device__ __forceinline__ float block_sum(float v, float* scratch, int nwaves) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < nwaves; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

// f32::total_cmp key (src/sample.rs:9 orders logits with total_cmp).
__device__ __forceinline__ int32_t total_key(float f) {
  int32_t i = __float_as_int(f);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// Unsigned byte k of a dword as float (v_cvt_f32_ubyte{k}).
__device__ __forceinline__ float ub0(uint32_t v) { return (float)(v & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t v) { return (float)(v >> 24); }

// Dot of the four unsigned bytes of `q` with x4, accumulated onto acc.
__device__ __forceinline__ float dot_ub4(uint32_t q, f4 x, float acc) {
  acc = __builtin_fmaf(ub0(q), x.x, acc);
  acc = __builtin_fmaf(ub1(q), x.y, acc);
  acc = __builtin_fmaf(ub2(q), x.z, acc);
  acc = __builtin_fmaf(ub3(q), x.w, acc);
  return acc;
}
