// device_common.h -- small device helpers shared by the decode kernels.
//
// Wavefront is 64 lanes (CDNA4).  All reductions are deterministic: fixed
// order, no float atomics.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define TALOS_WAVE 64

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Pointers read from memory (rather than kernel arguments) are generic, and
// generic accesses compile to flat instructions, which also count against
// lgkmcnt: every LDS wait would then also wait for them.  These casts state
// that an address is in global memory, so the access is a global_* one.
#define TALOS_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const TALOS_GLOBAL T* gptr(const T* p) {
  return (const TALOS_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ TALOS_GLOBAL T* gptr(T* p) {
  return (TALOS_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ T gld(const T* p) {
  return *gptr(p);
}
__device__ __forceinline__ f4 gld4(const float* p) { return gld(reinterpret_cast<const f4*>(p)); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

// DPP lane moves (VOP_DPP controls of the CDNA ISA): quad permutes, row
// (16-lane) rotates and row broadcasts.  Lanes a row mask leaves out take
// `old`.
#define DPP_QUAD_1032 0xB1
#define DPP_QUAD_2301 0x4E
#define DPP_ROW_ROR4 0x124
#define DPP_ROW_ROR8 0x128
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xF, false));
}

// Sum over each quad of 4 lanes; every lane of the quad receives it.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_f<DPP_QUAD_1032>(0.f, v);
  v += dpp_f<DPP_QUAD_2301>(0.f, v);
  return v;
}

// Sum over each row of 16 lanes; every lane of the row receives it.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<DPP_QUAD_1032>(0.f, v);
  v += dpp_f<DPP_QUAD_2301>(0.f, v);
  v += dpp_f<DPP_ROW_ROR4>(0.f, v);
  v += dpp_f<DPP_ROW_ROR8>(0.f, v);
  return v;
}

// x combined with the x of lane ^ 16 (lane ^ 32) by a commutative op, the
// same bits in both lanes of a pair: v_permlane16_swap (v_permlane32_swap)
// with x as both operands leaves each lane's own and partner values in the
// two results, a VALU exchange in place of an LDS permute.
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over the 64 lanes of a wave (row sums, then rows 0+1 into row 1,
// 2+3 into row 3, then row 1 into rows 2-3; lane 63 holds the total);
// every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v += dpp_f<DPP_ROW_BCAST15, 0xA>(0.f, v);
  v += dpp_f<DPP_ROW_BCAST31, 0xC>(0.f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<DPP_QUAD_1032>(v, v));
  v = fmaxf(v, dpp_f<DPP_QUAD_2301>(v, v));
  v = fmaxf(v, dpp_f<DPP_ROW_ROR4>(v, v));
  v = fmaxf(v, dpp_f<DPP_ROW_ROR8>(v, v));
  v = fmaxf(v, dpp_f<DPP_ROW_BCAST15, 0xA>(v, v));
  v = fmaxf(v, dpp_f<DPP_ROW_BCAST31, 0xC>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
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

// A staging source loaded as Src::kParts raw float4 (Src::part) and summed
// (Src::sum) after every load of the stage is issued; kParts == 0: the
// source's operator() yields the value directly.
template <class Src>
struct SrcRaw {
  f4 p[Src::kParts > 0 ? Src::kParts : 1];
};
// Parts [0, Src::kEarly) are final before the grid barrier that precedes
// the stage and may be loaded ahead of it (src_load_early); the rest after
// it (src_load_late).
template <class Src>
__device__ __forceinline__ void src_load_early(const Src& s, int e, SrcRaw<Src>& r) {
  if constexpr (Src::kParts > 0) {
#pragma unroll
    for (int k = 0; k < Src::kEarly; ++k) r.p[k] = s.part(k, e);
  }
}
template <class Src>
__device__ __forceinline__ void src_load_late(const Src& s, int e, SrcRaw<Src>& r) {
  if constexpr (Src::kParts > 0) {
#pragma unroll
    for (int k = Src::kEarly; k < Src::kParts; ++k) r.p[k] = s.part(k, e);
  } else {
    r.p[0] = s(e);
  }
}
template <class Src>
__device__ __forceinline__ f4 src_sum(const SrcRaw<Src>& r) {
  if constexpr (Src::kParts > 1)
    return Src::sum(r.p);
  else
    return r.p[0];
}
