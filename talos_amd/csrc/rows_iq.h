// rows_iq.h -- int8-plane x staging for the graph-path and standalone
// matvec kernels (k_qkv, k_rows, k_gateup of kernels.h): x (optionally
// rmsnorm(x)*w) staged as three int8 planes per 32-element block and the
// dot products on v_dot4 (mvstream.h's XI compute, the persistent kernel's
// layer engine) -- about a quarter of the vector-ALU work of dequantizing
// every Q4_0 / Q8_0 weight to f32, which otherwise costs as much time as the
// weight bytes take to arrive.  x is exact to f32 level in its planes
// (mfma.h).
#pragma once
#include "mega.h"

// XPlanes<NR>: NR rounds of 8 elements per thread of a 256-thread block, so
// n <= NR * 2048 (n % 32 == 0).
template <int NR>
struct XPlanes {
  XQ X;
  __device__ __forceinline__ XPlanes(float* smem, int n, int) : X(carve_xq(smem, n, 1, 4)) {}
  template <class After>
  __device__ __forceinline__ void stage(const float* x, int n, const float* w, float eps, bool norm,
                                        After after) const {
    Src1 src{x};
    stage_xq<NR, 256, true>(src, n, w, eps, norm, X, nullptr, 0, 0, after, [] {});
  }
  template <uint32_t FMT>
  __device__ __forceinline__ XI src() const {
    return XI{reinterpret_cast<const uint8_t*>(X.pl), X.bs, X.nb, 0};
  }
};

// Staging rounds for n columns (2: n <= 4096, 8: n <= 16384), or 0 when n is
// beyond the int8-plane staging (the f32 staging serves it).
static inline int rows_iq_rounds(size_t n) {
  if (n % 32) return 0;
  if (n <= 2 * 2048) return 2;
  if (n <= 8 * 2048) return 8;
  return 0;
}

static inline size_t rows_iq_lds_bytes(size_t n) { return xq_lds_bytes((int)n, 1, 4); }
