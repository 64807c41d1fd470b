// rows_iq.h -- the standalone Q4_0 / Q8_0 matvec (quant::matvec,
// src/math/quant.rs) with x staged as int8 planes and the dot products on
// v_dot4 (mvstream.h's XI compute, the persistent kernel's layer matvec):
// about a quarter of the vector-ALU work of dequantizing every weight to f32,
// which otherwise costs as much time as a 4096 x 4096 matrix takes to
// arrive.  x is exact to f32 level in its three planes (mfma.h).
#pragma once
#include "mega.h"

// NR rounds of 8 elements per thread of the 256-thread block stage x, so
// cols <= NR * 2048.
template <uint32_t FMT, int R, int U, int NR>
__global__ __launch_bounds__(256) void k_rows_iq(RowParams P) {
  extern __shared__ float smem[];
  const XQ X = carve_xq(smem, P.n, 1, 4);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t ubase = (blockIdx.x * 4 + wave) * P.upw;
  const int nunits = ubase >= P.units ? 0 : (int)min(P.upw, P.units - ubase);
  auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
    A0 = P.m;
    A1 = P.m;
    r0 = (ubase + k) * R;
    rmax = P.m.rows;
  };
  auto stage = [&](auto&& pf) {  // x loads, then the first weight loads, then the planes
    Src1 src{P.x};
    stage_xq<NR, 256, true>(src, (int)P.n, P.norm_w, P.eps, P.norm_w != nullptr, X, nullptr, 0, 0, pf, [] {});
  };
  auto epi = [&](int k, const float(&y)[R]) {
    const uint32_t r0 = (ubase + k) * R;
    if (lane != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r0 + r < P.m.rows) {
        if (P.accumulate) P.out[r0 + r] += y[r];
        else P.out[r0 + r] = y[r];
      }
    }
  };
  mv_stream<FMT, R, U, false>(nunits, unit, [] {}, stage, epi,
                              XI{reinterpret_cast<const uint8_t*>(X.pl), X.bs, X.nb, 0}, lane, true);
}

// Smallest staging round count for n columns, or 0 when n is beyond the
// int8-plane kernel (then the f32 kernel serves it).
static inline int rows_iq_rounds(size_t n) {
  if (n % 32) return 0;
  for (int nr = 1; nr <= 8; nr *= 2)
    if (n <= (size_t)nr * 2048) return nr;
  return 0;
}

static inline size_t rows_iq_lds_bytes(size_t n) { return xq_lds_bytes((int)n, 1, 4); }
