// mvstream.h -- double-buffered weight streaming for the decode matvecs.
//
// A wave owns a run of "units" (R output rows of one matrix, or R/2 row pairs
// of two matrices for gate/up) and walks each unit's columns in "items" of
// U chunks per lane.  While it computes item i, the loads of item i+1 are in
// flight; the first item's loads can be issued before the block waits for
// its input and stages x into LDS, so the HBM latency of the weights
// overlaps the grid barrier and the rmsnorm/x setup.
// Weights are read once with 128-bit non-temporal loads; x comes from LDS and
// is shared by the R rows of an item.
#pragma once
#include "matvec.h"

// Rows per unit for each format (register budget: Q8_0 and Q6_K carry 2-3
// 128-bit words per chunk, so they take two rows).
static inline __host__ __device__ constexpr int mv_rows(uint32_t fmt) {
  return (fmt == TALOS_FMT_Q8_0 || fmt == TALOS_FMT_Q6_K) ? 2 : 4;
}
// Chunk-steps per item: up to 4, fewer for short rows.
static inline __host__ __device__ int mv_u(uint32_t nchunk) {
  const uint32_t steps = (nchunk + 63) / 64;
  return steps >= 4 ? 4 : (steps >= 2 ? 2 : 1);
}

template <uint32_t FMT>
struct MvT {
  static constexpr int QW = FMT == TALOS_FMT_Q8_0 ? 2 : FMT == TALOS_FMT_Q6_K ? 3 : 1;  // u4 per chunk
  static constexpr int L = FMT == TALOS_FMT_Q6_K ? 1 : 0;                                // x layout
};

template <uint32_t FMT, int R, int U>
struct MvBuf {
  u4 q[R][U][MvT<FMT>::QW];
  uint32_t a[R][U];  // Q4_0/Q8_0: f16 scale bits; Q6_K: packed sub-scales
  uint32_t b[R][U];  // Q6_K: f16 super-scale bits
};

// Load one item: rows r0 + slot (clamped to rmax - 1; the caller masks
// those results), chunks c0 + u*64 + lane (clamped to nchunk - 1, masked in
// mv_compute).  PAIR interleaves two matrices: slot 2k -> A0 row r0+k,
// slot 2k+1 -> A1 row r0+k.  Q4_0/Q8_0 rows are cols / 32 chunks apart, so
// a view of a column range (q and d advanced to its first chunk, nchunk
// its length) reads like a whole matrix.
template <uint32_t FMT, int R, int U, bool PAIR>
__device__ __forceinline__ void mv_load(MvBuf<FMT, R, U>& B, const DevMat& A0, const DevMat& A1, uint32_t r0,
                                        uint32_t rmax, int c0, int lane) {
  const int nc = (int)A0.nchunk;
  const int rs = (FMT == TALOS_FMT_Q4_0 || FMT == TALOS_FMT_Q8_0) ? (int)(A0.cols >> 5) : nc;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const DevMat& M = (PAIR && (i & 1)) ? A1 : A0;
    uint32_t row = PAIR ? r0 + i / 2 : r0 + i;
    row = row < rmax ? row : rmax - 1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = c0 + u * TALOS_WAVE + lane;
      c = c < nc ? c : nc - 1;
      const size_t ci = (size_t)row * rs + c;
      if (FMT == TALOS_FMT_F32) {
        B.q[i][u][0] = ldg4(M.q + ci * 16);
      } else if (FMT == TALOS_FMT_Q4_0) {
        B.q[i][u][0] = ldg4(M.q + ci * 16);
        B.a[i][u] = gld(M.d + ci);
      } else if (FMT == TALOS_FMT_Q8_0) {
        B.q[i][u][0] = ldg4(M.q + ci * 32);
        B.q[i][u][MvT<FMT>::QW - 1] = ldg4(M.q + ci * 32 + 16);
        B.a[i][u] = gld(M.d + ci);
      } else {
        const uint8_t* p = M.q + (size_t)row * nc * 48 + (size_t)c * 16;
        B.q[i][u][0] = ldg4(p);
        B.q[i][u][MvT<FMT>::QW > 1 ? 1 : 0] = ldg4(p + (size_t)nc * 16);
        B.q[i][u][MvT<FMT>::QW - 1] = ldg4(p + (size_t)nc * 32);
        B.a[i][u] = gld(M.sc + ci);
        B.b[i][u] = gld(M.d + (size_t)row * (nc >> 2) + (c >> 2));
      }
    }
  }
}

// The staged x a matvec reads: f32 values (XF: xs in the xidx layout of
// the format, xsum per 16 elements), or int8 planes (XI, Q4_0/Q8_0 only:
// the [3][2][nb] 16-byte words and the XBlk per 32-element block of
// stage_xq with SPLIT).
struct XF {
  const float* xs;
  const float* xsum;
};
struct XI {
  const uint8_t* pl;
  const XBlk* bs;
  int nb;
  int c0;  // chunk c of the matvec reads block c0 + c of x
};

// acc[i] += <row slot i, x> over this item's chunks.
template <uint32_t FMT, int R, int U>
__device__ __forceinline__ void mv_compute(const MvBuf<FMT, R, U>& B, const XF& X, int nc, int c0, int lane,
                                           float (&acc)[R]) {
  const float* xs = X.xs;
  const float* xsum = X.xsum;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = c0 + u * TALOS_WAVE + lane;
    const bool ok = c < nc;
    const int cc = ok ? c : nc - 1;
    if (FMT == TALOS_FMT_F32) {
      f4 x = lds4(xs, xidx<0>(cc * 4));
      if (!ok) x = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const f4 w = __builtin_bit_cast(f4, B.q[i][u][0]);
        float a = acc[i];
        a = __builtin_fmaf(w.x, x.x, a);
        a = __builtin_fmaf(w.y, x.y, a);
        a = __builtin_fmaf(w.z, x.z, a);
        a = __builtin_fmaf(w.w, x.w, a);
        acc[i] = a;
      }
    } else if (FMT == TALOS_FMT_Q4_0 || FMT == TALOS_FMT_Q8_0) {
      f4 x[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = lds4(xs, xidx<0>(cc * 32 + k * 4));
      const float xsb = xsum[2 * cc] + xsum[2 * cc + 1];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float d = ok ? f16_to_f32((uint16_t)B.a[i][u]) : 0.f;
        const float p = FMT == TALOS_FMT_Q4_0
                            ? q4_block_dot(B.q[i][u][0], x, 8.f * xsb)
                            : q8_block_dot(B.q[i][u][0], B.q[i][u][MvT<FMT>::QW - 1], x, 128.f * xsb);
        acc[i] = __builtin_fmaf(d, p, acc[i]);
      }
    } else {
      const int base = (cc >> 2) * 256 + ((cc >> 1) & 1) * 128 + (cc & 1) * 16;
      f4 x[16];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int k = 0; k < 4; ++k) x[r * 4 + k] = lds4(xs, xidx<1>(base + r * 32 + k * 4));
      float xsr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) xsr[r] = 32.f * xsum[(base + r * 32) >> 4];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float d = ok ? f16_to_f32((uint16_t)B.b[i][u]) : 0.f;
        const float p = q6_chunk_dot(B.q[i][u][0], B.q[i][u][MvT<FMT>::QW > 1 ? 1 : 0],
                                     B.q[i][u][MvT<FMT>::QW - 1], B.a[i][u], x, xsr);
        acc[i] = __builtin_fmaf(d, p, acc[i]);
      }
    }
  }
}

// acc[i] += <row slot i, x> with x as three int8 planes:
// x_e = s_b * (a_e + b_e/254 + c_e/254^2) for the elements e of block b
// (error <= 2^-24 * max|x_b|, f32-level).  The piece dots with the signed
// quants w (Q4_0: nibble - 8, src/gguf/dtype.rs:83-90; Q8_0: the byte) are
// exact integers: v_dot4_i32_i8 of the raw nibbles 0..15 (or Q8_0 bytes)
// against a plane, its chain started at -8 * (plane sum over the block) for
// Q4_0, so A = sum(w a), B = sum(w b), C = sum(w c) come out offset-free.
// 254 A + B is formed in the B chain's start (|A| < 2^16, v_mad_i32_i24),
// so a block costs three dot4 chains and one float combine:
//   acc += d * (s/254) * ((254 A + B) + C/254).
__device__ __forceinline__ int dot4_i8(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// One lane's x for one chunk-step: the chunk's three planes, s/254 (0 for a
// chunk past the row end, which then adds nothing) and the chain starts.
struct XIr {
  u4 pw[3][2];
  float s254;
  int ia, ib, ic;
};

template <uint32_t FMT>
__device__ __forceinline__ XIr xi_fetch(const XI& X, int cc, bool ok) {
  XIr r;
  cc += X.c0;
  const size_t plane = (size_t)X.nb * 32;
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r.pw[p][h] = *reinterpret_cast<const u4*>(X.pl + p * plane + ((size_t)h * X.nb + cc) * 16);
  const XBlk sx = X.bs[cc];
  r.s254 = ok ? sx.s * (1.0f / 254.0f) : 0.f;
  constexpr int off = FMT == TALOS_FMT_Q4_0 ? -8 : 0;
  r.ia = off * sx.sa;
  r.ib = off * sx.sb;
  r.ic = off * sx.sc;
  return r;
}

// acc[i] += row slot i of chunk-step u against x.  Per row two chains (the
// a-then-b chain and the c chain), interleaved over the R rows.
template <uint32_t FMT, int R, int U>
__device__ __forceinline__ void xi_dot(const MvBuf<FMT, R, U>& B, int u, const XIr& x, float (&acc)[R]) {
  static_assert(FMT == TALOS_FMT_Q4_0 || FMT == TALOS_FMT_Q8_0, "int8-plane x is for Q4_0 / Q8_0");
  constexpr float k254 = 1.0f / 254.0f;
  uint32_t w[R][8];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (FMT == TALOS_FMT_Q4_0) {
      const u4 q = B.q[i][u][0];
      w[i][0] = q.x & 0x0F0F0F0Fu;
      w[i][1] = q.y & 0x0F0F0F0Fu;
      w[i][2] = q.z & 0x0F0F0F0Fu;
      w[i][3] = q.w & 0x0F0F0F0Fu;
      w[i][4] = (q.x >> 4) & 0x0F0F0F0Fu;
      w[i][5] = (q.y >> 4) & 0x0F0F0F0Fu;
      w[i][6] = (q.z >> 4) & 0x0F0F0F0Fu;
      w[i][7] = (q.w >> 4) & 0x0F0F0F0Fu;
    } else {  // the device layout keeps Q8_0 quants biased by 128 (q ^ 0x80)
      const u4 q0 = B.q[i][u][0], q1 = B.q[i][u][MvT<FMT>::QW - 1];
      w[i][0] = q0.x ^ 0x80808080u;
      w[i][1] = q0.y ^ 0x80808080u;
      w[i][2] = q0.z ^ 0x80808080u;
      w[i][3] = q0.w ^ 0x80808080u;
      w[i][4] = q1.x ^ 0x80808080u;
      w[i][5] = q1.y ^ 0x80808080u;
      w[i][6] = q1.z ^ 0x80808080u;
      w[i][7] = q1.w ^ 0x80808080u;
    }
  }
  // plane word k of the lane's chunk: element order of the quants above
  auto xw = [&](int p, int k) {
    const u4& v = x.pw[p][k >> 2];
    return (k & 3) == 0 ? v.x : (k & 3) == 1 ? v.y : (k & 3) == 2 ? v.z : v.w;
  };
  int ab[R], c[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    ab[i] = x.ia;
    c[i] = x.ic;
  }
  // the c chain runs half beside the a chain, half beside the b chain
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      ab[i] = dot4_i8(w[i][k], xw(0, k), ab[i]);
      if (k < 4) c[i] = dot4_i8(w[i][k], xw(2, k), c[i]);
    }
  // |A| <= 32 * 128 * 127 < 2^23: a 24-bit multiply-add starts the b chain
#pragma unroll
  for (int i = 0; i < R; ++i) ab[i] = __mul24(ab[i], 254) + x.ib;
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      ab[i] = dot4_i8(w[i][k], xw(1, k), ab[i]);
      if (k >= 4) c[i] = dot4_i8(w[i][k], xw(2, k), c[i]);
    }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const float t = __builtin_fmaf((float)c[i], k254, (float)ab[i]);
    const float d = f16_to_f32((uint16_t)B.a[i][u]);
    acc[i] = __builtin_fmaf(d, x.s254 * t, acc[i]);
  }
}

// x from LDS, the next chunk-step's planes read while this one computes.
template <uint32_t FMT, int R, int U>
__device__ __forceinline__ void mv_compute(const MvBuf<FMT, R, U>& B, const XI& X, int nc, int c0, int lane,
                                           float (&acc)[R]) {
  auto cc = [&](int u) {
    const int c = c0 + u * TALOS_WAVE + lane;
    return c < nc ? c : nc - 1;
  };
  auto ok = [&](int u) { return c0 + u * TALOS_WAVE + lane < nc; };
  XIr x = xi_fetch<FMT>(X, cc(0), ok(0));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    XIr xn;
    if (u + 1 < U) xn = xi_fetch<FMT>(X, cc(u + 1), ok(u + 1));
    xi_dot<FMT, R, U>(B, u, x, acc);
    if (u + 1 < U) x = xn;
  }
}

// x held in registers for the whole phase (rows that fit one item: every
// item covers the same chunks, so a lane's x never changes).
template <int U>
struct XIreg {
  XIr x[U];
};

template <uint32_t FMT, int R, int U>
__device__ __forceinline__ void mv_compute(const MvBuf<FMT, R, U>& B, const XIreg<U>& X, int, int, int,
                                           float (&acc)[R]) {
#pragma unroll
  for (int u = 0; u < U; ++u) xi_dot<FMT, R, U>(B, u, X.x[u], acc);
}

// Run this wave's units.  unit(k, &A0, &A1, &r0, &rmax) describes the k-th
// unit of the wave; epi(k, y) consumes the R row results (every lane holds
// them).  `arrive()` and `stage(pf)` are called once by every thread of the
// block; `stage` calls pf() once, at the point where the first item's weight
// loads should be issued.  Without `pre` they are issued after `stage`.
template <uint32_t FMT, int R, int U, bool PAIR, class UnitFn, class EpiFn, class XS>
__device__ __forceinline__ void mv_run(int nitems, int iters, int nc, UnitFn& unit, EpiFn& epi, const XS& xs, int lane,
                                       MvBuf<FMT, R, U>& b0, MvBuf<FMT, R, U>& b1, const DevMat& A0, const DevMat& A1,
                                       uint32_t r0, uint32_t rmax);

template <uint32_t FMT, int R, int U, bool PAIR, class UnitFn, class EpiFn, class XS>
__device__ __forceinline__ void mv_run3(int nitems, int iters, int nc, UnitFn& unit, EpiFn& epi, const XS& xs,
                                        int lane, MvBuf<FMT, R, U>& b0, MvBuf<FMT, R, U>& b1, DevMat N0, DevMat N1,
                                        uint32_t nr0, uint32_t nrmax);

// XREG (int8-plane x only): the caller guarantees a row fits one item
// (nchunk <= U * 64), so a lane's x is the same for every item and is read
// from LDS once, into registers.
// DEPTH: items in flight, 2 (compute item i while item i+1 loads) or 3
// (items i+1 and i+2 load while item i computes).
template <uint32_t FMT, int R, int U, bool PAIR, bool XREG = false, int DEPTH = 2, class UnitFn, class ArriveFn,
          class StageFn, class EpiFn, class XS>
__device__ __forceinline__ void mv_stream(int nunits, UnitFn unit, ArriveFn arrive, StageFn stage, EpiFn epi,
                                          const XS& xs, int lane, bool pre) {
  static_assert(DEPTH == 2 || DEPTH == 3, "two or three items in flight");
  // Every weight load below is issued unconditionally (an idle wave's first
  // load reads row 0, discarded): the compiler's wait counts then stay exact,
  // so computing item i waits only for item i's loads, never for item i+1's
  // (a load under a branch makes the merged count fall back to waiting for
  // everything).
  MvBuf<FMT, R, U> b0, b1;
  DevMat A0{}, A1{};
  uint32_t r0 = 0, rmax = 1;
  unit(0, A0, A1, r0, rmax);
  const int nc = (int)A0.nchunk;
  const int iters = (nc + U * TALOS_WAVE - 1) / (U * TALOS_WAVE);
  if (nunits <= 0) {
    r0 = 0;
    rmax = 1;
  }
  arrive();
  const int nitems = nunits > 0 ? nunits * iters : 0;
  auto pf = [&] { mv_load<FMT, R, U, PAIR>(b0, A0, A1, r0, rmax, 0, lane); };
  if (pre) {
    stage(pf);
  } else {
    stage([] {});
    pf();
  }
  // DEPTH 3: item 1 (item 0 again when there is no second item) goes into
  // b1 unconditionally, after the staging: issued with item 0 its loads
  // slow the staging's own reads of x more than they gain.
  DevMat N0 = A0, N1 = A1;
  uint32_t nr0 = r0, nrmax = rmax;
  if constexpr (DEPTH == 3) {
    const bool two = nitems > 1;
    if (two && iters == 1) unit(1, N0, N1, nr0, nrmax);
    mv_load<FMT, R, U, PAIR>(b1, N0, N1, nr0, nrmax, two && iters > 1 ? U * TALOS_WAVE : 0, lane);
  }
  if constexpr (XREG) {
    XIreg<U> xr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = u * TALOS_WAVE + lane;
      xr.x[u] = xi_fetch<FMT>(xs, c < nc ? c : nc - 1, c < nc);
    }
    if constexpr (DEPTH == 3)
      mv_run3<FMT, R, U, PAIR>(nitems, 1, nc, unit, epi, xr, lane, b0, b1, N0, N1, nr0, nrmax);
    else
      mv_run<FMT, R, U, PAIR>(nitems, 1, nc, unit, epi, xr, lane, b0, b1, A0, A1, r0, rmax);
  } else {
    if constexpr (DEPTH == 3)
      mv_run3<FMT, R, U, PAIR>(nitems, iters, nc, unit, epi, xs, lane, b0, b1, N0, N1, nr0, nrmax);
    else
      mv_run<FMT, R, U, PAIR>(nitems, iters, nc, unit, epi, xs, lane, b0, b1, A0, A1, r0, rmax);
  }
}

// The item loop with three items in flight: items 0 and 1 are already
// issued into b0 and b1 (N0/N1/nr0/nrmax describe item 1's unit); item i+2
// is issued before item i is computed.  Each tail is straight-line code, so
// every wait count stays exact.
template <uint32_t FMT, int R, int U, bool PAIR, class UnitFn, class EpiFn, class XS>
__device__ __forceinline__ void mv_run3(int nitems, int iters, int nc, UnitFn& unit, EpiFn& epi, const XS& xs,
                                        int lane, MvBuf<FMT, R, U>& b0, MvBuf<FMT, R, U>& b1, DevMat N0, DevMat N1,
                                        uint32_t nr0, uint32_t nrmax) {
  MvBuf<FMT, R, U> b2;
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.f;
  auto col = [&](int i) { return (i % iters) * U * TALOS_WAVE; };
  auto ld = [&](MvBuf<FMT, R, U>& b, int i) {  // items are issued in order, so the unit changes at i % iters == 0
    if (i % iters == 0) unit(i / iters, N0, N1, nr0, nrmax);
    mv_load<FMT, R, U, PAIR>(b, N0, N1, nr0, nrmax, col(i), lane);
  };
  auto step = [&](const MvBuf<FMT, R, U>& b, int i) {
    mv_compute<FMT, R, U>(b, xs, nc, col(i), lane, acc);
    if (i % iters == iters - 1) {
      float y[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        y[r] = wave_sum(acc[r]);
        acc[r] = 0.f;
      }
      epi(i / iters, y);
    }
  };
  int i = 0;
  for (; i + 4 < nitems; i += 3) {  // items i+2, i+3 and i+4 exist
    ld(b2, i + 2);
    step(b0, i);
    ld(b0, i + 3);
    step(b1, i + 1);
    ld(b1, i + 4);
    step(b2, i + 2);
  }
  const int left = nitems - i;  // 0..4; b0 = item i, b1 = item i+1 when they exist
  if (left == 4) {
    ld(b2, i + 2);
    step(b0, i);
    ld(b0, i + 3);
    step(b1, i + 1);
    step(b2, i + 2);
    step(b0, i + 3);
  } else if (left == 3) {
    ld(b2, i + 2);
    step(b0, i);
    step(b1, i + 1);
    step(b2, i + 2);
  } else if (left == 2) {
    step(b0, i);
    step(b1, i + 1);
  } else if (left == 1) {
    step(b0, i);
  }
}

// The item loop of mv_stream (item 0 already issued into b0).
template <uint32_t FMT, int R, int U, bool PAIR, class UnitFn, class EpiFn, class XS>
__device__ __forceinline__ void mv_run(int nitems, int iters, int nc, UnitFn& unit, EpiFn& epi, const XS& xs, int lane,
                                       MvBuf<FMT, R, U>& b0, MvBuf<FMT, R, U>& b1, const DevMat& A0, const DevMat& A1,
                                       uint32_t r0, uint32_t rmax) {
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.f;
  // item i -> (unit i / iters, chunk offset (i % iters) * U * 64)
  DevMat N0 = A0, N1 = A1;
  uint32_t nr0 = r0, nrmax = rmax;
  auto next_desc = [&](int i) {
    const int k = i / iters;
    if (i % iters == 0) unit(k, N0, N1, nr0, nrmax);
  };
  auto finish = [&](int i) {
    if (i % iters == iters - 1) {
      float y[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        y[r] = wave_sum(acc[r]);
        acc[r] = 0.f;
      }
      epi(i / iters, y);
    }
  };
  auto col = [&](int i) { return (i % iters) * U * TALOS_WAVE; };
  int i = 0;
  for (; i + 2 < nitems; i += 2) {  // items i+1 and i+2 exist
    next_desc(i + 1);
    mv_load<FMT, R, U, PAIR>(b1, N0, N1, nr0, nrmax, col(i + 1), lane);
    mv_compute<FMT, R, U>(b0, xs, nc, col(i), lane, acc);
    finish(i);
    next_desc(i + 2);
    mv_load<FMT, R, U, PAIR>(b0, N0, N1, nr0, nrmax, col(i + 2), lane);
    mv_compute<FMT, R, U>(b1, xs, nc, col(i + 1), lane, acc);
    finish(i + 1);
  }
  if (i + 1 < nitems) {  // two items left
    next_desc(i + 1);
    mv_load<FMT, R, U, PAIR>(b1, N0, N1, nr0, nrmax, col(i + 1), lane);
    mv_compute<FMT, R, U>(b0, xs, nc, col(i), lane, acc);
    finish(i);
    mv_compute<FMT, R, U>(b1, xs, nc, col(i + 1), lane, acc);
    finish(i + 1);
  } else if (i < nitems) {  // one item left
    mv_compute<FMT, R, U>(b0, xs, nc, col(i), lane, acc);
    finish(i);
  }
}
