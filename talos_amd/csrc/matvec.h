// matvec.h -- fused dequant-matvec cores for batch-1 decode (gfx950).
//
// Restates the arithmetic of the reference's CPU matvec (src/math/matmul.rs:
// 15-47 for F32, src/math/quant.rs:18-51 for the block formats, whose
// dequantize is src/gguf/dtype.rs:64-121) as a bandwidth-bound GEMV:
//
//  * one wavefront computes two output rows that share x; lane l consumes
//    chunks l, l+64, ... of both rows (one 128-bit load per row per chunk);
//  * x lives in LDS with a 16-B pad every 32 (or 64) floats so the strided
//    per-lane 128-bit reads are bank-conflict free;
//  * the quant offset (-8 for Q4_0, -128 for the xor-ed Q8_0 bytes, -32 for
//    Q6_K) is folded out through the sum of x over each 16-element group:
//    sum((q-o)x) = sum(qx) - o*sum(x), so each weight costs one byte->float
//    convert and one FMA;
//  * fp32 accumulation, one scale multiply per block, a fixed-order
//    butterfly across lanes at the end.  No MFMA: batch-1 is HBM-bound.
#pragma once
#include "device_common.h"
#include "layout.h"

// Per 32-element block of x staged as int8 planes: the plane scale s
// (x ~= s * (a + b/254 + c/254^2)) and the integer sums of the a, b and c
// planes over the block.
struct XBlk {
  float s;
  int sa, sb, sc;
};

// LDS index of x element e in layout L (0: pad 4 floats per 32; 1: per 64).
template <int L>
__device__ __forceinline__ int xidx(int e) {
  return L == 0 ? e + ((e >> 5) << 2) : e + ((e >> 6) << 2);
}
static inline __host__ __device__ int xlds_floats(int n, int L) {
  n = (n + 15) & ~15;
  return L == 0 ? n + (n >> 5) * 4 + 4 : n + (n >> 6) * 4 + 4;
}

__device__ __forceinline__ f4 lds4(const float* xs, int i) {
  return *reinterpret_cast<const f4*>(xs + i);
}

// 16 weight bytes, read once: non-temporal global load.
__device__ __forceinline__ u4 ldg4(const uint8_t* p) {
  return __builtin_nontemporal_load(gptr(reinterpret_cast<const u4*>(p)));
}

// ---- per-format block dots: the dot of one block's raw (unsigned) quants
// with x, minus the quant offset folded in through the x group sums.

// A masked word whose known-zero bits the compiler may not exploit: with
// them visible it folds mask + byte extract into v_bfe_u32 + cvt_f32_ubyte0
// (two ops per element) instead of one v_cvt_f32_ubyte{0..3} per element.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

__device__ __forceinline__ float q4_block_dot(u4 q, const f4* x, float xs8) {
  float s = 0.f;
  s = dot_ub4(opaque(q.x & 0x0F0F0F0Fu), x[0], s);
  s = dot_ub4(opaque(q.y & 0x0F0F0F0Fu), x[1], s);
  s = dot_ub4(opaque(q.z & 0x0F0F0F0Fu), x[2], s);
  s = dot_ub4(opaque(q.w & 0x0F0F0F0Fu), x[3], s);
  float t = 0.f;
  t = dot_ub4(opaque((q.x >> 4) & 0x0F0F0F0Fu), x[4], t);
  t = dot_ub4(opaque((q.y >> 4) & 0x0F0F0F0Fu), x[5], t);
  t = dot_ub4(opaque((q.z >> 4) & 0x0F0F0F0Fu), x[6], t);
  t = dot_ub4(opaque((q.w >> 4) & 0x0F0F0F0Fu), x[7], t);
  return (s + t) - xs8;
}

__device__ __forceinline__ float q8_block_dot(u4 q0, u4 q1, const f4* x, float xs128) {
  float s = 0.f, t = 0.f;
  s = dot_ub4(q0.x, x[0], s);
  t = dot_ub4(q0.y, x[1], t);
  s = dot_ub4(q0.z, x[2], s);
  t = dot_ub4(q0.w, x[3], t);
  s = dot_ub4(q1.x, x[4], s);
  t = dot_ub4(q1.y, x[5], t);
  s = dot_ub4(q1.z, x[6], s);
  t = dot_ub4(q1.w, x[7], t);
  return (s + t) - xs128;
}

// One quarter super-block of Q6_K: byte j of the three planes yields the four
// 6-bit quants of elements base+j, +32, +64, +96 (src/gguf/dtype.rs:106-115).
__device__ __forceinline__ float q6_chunk_dot(u4 a, u4 b, u4 h, uint32_t scw, const f4* x,
                                              const float* xsr) {
  float r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
  const uint32_t av[4] = {a.x, a.y, a.z, a.w};
  const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
  const uint32_t hv[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t q1 = (av[k] & 0x0F0F0F0Fu) | ((hv[k] & 0x03030303u) << 4);
    const uint32_t q2 = (bv[k] & 0x0F0F0F0Fu) | ((hv[k] & 0x0C0C0C0Cu) << 2);
    const uint32_t q3 = ((av[k] >> 4) & 0x0F0F0F0Fu) | (hv[k] & 0x30303030u);
    const uint32_t q4 = ((bv[k] >> 4) & 0x0F0F0F0Fu) | ((hv[k] & 0xC0C0C0C0u) >> 2);
    r0 = dot_ub4(opaque(q1), x[k], r0);
    r1 = dot_ub4(opaque(q2), x[4 + k], r1);
    r2 = dot_ub4(opaque(q3), x[8 + k], r2);
    r3 = dot_ub4(opaque(q4), x[12 + k], r3);
  }
  const float s0 = (float)(int8_t)(scw & 0xFF), s1 = (float)(int8_t)((scw >> 8) & 0xFF);
  const float s2 = (float)(int8_t)((scw >> 16) & 0xFF), s3 = (float)(int8_t)(scw >> 24);
  float t = s0 * (r0 - xsr[0]);
  t = __builtin_fmaf(s1, r1 - xsr[1], t);
  t = __builtin_fmaf(s2, r2 - xsr[2], t);
  t = __builtin_fmaf(s3, r3 - xsr[3], t);
  return t;
}

// Stage n floats of x into LDS (layouts flagged by need0/need1) plus the
// per-16 group sums, zero-padded up to a multiple of 16.  With `norm`, x is
// replaced by rmsnorm(x)*w as in src/math/ops.rs:5-12:
// x[i] * (1/sqrt(sum(x^2)/n + eps)) * w[i].  blockDim.x must be 256; x and w
// must be 16-byte aligned.  Ends with __syncthreads().
__device__ __forceinline__ f4 load_x4(const float* __restrict__ p, int e, int n) {
  if (e + 3 < n) return *reinterpret_cast<const f4*>(p + e);
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (e < n) v.x = p[e];
  if (e + 1 < n) v.y = p[e + 1];
  if (e + 2 < n) v.z = p[e + 2];
  return v;
}

__device__ __forceinline__ void stage_x(const float* __restrict__ x, int n, const float* __restrict__ w,
                                        float eps, bool norm, float* xs0, float* xs1, float* xsum,
                                        float* red, bool need0, bool need1) {
  const int tid = threadIdx.x;
  const int npad = (n + 15) & ~15;
  float scale = 1.f;
  if (norm) {
    float ss = 0.f;
    for (int i = tid * 4; i < npad; i += 256 * 4) {
      const f4 v = load_x4(x, i, n);
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum(ss, red, 4);
    scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
  // Every group of four consecutive threads holds one complete 16-element
  // group for the xsum shuffle.
  const int n4 = npad >> 2;
  const int iters = (n4 + 255) >> 8;
  for (int it = 0; it < iters; ++it) {
    const int e4 = it * 256 + tid;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (e4 < n4) {
      v = load_x4(x, e4 * 4, n);
      if (norm) {
        const f4 ww = load_x4(w, e4 * 4, n);
        v.x = v.x * scale * ww.x;
        v.y = v.y * scale * ww.y;
        v.z = v.z * scale * ww.z;
        v.w = v.w * scale * ww.w;
      }
      if (need0) *reinterpret_cast<f4*>(xs0 + xidx<0>(e4 * 4)) = v;
      if (need1) *reinterpret_cast<f4*>(xs1 + xidx<1>(e4 * 4)) = v;
    }
    float s = (v.x + v.y) + (v.z + v.w);
    s = quad_sum(s);
    if (e4 < n4 && (tid & 3) == 0) xsum[e4 >> 2] = s;
  }
  __syncthreads();
}

// stage_x with every load of x (and w) issued in one batch, B float4 per
// thread (n % 4 == 0, n <= B * 1024), and `after()` run right behind that
// batch: a wave's loads return in issue order, so weight loads issued there
// do not delay x.  Same operations in the same order as stage_x, so the
// same bits.
template <int B, class After>
__device__ __forceinline__ void stage_x_batch(const float* __restrict__ x, int n, const float* __restrict__ w,
                                              float eps, bool norm, float* xs0, float* xs1, float* xsum,
                                              float* red, bool need0, bool need1, After after) {
  const int tid = threadIdx.x;
  const int nr = n >> 2, n4 = ((n + 15) & ~15) >> 2;
  f4 v[B], wv[B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const int e4 = i * 256 + tid;
    v[i] = *reinterpret_cast<const f4*>(x + (size_t)(e4 < nr ? e4 : nr - 1) * 4);
  }
  if (norm) {
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int e4 = i * 256 + tid;
      wv[i] = *reinterpret_cast<const f4*>(w + (size_t)(e4 < nr ? e4 : nr - 1) * 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  after();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < B; ++i)
    if (i * 256 + tid >= nr) v[i] = f4{0.f, 0.f, 0.f, 0.f};
  float scale = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < B; ++i)
      if (i * 256 + tid < n4) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = block_sum(ss, red, 4);
    scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const int e4 = i * 256 + tid;
    if (i * 256 >= n4) break;  // uniform: no thread of this round holds a group
    f4 vv = v[i];
    if (e4 < n4) {
      if (norm) {
        const f4 ww = e4 < nr ? wv[i] : f4{0.f, 0.f, 0.f, 0.f};
        vv.x = vv.x * scale * ww.x;
        vv.y = vv.y * scale * ww.y;
        vv.z = vv.z * scale * ww.z;
        vv.w = vv.w * scale * ww.w;
      }
      if (need0) *reinterpret_cast<f4*>(xs0 + xidx<0>(e4 * 4)) = vv;
      if (need1) *reinterpret_cast<f4*>(xs1 + xidx<1>(e4 * 4)) = vv;
    }
    float s = (vv.x + vv.y) + (vv.z + vv.w);
    s = quad_sum(s);
    if (e4 < n4 && (tid & 3) == 0) xsum[e4 >> 2] = s;
  }
  __syncthreads();
}

// Stage x for a matvec kernel whose first weight loads `after()` issues:
// one batch of x loads ahead of them when n allows, else after them.
template <class After>
__device__ __forceinline__ void stage_x_then(const float* __restrict__ x, int n, const float* __restrict__ w,
                                             float eps, bool norm, float* xs0, float* xs1, float* xsum,
                                             float* red, bool need0, bool need1, After after) {
  const int n4 = ((n + 15) & ~15) >> 2;
  if (n & 3) {
    after();
    stage_x(x, n, w, eps, norm, xs0, xs1, xsum, red, need0, need1);
  } else if (n4 <= 256) {
    stage_x_batch<1>(x, n, w, eps, norm, xs0, xs1, xsum, red, need0, need1, after);
  } else if (n4 <= 512) {
    stage_x_batch<2>(x, n, w, eps, norm, xs0, xs1, xsum, red, need0, need1, after);
  } else if (n4 <= 1024) {
    stage_x_batch<4>(x, n, w, eps, norm, xs0, xs1, xsum, red, need0, need1, after);
  } else {
    after();
    stage_x(x, n, w, eps, norm, xs0, xs1, xsum, red, need0, need1);
  }
}
