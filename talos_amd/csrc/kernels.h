// kernels.h -- the per-token decode kernels.
//
// One token's forward (src/model/llama.rs:96-183 restated for the GPU) is
//   [embed] -> per layer { k_qkv, k_attn, k_resid(o), k_gateup, k_resid(down) }
//   -> k_out (final rmsnorm + output projection) [-> k_argmax]
// and is captured once into a hipGraph.  The position and token live in a
// device `state` block, so the same graph replays for every step.
#pragma once
#include "matvec.h"

// state[] slots
enum { ST_POS = 0, ST_TOKEN = 1, ST_ARGMAX = 2, ST_STEP = 3 };

#define TALOS_MAX_GROUP 8

// Dynamic LDS carve-up shared by the matvec kernels.
struct XStage {
  float* xs[2];
  float* xsum;
  float* red;
};

__device__ __forceinline__ XStage carve_x(float* smem, int n, int need) {
  XStage s;
  float* p = smem;
  s.xs[0] = p;
  if (need & 1) p += xlds_floats(n, 0);
  s.xs[1] = p;
  if (need & 2) p += xlds_floats(n, 1);
  s.xsum = p;
  p += (n + 15) / 16;
  s.red = p;
  return s;
}

static inline size_t stage_lds_bytes(int n, int need) {
  size_t f = 0;
  if (need & 1) f += xlds_floats(n, 0);
  if (need & 2) f += xlds_floats(n, 1);
  f += (n + 15) / 16 + 16;
  return f * 4;
}

// Chunks per lane per K-step: enough to keep ~4 loads in flight without
// issuing dead chunks on the short 4096-column rows.
template <uint32_t FMT, int U>
__device__ __forceinline__ void dot_rows_u(const DevMat& A, uint32_t ra, const DevMat& B, uint32_t rb,
                                           bool two, const float* xs, const float* xsum, int lane,
                                           float& ya, float& yb) {
  float accA = 0.f, accB = 0.f;
  const int nc = (int)A.nchunk;
  for (int c0 = 0; c0 < nc; c0 += U * TALOS_WAVE) {
    float pa[U], pb[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int c = c0 + i * TALOS_WAVE + lane;
      const int cc = c < nc ? c : nc - 1;
      pa[i] = 0.f;
      pb[i] = 0.f;
      if (FMT == TALOS_FMT_F32) chunk_f32(A, ra, B, rb, two, xs, cc, pa[i], pb[i]);
      else if (FMT == TALOS_FMT_Q4_0) chunk_q4_0(A, ra, B, rb, two, xs, xsum, cc, pa[i], pb[i]);
      else if (FMT == TALOS_FMT_Q8_0) chunk_q8_0(A, ra, B, rb, two, xs, xsum, cc, pa[i], pb[i]);
      else chunk_q6_k(A, ra, B, rb, two, xs, xsum, cc, pa[i], pb[i]);
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const bool ok = c0 + i * TALOS_WAVE + lane < nc;
      accA += ok ? pa[i] : 0.f;
      accB += ok ? pb[i] : 0.f;
    }
  }
  ya = wave_sum(accA);
  yb = two ? wave_sum(accB) : 0.f;
}

template <uint32_t FMT>
__device__ __forceinline__ void dot_rows_fmt(const DevMat& A, uint32_t ra, const DevMat& B, uint32_t rb,
                                             bool two, const float* xs, const float* xsum, int lane,
                                             float& ya, float& yb) {
  const int steps = ((int)A.nchunk + TALOS_WAVE - 1) / TALOS_WAVE;
  if (steps >= 4) dot_rows_u<FMT, 4>(A, ra, B, rb, two, xs, xsum, lane, ya, yb);
  else if (steps >= 2) dot_rows_u<FMT, 2>(A, ra, B, rb, two, xs, xsum, lane, ya, yb);
  else dot_rows_u<FMT, 1>(A, ra, B, rb, two, xs, xsum, lane, ya, yb);
}

__device__ __forceinline__ void dot2(const DevMat& A, uint32_t ra, const DevMat& B, uint32_t rb, bool two,
                                     const XStage& X, int lane, float& ya, float& yb) {
  switch (A.fmt) {
    case TALOS_FMT_F32: dot_rows_fmt<TALOS_FMT_F32>(A, ra, B, rb, two, X.xs[0], X.xsum, lane, ya, yb); break;
    case TALOS_FMT_Q4_0: dot_rows_fmt<TALOS_FMT_Q4_0>(A, ra, B, rb, two, X.xs[0], X.xsum, lane, ya, yb); break;
    case TALOS_FMT_Q8_0: dot_rows_fmt<TALOS_FMT_Q8_0>(A, ra, B, rb, two, X.xs[0], X.xsum, lane, ya, yb); break;
    default: dot_rows_fmt<TALOS_FMT_Q6_K>(A, ra, B, rb, two, X.xs[1], X.xsum, lane, ya, yb); break;
  }
}

__device__ __forceinline__ DevMat pick3(const DevMat& a, const DevMat& b, const DevMat& c, int s) {
  return s == 0 ? a : (s == 1 ? b : c);
}

// ---------------------------------------------------------------- k_qkv --
// rmsnorm(x, attn_norm) -> q/k/v rows -> RoPE(q, k) -> q buffer and the K/V
// cache row at `pos` (src/model/llama.rs:118-130, src/math/ops.rs:48-61).
struct QKVParams {
  DevMat m[3];
  uint32_t units[3];  // row pairs per matrix
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t n;
  float* q_out;
  float* kc;  // this layer's K cache [ctx][kv_dim]
  float* vc;
  uint32_t kv_dim, hd;
  const float* rope;  // [ctx][hd/2] (cos, sin)
  const int32_t* state;
  uint32_t upw;
  int need;
};

__global__ __launch_bounds__(256) void k_qkv(QKVParams P) {
  extern __shared__ float smem[];
  const XStage X = carve_x(smem, P.n, P.need);
  stage_x(P.x, P.n, P.norm_w, P.eps, true, X.xs[0], X.xs[1], X.xsum, X.red, P.need & 1, P.need & 2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t total = P.units[0] + P.units[1] + P.units[2];
  const int pos = P.state[ST_POS];
  const uint32_t half = P.hd / 2;
  for (uint32_t k = 0; k < P.upw; ++k) {
    const uint32_t u = (blockIdx.x * 4 + wave) * P.upw + k;
    if (u >= total) break;
    int s = 0;
    uint32_t p = u;
    if (p >= P.units[0]) {
      p -= P.units[0];
      s = 1;
      if (p >= P.units[1]) {
        p -= P.units[1];
        s = 2;
      }
    }
    const DevMat M = pick3(P.m[0], P.m[1], P.m[2], s);
    const uint32_t r0 = 2 * p;
    float y0, y1;
    dot2(M, r0, M, r0 + 1, true, X, lane, y0, y1);
    if (lane == 0) {
      if (s < 2) {
        const uint32_t i = (r0 % P.hd) / 2;
        const float c = P.rope[((size_t)pos * half + i) * 2 + 0];
        const float sn = P.rope[((size_t)pos * half + i) * 2 + 1];
        const float a = y0 * c - y1 * sn;
        const float b = y0 * sn + y1 * c;
        if (s == 0) {
          P.q_out[r0] = a;
          P.q_out[r0 + 1] = b;
        } else {
          P.kc[(size_t)pos * P.kv_dim + r0] = a;
          P.kc[(size_t)pos * P.kv_dim + r0 + 1] = b;
        }
      } else {
        P.vc[(size_t)pos * P.kv_dim + r0] = y0;
        P.vc[(size_t)pos * P.kv_dim + r0 + 1] = y1;
      }
    }
  }
}

// -------------------------------------------------------------- k_resid --
// resid[r] += <W row r, x> : the o-projection and down-projection with the
// residual add fused (src/model/llama.rs:157-161, 172-176).  Also the plain
// store used by the standalone matvec and the output projection (k_out).
struct RowParams {
  DevMat m;
  const float* x;
  const float* norm_w;  // non-null: stage rmsnorm(x)*w (final norm)
  float eps;
  uint32_t n;
  float* out;
  int accumulate;  // 1: out[r] += y, 0: out[r] = y
  uint32_t units;  // row pairs
  uint32_t upw;
  int need;
};

__global__ __launch_bounds__(256) void k_rows(RowParams P) {
  extern __shared__ float smem[];
  const XStage X = carve_x(smem, P.n, P.need);
  stage_x(P.x, P.n, P.norm_w, P.eps, P.norm_w != nullptr, X.xs[0], X.xs[1], X.xsum, X.red, P.need & 1,
          P.need & 2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (uint32_t k = 0; k < P.upw; ++k) {
    const uint32_t u = (blockIdx.x * 4 + wave) * P.upw + k;
    if (u >= P.units) break;
    const uint32_t r0 = 2 * u;
    const bool two = r0 + 1 < P.m.rows;
    float y0, y1;
    dot2(P.m, r0, P.m, two ? r0 + 1 : r0, two, X, lane, y0, y1);
    if (lane == 0) {
      if (P.accumulate) {
        P.out[r0] += y0;
        if (two) P.out[r0 + 1] += y1;
      } else {
        P.out[r0] = y0;
        if (two) P.out[r0 + 1] = y1;
      }
    }
  }
}

// ------------------------------------------------------------- k_gateup --
// rmsnorm(x, ffn_norm) -> gate row p and up row p -> silu(g)*u
// (src/model/llama.rs:164-171, src/math/ops.rs:28-37).
struct GateUpParams {
  DevMat g, u;
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t n;
  float* h;
  uint32_t units;  // n_ff
  uint32_t upw;
  int need;
};

__global__ __launch_bounds__(256) void k_gateup(GateUpParams P) {
  extern __shared__ float smem[];
  const XStage X = carve_x(smem, P.n, P.need);
  stage_x(P.x, P.n, P.norm_w, P.eps, true, X.xs[0], X.xs[1], X.xsum, X.red, P.need & 1, P.need & 2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool same = P.g.fmt == P.u.fmt;
  for (uint32_t k = 0; k < P.upw; ++k) {
    const uint32_t p = (blockIdx.x * 4 + wave) * P.upw + k;
    if (p >= P.units) break;
    float yg, yu, dummy;
    if (same) {
      dot2(P.g, p, P.u, p, true, X, lane, yg, yu);
    } else {
      dot2(P.g, p, P.g, p, false, X, lane, yg, dummy);
      dot2(P.u, p, P.u, p, false, X, lane, yu, dummy);
    }
    if (lane == 0) P.h[p] = (yg / (1.0f + expf(-yg))) * yu;
  }
}

// ---------------------------------------------------------------- k_attn --
// GQA decode attention for one KV head and one slice of positions
// (src/model/llama.rs:135-155): scores = <q_h, K_t> * scale, softmax,
// o = sum_t p_t V_t, with an online (max-shifted) softmax per slice.  Slices
// are combined by the last block to finish for that KV head, in slice
// order, so results do not depend on block timing.
struct AttnParams {
  const float* q;
  const float* kc;
  const float* vc;
  float* out;       // [n_head * hd]
  float* part;      // [n_kv][nsplit][group][hd + 2]
  uint32_t* count;  // [n_kv], self-resetting
  const int32_t* state;
  uint32_t hd, kv_dim, group, nsplit, max_chunk;
  float scale;
};

static inline size_t attn_lds_bytes(uint32_t hd, uint32_t group, uint32_t max_chunk) {
  const uint32_t ns = 256 / hd;
  return (size_t)(group * max_chunk + ns * group * hd + group * hd + 64) * 4;
}

template <int DPL>
__global__ __launch_bounds__(256) void k_attn(AttnParams P) {
  extern __shared__ float smem[];
  const uint32_t hd = P.hd, group = P.group;
  const uint32_t ns = 256 / hd;
  float* sc = smem;                          // [group][max_chunk]
  float* ored = sc + group * P.max_chunk;    // [ns][group][hd]
  float* qs = ored + ns * group * hd;        // [group][hd]
  float* red = qs + group * hd;              // 64 floats
  __shared__ float mh[TALOS_MAX_GROUP], lh[TALOS_MAX_GROUP];
  __shared__ int am_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t j = blockIdx.x, split = blockIdx.y;
  const int seq = P.state[ST_POS] + 1;
  const int chunk = (seq + (int)P.nsplit - 1) / (int)P.nsplit;
  const int t0 = (int)split * chunk;
  const int t1 = min(seq, t0 + chunk);
  const int len = max(0, t1 - t0);

  for (uint32_t i = tid; i < group * hd; i += 256) qs[i] = P.q[(size_t)j * group * hd + i];
  __syncthreads();

  // scores: 16 lanes per position, DPL dims per lane, reduced over the 16
  const int dl = lane & 15;
  float qr[TALOS_MAX_GROUP][DPL];
#pragma unroll
  for (int h = 0; h < TALOS_MAX_GROUP; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) qr[h][i] = h < (int)group ? qs[h * hd + dl * DPL + i] : 0.f;
  for (int b = 0; b < len; b += 16) {
    const int tl = b + wave * 4 + (lane >> 4);
    const bool ok = tl < len;
    const float* kp = P.kc + (size_t)(t0 + (ok ? tl : 0)) * P.kv_dim + j * hd + dl * DPL;
    float kv[DPL];
    if constexpr (DPL % 4 == 0) {
#pragma unroll
      for (int i = 0; i < DPL; i += 4) {
        const f4 v = *reinterpret_cast<const f4*>(kp + i);
        kv[i] = v.x;
        kv[i + 1] = v.y;
        kv[i + 2] = v.z;
        kv[i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < DPL; ++i) kv[i] = kp[i];
    }
#pragma unroll
    for (int h = 0; h < TALOS_MAX_GROUP; ++h) {
      if (h < (int)group) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) d = __builtin_fmaf(qr[h][i], kv[i], d);
        d += __shfl_xor(d, 1, TALOS_WAVE);
        d += __shfl_xor(d, 2, TALOS_WAVE);
        d += __shfl_xor(d, 4, TALOS_WAVE);
        d += __shfl_xor(d, 8, TALOS_WAVE);
        if (ok && dl == 0) sc[h * P.max_chunk + tl] = d * P.scale;
      }
    }
  }
  __syncthreads();

  // softmax statistics per head over this slice; sc becomes exp(s - m)
  for (uint32_t h = 0; h < group; ++h) {
    float m = -INFINITY;
    for (int t = tid; t < len; t += 256) m = fmaxf(m, sc[h * P.max_chunk + t]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (int t = tid; t < len; t += 256) {
      const float e = expf(sc[h * P.max_chunk + t] - m);
      sc[h * P.max_chunk + t] = e;
      l += e;
    }
    l = block_sum(l, red, 4);
    if (tid == 0) {
      mh[h] = m;
      lh[h] = l;
    }
  }
  __syncthreads();

  // o[h][d] = sum_t p[h][t] V_t[d]; ns position subsets per dim
  const int d = tid % hd, sub = tid / hd;
  if (sub < (int)ns) {
    float acc[TALOS_MAX_GROUP];
#pragma unroll
    for (int h = 0; h < TALOS_MAX_GROUP; ++h) acc[h] = 0.f;
    for (int t = sub; t < len; t += ns) {
      const float v = P.vc[(size_t)(t0 + t) * P.kv_dim + j * hd + d];
#pragma unroll
      for (int h = 0; h < TALOS_MAX_GROUP; ++h)
        if (h < (int)group) acc[h] = __builtin_fmaf(sc[h * P.max_chunk + t], v, acc[h]);
    }
#pragma unroll
    for (int h = 0; h < TALOS_MAX_GROUP; ++h)
      if (h < (int)group) ored[(sub * group + h) * hd + d] = acc[h];
  }
  __syncthreads();

  if (P.nsplit == 1) {
    for (uint32_t i = tid; i < group * hd; i += 256) {
      const uint32_t h = i / hd, dd = i % hd;
      float o = 0.f;
      for (uint32_t s = 0; s < ns; ++s) o += ored[(s * group + h) * hd + dd];
      P.out[((size_t)j * group + h) * hd + dd] = o / lh[h];
    }
    return;
  }

  const size_t pstride = hd + 2;
  float* mypart = P.part + ((size_t)j * P.nsplit + split) * group * pstride;
  for (uint32_t i = tid; i < group * hd; i += 256) {
    const uint32_t h = i / hd, dd = i % hd;
    float o = 0.f;
    for (uint32_t s = 0; s < ns; ++s) o += ored[(s * group + h) * hd + dd];
    mypart[h * pstride + dd] = o;
  }
  if (tid < (int)group) {
    mypart[tid * pstride + hd] = len > 0 ? mh[tid] : -INFINITY;
    mypart[tid * pstride + hd + 1] = len > 0 ? lh[tid] : 0.f;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = atomicAdd(&P.count[j], 1u);
    am_last = old == P.nsplit - 1;
  }
  __syncthreads();
  if (!am_last) return;
  __threadfence();
  const float* parts = P.part + (size_t)j * P.nsplit * group * pstride;
  for (uint32_t i = tid; i < group * hd; i += 256) {
    const uint32_t h = i / hd, dd = i % hd;
    float M = -INFINITY;
    for (uint32_t s = 0; s < P.nsplit; ++s) M = fmaxf(M, parts[(s * group + h) * pstride + hd]);
    float L = 0.f, O = 0.f;
    for (uint32_t s = 0; s < P.nsplit; ++s) {
      const float* ps = parts + (s * group + h) * pstride;
      const float w = ps[hd + 1] > 0.f ? expf(ps[hd] - M) : 0.f;
      L = __builtin_fmaf(ps[hd + 1], w, L);
      O = __builtin_fmaf(ps[dd], w, O);
    }
    P.out[((size_t)j * group + h) * hd + dd] = O / L;
  }
  if (tid == 0) atomicExch(&P.count[j], 0u);
}

// --------------------------------------------------------------- k_embed --
// x = dequant_row(token_embd, token) (src/model/weights.rs:58-62,
// src/gguf/dtype.rs:64-121), on the device, from the repacked layout.
__device__ __forceinline__ float dq_elem(const DevMat& M, uint32_t r, uint32_t e) {
  switch (M.fmt) {
    case TALOS_FMT_F32:
      return reinterpret_cast<const float*>(M.q)[(size_t)r * M.nchunk * 4 + e];
    case TALOS_FMT_Q8_0: {
      const size_t b = (size_t)r * M.nchunk + e / 32;
      const float dd = f16_to_f32(M.d[b]);
      return dd * (float)(int8_t)(M.q[b * 32 + (e & 31)] ^ 0x80);
    }
    case TALOS_FMT_Q4_0: {
      const size_t b = (size_t)r * M.nchunk + e / 32;
      const float dd = f16_to_f32(M.d[b]);
      const uint32_t j = e & 31;
      const uint8_t by = M.q[b * 16 + (j & 15)];
      const int v = (int)(j < 16 ? (by & 0x0F) : (by >> 4)) - 8;
      return dd * (float)v;
    }
    default: {  // Q6_K
      const uint32_t sb = e / 256, w = e % 256, n = w / 128, l = w % 32, quarter = (w % 128) / 32;
      const uint32_t g = l / 16, jj = l % 16;
      const uint32_t c = sb * 4 + n * 2 + g;
      const size_t nc = M.nchunk;
      const uint8_t* base = M.q + (size_t)r * nc * 48 + (size_t)c * 16 + jj;
      const uint8_t a = base[0], bq = base[nc * 16], hq = base[nc * 32];
      uint32_t q;
      if (quarter == 0) q = (a & 0xF) | ((hq & 3) << 4);
      else if (quarter == 1) q = (bq & 0xF) | (((hq >> 2) & 3) << 4);
      else if (quarter == 2) q = (a >> 4) | (((hq >> 4) & 3) << 4);
      else q = (bq >> 4) | (((hq >> 6) & 3) << 4);
      const int8_t s = (int8_t)((M.sc[(size_t)r * nc + c] >> (8 * quarter)) & 0xFF);
      const float dd = f16_to_f32(M.d[(size_t)r * (nc / 4) + sb]);
      return dd * (float)s * (float)((int)q - 32);
    }
  }
}

__global__ __launch_bounds__(256) void k_embed(DevMat M, const int32_t* state, float* x) {
  const uint32_t tok = (uint32_t)state[ST_TOKEN];
  for (uint32_t e = threadIdx.x; e < M.cols; e += 256) x[e] = dq_elem(M, tok, e);
}

// --------------------------------------------------------------- k_norm --
// hidden = rmsnorm(x, output_norm) (src/model/llama.rs:180-181).
__global__ __launch_bounds__(256) void k_norm(const float* x, const float* w, float eps, uint32_t n, float* out) {
  __shared__ float red[8];
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss += x[i] * x[i];
  ss = block_sum(ss, red, 4);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += 256) out[i] = x[i] * scale * w[i];
}

// ------------------------------------------------------------- k_argmax --
// argmax by total_cmp, ties to the last index (src/sample.rs:7-14).  With
// `advance`, the result becomes the next step's token, the position moves
// on, and the token is appended to `tokens` -- the greedy decode loop runs
// without host round trips.
__global__ __launch_bounds__(1024) void k_argmax(const float* logits, uint32_t n, int32_t* state,
                                                 int32_t* tokens, int advance) {
  __shared__ int32_t sk[16];
  __shared__ int32_t si[16];
  int32_t bk = INT32_MIN, bi = -1;
  for (uint32_t i = threadIdx.x; i < n; i += 1024) {
    const int32_t k = total_key(logits[i]);
    if (k > bk || (k == bk && (int32_t)i > bi)) {
      bk = k;
      bi = (int32_t)i;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int32_t ok = __shfl_xor(bk, off, TALOS_WAVE);
    const int32_t oi = __shfl_xor(bi, off, TALOS_WAVE);
    if (ok > bk || (ok == bk && oi > bi)) {
      bk = ok;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (sk[w] > bk || (sk[w] == bk && si[w] > bi)) {
        bk = sk[w];
        bi = si[w];
      }
    state[ST_ARGMAX] = bi;
    if (advance) {
      const int32_t step = state[ST_STEP];
      tokens[step] = bi;
      state[ST_TOKEN] = bi;
      state[ST_POS] = state[ST_POS] + 1;
      state[ST_STEP] = step + 1;
    }
  }
}
