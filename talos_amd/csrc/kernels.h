// kernels.h -- the per-token decode kernels.
//
// One token's forward (src/model/llama.rs:96-183 restated for the GPU) is
//   [embed] -> per layer { k_qkv, k_attn, k_resid(o), k_gateup, k_resid(down) }
//   -> k_out (final rmsnorm + output projection) [-> k_argmax]
// and is captured once into a hipGraph.  The position and token live in a
// device `state` block, so the same graph replays for every step.
#pragma once
#include "mvstream.h"

// state[] slots
// ST_NFEED: tokens in tokens[] that a feed (prompt) run consumes in order.
enum { ST_POS = 0, ST_TOKEN = 1, ST_ARGMAX = 2, ST_STEP = 3, ST_NFEED = 4 };

// Advance the device token state after a step whose argmax is `am`.
// mode 2 (greedy): the argmax is the next input and is appended to tokens[].
// mode 3 (feed): the next input is tokens[step + 1] while the feed lasts.
__device__ __forceinline__ void advance_state(int32_t* state, int32_t* tokens, int32_t am, int mode) {
  const int32_t step = state[ST_STEP];
  if (mode == 2) {
    tokens[step] = am;
    state[ST_TOKEN] = am;
  } else if (step + 1 < state[ST_NFEED]) {
    state[ST_TOKEN] = tokens[step + 1];
  }
  state[ST_POS] = state[ST_POS] + 1;
  state[ST_STEP] = step + 1;
}

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

__device__ __forceinline__ DevMat pick3(const DevMat& a, const DevMat& b, const DevMat& c, int s) {
  return s == 0 ? a : (s == 1 ? b : c);
}

// x staging of the graph-path matvec kernels, a template policy: XF32 keeps
// f32 x in LDS (carve_x / stage_x_then, every format); rows_iq.h's
// XPlanes<NR> stages int8 planes for the v_dot4 engine (Q4_0 / Q8_0).
struct XF32 {
  XStage X;
  int need;
  __device__ __forceinline__ XF32(float* smem, int n, int need_) : X(carve_x(smem, n, need_)), need(need_) {}
  template <class After>
  __device__ __forceinline__ void stage(const float* x, int n, const float* w, float eps, bool norm,
                                        After after) const {
    stage_x_then(x, n, w, eps, norm, X.xs[0], X.xs[1], X.xsum, X.red, need & 1, need & 2, after);
  }
  template <uint32_t FMT>
  __device__ __forceinline__ XF src() const {
    return XF{X.xs[MvT<FMT>::L], X.xsum};
  }
};

// ---------------------------------------------------------------- k_qkv --
// rmsnorm(x, attn_norm) -> q/k/v rows -> RoPE(q, k) -> q buffer and the K/V
// cache row at `pos` (src/model/llama.rs:118-130, src/math/ops.rs:48-61).
// q, k and v share one format; a unit is R consecutive rows of one of them.
struct QKVParams {
  DevMat m[3];
  uint32_t units[3];  // units per matrix (rows / R)
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

template <uint32_t FMT, int R, int U, class XP = XF32>
__global__ __launch_bounds__(256) void k_qkv(QKVParams P) {
  extern __shared__ float smem[];
  const XP X(smem, (int)P.n, P.need);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t total = P.units[0] + P.units[1] + P.units[2];
  const uint32_t ubase = (blockIdx.x * 4 + wave) * P.upw;
  const int nunits = ubase >= total ? 0 : (int)min(P.upw, total - ubase);
  const int pos = P.state[ST_POS];
  const uint32_t half = P.hd / 2;
  auto seg = [&](uint32_t u, int& s, uint32_t& p) {
    s = 0;
    p = u;
    if (p >= P.units[0]) {
      p -= P.units[0];
      s = 1;
      if (p >= P.units[1]) {
        p -= P.units[1];
        s = 2;
      }
    }
  };
  auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
    int s;
    uint32_t p;
    seg(ubase + k, s, p);
    A0 = pick3(P.m[0], P.m[1], P.m[2], s);
    A1 = A0;
    r0 = p * R;
    rmax = A0.rows;
  };
  auto stage = [&](auto&& pf) {  // x loads, then the first weight loads, then the staging
    X.stage(P.x, (int)P.n, P.norm_w, P.eps, true, pf);
  };
  auto epi = [&](int k, const float(&y)[R]) {
    if (lane != 0) return;
    int s;
    uint32_t p;
    seg(ubase + k, s, p);
    const uint32_t r0 = p * R;
#pragma unroll
    for (int r = 0; r < R; r += 2) {
      const uint32_t row = r0 + r;
      const float y0 = y[r], y1 = y[r + 1];
      const uint32_t i = (row % P.hd) / 2;  // loaded for v rows too (exact wait counts)
      const float c = P.rope[((size_t)pos * half + i) * 2 + 0];
      const float sn = P.rope[((size_t)pos * half + i) * 2 + 1];
      if (s < 2) {
        const float a = y0 * c - y1 * sn;
        const float b = y0 * sn + y1 * c;
        float* dst = s == 0 ? P.q_out + row : P.kc + (size_t)pos * P.kv_dim + row;
        dst[0] = a;
        dst[1] = b;
      } else {
        P.vc[(size_t)pos * P.kv_dim + row] = y0;
        P.vc[(size_t)pos * P.kv_dim + row + 1] = y1;
      }
    }
  };
  mv_stream<FMT, R, U, false>(nunits, unit, [] {}, stage, epi, X.template src<FMT>(), lane, true);
}

// --------------------------------------------------------------- k_rows --
// out[r] (+)= <W row r, x>: the o-projection and down-projection with the
// residual add fused (src/model/llama.rs:157-161, 172-176), the output
// projection after the final rmsnorm (llama.rs:180-181, 87-89), and the
// standalone matvec.  A unit is R consecutive rows.
struct RowParams {
  DevMat m;
  const float* x;
  const float* norm_w;  // non-null: stage rmsnorm(x)*w (final norm)
  float eps;
  uint32_t n;
  float* out;
  int accumulate;  // 1: out[r] += y, 0: out[r] = y
  uint32_t units;  // ceil(rows / R)
  uint32_t upw;
  int need;
};

template <uint32_t FMT, int R, int U, class XP = XF32>
__global__ __launch_bounds__(256) void k_rows(RowParams P) {
  extern __shared__ float smem[];
  const XP X(smem, (int)P.n, P.need);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t ubase = (blockIdx.x * 4 + wave) * P.upw;
  const int nunits = ubase >= P.units ? 0 : (int)min(P.upw, P.units - ubase);
  auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
    A0 = P.m;
    A1 = P.m;
    r0 = (ubase + k) * R;
    rmax = P.m.rows;
  };
  auto stage = [&](auto&& pf) {  // x loads, then the first weight loads, then the staging
    X.stage(P.x, (int)P.n, P.norm_w, P.eps, P.norm_w != nullptr, pf);
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
  mv_stream<FMT, R, U, false>(nunits, unit, [] {}, stage, epi, X.template src<FMT>(), lane, true);
}

// ------------------------------------------------------------- k_gateup --
// rmsnorm(x, ffn_norm) -> gate and up rows -> silu(g)*u (src/model/
// llama.rs:164-171, src/math/ops.rs:28-37).  A unit is R/2 (gate, up) row
// pairs, interleaved so one x read serves both matrices.
struct GateUpParams {
  DevMat g, u;
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t n;
  float* h;
  uint32_t units;  // ceil(n_ff / (R/2))
  uint32_t upw;
  int need;
};

template <uint32_t FMT, int R, int U, class XP = XF32>
__global__ __launch_bounds__(256) void k_gateup(GateUpParams P) {
  extern __shared__ float smem[];
  const XP X(smem, (int)P.n, P.need);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t ubase = (blockIdx.x * 4 + wave) * P.upw;
  const int nunits = ubase >= P.units ? 0 : (int)min(P.upw, P.units - ubase);
  constexpr int PR = R / 2;
  auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
    A0 = P.g;
    A1 = P.u;
    r0 = (ubase + k) * PR;
    rmax = P.g.rows;
  };
  auto stage = [&](auto&& pf) {  // x loads, then the first weight loads, then the staging
    X.stage(P.x, (int)P.n, P.norm_w, P.eps, true, pf);
  };
  auto epi = [&](int k, const float(&y)[R]) {
    const uint32_t p0 = (ubase + k) * PR;
    if (lane != 0) return;
#pragma unroll
    for (int r = 0; r < PR; ++r) {
      if (p0 + r < P.g.rows) {
        const float g = y[2 * r], u = y[2 * r + 1];
        P.h[p0 + r] = (g / (1.0f + expf(-g))) * u;
      }
    }
  };
  mv_stream<FMT, R, U, true>(nunits, unit, [] {}, stage, epi, X.template src<FMT>(), lane, true);
}

// ---------------------------------------------------------------- k_attn --
// GQA decode attention for one KV head and one slice of at most
// TALOS_ATTN_CHUNK positions (src/model/llama.rs:135-155): scores =
// <q_h, K_t> * scale, max-shifted softmax, o = sum_t p_t V_t.  The number of
// slices follows the live sequence length (ceil(seq / chunk), at most
// nsplit), so short sequences need no combine.  Slices are combined by the
// last block to finish for that KV head, in slice order, so results do not
// depend on block timing.
#define TALOS_ATTN_CHUNK 64

struct AttnParams {
  const float* q;
  const float* kc;
  const float* vc;
  float* out;       // [n_head * hd]
  float* part;      // [n_kv][nsplit][group][hd + 2]
  uint32_t* count;  // [n_kv], self-resetting
  const int32_t* state;
  uint32_t hd, kv_dim, group, nsplit;
  uint32_t max_chunk;  // ceil(context_length / nsplit) >= any live slice
  float scale;
};

static inline size_t attn_lds_bytes(uint32_t hd, uint32_t group, uint32_t nsplit, uint32_t max_chunk) {
  const uint32_t ns = 256 / hd;
  const uint32_t comb = 3 * nsplit * group;
  const uint32_t body = group * max_chunk + ns * group * hd;
  return (size_t)((body > comb ? body : comb) + group * hd + 64) * 4;
}

template <int DPL>
__global__ __launch_bounds__(256) void k_attn(AttnParams P) {
  extern __shared__ float smem[];
  const uint32_t hd = P.hd, group = P.group;
  const uint32_t ns = 256 / hd;
  const uint32_t mc = P.max_chunk;
  float* sc = smem;                             // [group][max_chunk]
  float* ored = sc + group * mc;                // [ns][group][hd]
  const uint32_t comb = 3 * P.nsplit * group;
  const uint32_t body = group * mc + ns * group * hd;
  float* qs = smem + (body > comb ? body : comb);  // [group][hd]
  __shared__ float mh[TALOS_MAX_GROUP], lh[TALOS_MAX_GROUP];
  __shared__ int am_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t j = blockIdx.x, split = blockIdx.y;
  const int seq = P.state[ST_POS] + 1;
  int nsp = (seq + TALOS_ATTN_CHUNK - 1) / TALOS_ATTN_CHUNK;
  if (nsp > (int)P.nsplit) nsp = (int)P.nsplit;
  if ((int)split >= nsp) return;  // uniform per block
  const int chunk = (seq + nsp - 1) / nsp;
  const int t0 = (int)split * chunk;
  const int t1 = min(seq, t0 + chunk);
  const int len = max(0, t1 - t0);

  for (uint32_t i = tid; i < group * hd; i += 256) qs[i] = P.q[(size_t)j * group * hd + i];
  __syncthreads();

  // scores: 16 lanes per position, DPL dims per lane; the block covers 16
  // positions per round and issues all rounds' K loads before reducing.
  const int dl = lane & 15, slot = wave * 4 + (lane >> 4);
  float qr[TALOS_MAX_GROUP][DPL];
#pragma unroll
  for (int h = 0; h < TALOS_MAX_GROUP; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) qr[h][i] = h < (int)group ? qs[h * hd + dl * DPL + i] : 0.f;
  for (int b = 0; b < len; b += 64) {
    float kv[4][DPL];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = b + r * 16 + slot;
      const float* kp = P.kc + (size_t)(t0 + (tl < len ? tl : 0)) * P.kv_dim + j * hd + dl * DPL;
      if constexpr (DPL % 4 == 0) {
#pragma unroll
        for (int i = 0; i < DPL; i += 4) {
          const f4 v = *reinterpret_cast<const f4*>(kp + i);
          kv[r][i] = v.x;
          kv[r][i + 1] = v.y;
          kv[r][i + 2] = v.z;
          kv[r][i + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < DPL; ++i) kv[r][i] = kp[i];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = b + r * 16 + slot;
#pragma unroll
      for (int h = 0; h < TALOS_MAX_GROUP; ++h) {
        if (h < (int)group) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < DPL; ++i) d = __builtin_fmaf(qr[h][i], kv[r][i], d);
          d = row_sum16(d);
          if (tl < len && dl == 0) sc[h * mc + tl] = d * P.scale;
        }
      }
    }
  }
  __syncthreads();

  // softmax statistics per head (one wave per head); sc becomes exp(s - m)
  for (uint32_t h = wave; h < group; h += 4) {
    float m = -INFINITY;
    for (int t = lane; t < len; t += 64) m = fmaxf(m, sc[h * mc + t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < len; t += 64) {
      const float e = expf(sc[h * mc + t] - m);
      sc[h * mc + t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      mh[h] = m;
      lh[h] = l;
    }
  }
  __syncthreads();

  // o[h][d] = sum_t p[h][t] V_t[d]; ns position subsets per dim, 4 loads in
  // flight per thread
  const int d = tid % hd, sub = tid / hd;
  if (sub < (int)ns) {
    float acc[TALOS_MAX_GROUP];
#pragma unroll
    for (int h = 0; h < TALOS_MAX_GROUP; ++h) acc[h] = 0.f;
    for (int t = sub; t < len; t += 4 * (int)ns) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tt = t + r * (int)ns;
        v[r] = tt < len ? P.vc[(size_t)(t0 + tt) * P.kv_dim + j * hd + d] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tt = t + r * (int)ns;
        if (tt < len) {
#pragma unroll
          for (int h = 0; h < TALOS_MAX_GROUP; ++h)
            if (h < (int)group) acc[h] = __builtin_fmaf(sc[h * mc + tt], v[r], acc[h]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < TALOS_MAX_GROUP; ++h)
      if (h < (int)group) ored[(sub * group + h) * hd + d] = acc[h];
  }
  __syncthreads();

  if (nsp == 1) {
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
    mypart[tid * pstride + hd] = mh[tid];
    mypart[tid * pstride + hd + 1] = lh[tid];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = atomicAdd(&P.count[j], 1u);
    am_last = old == (uint32_t)nsp - 1;
  }
  __syncthreads();
  if (!am_last) return;
  __threadfence();
  // Combine: slice statistics into LDS (parallel loads), then weights.
  const float* parts = P.part + (size_t)j * P.nsplit * group * pstride;
  float* cm = smem;                 // [nsp][group] m
  float* cl = cm + nsp * group;     // [nsp][group] l
  float* cw = cl + nsp * group;     // [nsp][group] exp(m - M)
  for (int i = tid; i < nsp * (int)group; i += 256) {
    const int s = i / (int)group, h = i % (int)group;
    cm[i] = parts[((size_t)s * group + h) * pstride + hd];
    cl[i] = parts[((size_t)s * group + h) * pstride + hd + 1];
  }
  __syncthreads();
  if (tid < (int)group) {
    float M = -INFINITY;
    for (int s = 0; s < nsp; ++s) M = fmaxf(M, cm[s * group + tid]);
    float L = 0.f;
    for (int s = 0; s < nsp; ++s) {
      const float w = expf(cm[s * group + tid] - M);
      cw[s * group + tid] = w;
      L = __builtin_fmaf(cl[s * group + tid], w, L);
    }
    lh[tid] = L;
  }
  __syncthreads();
  for (uint32_t i = tid; i < group * hd; i += 256) {
    const uint32_t h = i / hd, dd = i % hd;
    float O = 0.f;
    int s = 0;
    for (; s + 4 <= nsp; s += 4) {
      float o4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o4[r] = parts[((size_t)(s + r) * group + h) * pstride + dd];
#pragma unroll
      for (int r = 0; r < 4; ++r) O = __builtin_fmaf(o4[r], cw[(s + r) * group + h], O);
    }
    for (; s < nsp; ++s) O = __builtin_fmaf(parts[((size_t)s * group + h) * pstride + dd], cw[s * group + h], O);
    P.out[((size_t)j * group + h) * hd + dd] = O / lh[h];
  }
  if (tid == 0) atomicExch(&P.count[j], 0u);
}

// ------------------------------------------------ generic-shape kernels --
// The forms of a layer that any Llama config takes (src/model/llama.rs:
// 45-51 accepts every n_head that n_head_kv divides): q/k/v or gate/up of
// different formats, any head_dim (odd included), n_embd not a multiple of
// n_head, GQA groups of any size.  They follow the reference's steps one by
// one: raw projections, then RoPE and the cache append, then attention in
// three passes over a scores buffer [n_head][context_length] (the passes of
// src/math/metal/kernels.metal:186-237, which take the same shapes).

// RoPE (src/math/ops.rs:48-61: adjacent pairs (2i, 2i+1), i < head_dim / 2,
// of each head, theta from the host-built table; an odd head_dim leaves each
// head's last element as it is) of the raw q into q_out, elements past the
// heads (n_embd > n_head * head_dim) copied; the raw k rotated into the K
// cache row at `pos` and the raw v copied into the V row (the append of
// src/kv_cache.rs).  One thread per element; inputs and outputs are separate
// buffers, so a pair is read whole by both of its threads.
__device__ __forceinline__ float rope_elem(const float* __restrict__ src, uint32_t i, uint32_t hd, int pos,
                                           const float* __restrict__ rope) {
  const uint32_t half = hd / 2, h = i / hd, w = i % hd, p = w / 2;
  if (p >= half) return src[i];
  const float c = rope[((size_t)pos * half + p) * 2 + 0];
  const float sn = rope[((size_t)pos * half + p) * 2 + 1];
  const float a = src[h * hd + 2 * p], b = src[h * hd + 2 * p + 1];
  return (w & 1) ? a * sn + b * c : a * c - b * sn;
}

static __global__ __attribute__((unused)) __launch_bounds__(256) void k_rope_qkv(const float* __restrict__ qraw, const float* __restrict__ kraw,
                                                  const float* __restrict__ vraw, float* __restrict__ q_out,
                                                  float* __restrict__ kc, float* __restrict__ vc,
                                                  const float* __restrict__ rope, const int32_t* __restrict__ state,
                                                  uint32_t n, uint32_t n_head, uint32_t hd, uint32_t kv_dim) {
  const int pos = state[ST_POS];
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) q_out[i] = i < n_head * hd ? rope_elem(qraw, i, hd, pos, rope) : qraw[i];
  if (i < kv_dim) {
    kc[(size_t)pos * kv_dim + i] = rope_elem(kraw, i, hd, pos, rope);
    vc[(size_t)pos * kv_dim + i] = vraw[i];
  }
}

// h[i] = silu(g[i]) * u[i] (src/math/ops.rs:28-37), for gate and up rows of
// different formats (computed by two matvecs).
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                                                float* __restrict__ h, uint32_t n) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) h[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

// Attention in three passes, any head_dim and group (src/model/llama.rs:
// 135-155).  Pass 1: scores[h][t] = <q_h, K_t of KV head h / group> * scale
// for t <= pos; one thread per (head, position), q_h in LDS.
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_attn_scores(const float* __restrict__ q, const float* __restrict__ kc,
                                                     float* __restrict__ scores, const int32_t* __restrict__ state,
                                                     uint32_t hd, uint32_t kv_dim, uint32_t group, uint32_t ctx,
                                                     float scale) {
  extern __shared__ float qs[];
  const int seq = state[ST_POS] + 1;
  const uint32_t h = blockIdx.x, kvh = h / group;
  const int t0 = (int)blockIdx.y * 256;
  if (t0 >= seq) return;  // uniform per block
  for (uint32_t i = threadIdx.x; i < hd; i += 256) qs[i] = q[(size_t)h * hd + i];
  __syncthreads();
  const int t = t0 + (int)threadIdx.x;
  if (t >= seq) return;
  const float* kp = kc + (size_t)t * kv_dim + (size_t)kvh * hd;
  float d = 0.f;
  for (uint32_t i = 0; i < hd; ++i) d += qs[i] * kp[i];
  scores[(size_t)h * ctx + t] = d * scale;
}

// Pass 2 (src/math/ops.rs:15-25): per head, scores become
// exp(s - max) / sum over t <= pos.  One block per head; fixed-order
// reductions.
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_attn_softmax(float* __restrict__ scores, const int32_t* __restrict__ state,
                                                      uint32_t ctx) {
  __shared__ float red[8];
  const int seq = state[ST_POS] + 1;
  float* s = scores + (size_t)blockIdx.x * ctx;
  float m = -INFINITY;
  for (int t = threadIdx.x; t < seq; t += 256) m = fmaxf(m, s[t]);
  m = wave_max(m);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float l = 0.f;
  for (int t = threadIdx.x; t < seq; t += 256) {
    const float e = expf(s[t] - m);
    s[t] = e;
    l += e;
  }
  l = block_sum(l, red, 4);
  const float inv = 1.0f / l;
  for (int t = threadIdx.x; t < seq; t += 256) s[t] *= inv;
}

// Pass 3: out[h][d] = sum_t p[h][t] V_t[kvh][d].  Block (head, 64 dims): four
// position subsets per dim, summed in subset order.
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_attn_out(const float* __restrict__ scores, const float* __restrict__ vc,
                                                  float* __restrict__ out, const int32_t* __restrict__ state,
                                                  uint32_t hd, uint32_t kv_dim, uint32_t group, uint32_t ctx) {
  __shared__ float part[4][64];
  const int seq = state[ST_POS] + 1;
  const uint32_t h = blockIdx.x, kvh = h / group;
  const uint32_t dl = threadIdx.x & 63, sub = threadIdx.x >> 6;
  const uint32_t d = blockIdx.y * 64 + dl;
  const float* s = scores + (size_t)h * ctx;
  float acc = 0.f;
  if (d < hd)
    for (int t = (int)sub; t < seq; t += 4) acc = __builtin_fmaf(s[t], vc[(size_t)t * kv_dim + (size_t)kvh * hd + d], acc);
  part[sub][dl] = acc;
  __syncthreads();
  if (sub == 0 && d < hd) out[(size_t)h * hd + d] = ((part[0][dl] + part[1][dl]) + part[2][dl]) + part[3][dl];
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

static __global__ __attribute__((unused)) __launch_bounds__(256) void k_embed(DevMat M, const int32_t* state, float* x) {
  const uint32_t tok = (uint32_t)state[ST_TOKEN];
  for (uint32_t e = threadIdx.x; e < M.cols; e += 256) x[e] = dq_elem(M, tok, e);
}

// ------------------------------------------------------- k_copy, k_fill --
// Plain device copy (reference point for HBM bandwidth and for scaling the
// FETCH_SIZE / WRITE_SIZE counters), and a fill of distinct values.
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_copy(const u4* __restrict__ src, u4* __restrict__ dst, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_fill(u4* __restrict__ dst, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
    const uint32_t v = (uint32_t)i * 2654435761u;
    dst[i] = u4{v, v + 1, v + 2, v + 3};
  }
}

// --------------------------------------------------------------- k_norm --
// hidden = rmsnorm(x, output_norm) (src/model/llama.rs:180-181).
static __global__ __attribute__((unused)) __launch_bounds__(256) void k_norm(const float* x, const float* w, float eps, uint32_t n, float* out) {
  __shared__ float red[8];
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss += x[i] * x[i];
  ss = block_sum(ss, red, 4);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += 256) out[i] = x[i] * scale * w[i];
}

// ------------------------------------------------------------- k_argmax --
// argmax by total_cmp, ties to the last index (src/sample.rs:7-14).  With
// `advance` (advance_state), the position moves on and the next step's token
// is set on the device: the argmax itself (2, the greedy loop, which also
// appends it to `tokens`) or the next fed prompt token (3) -- both loops run
// without host round trips.
static __global__ __attribute__((unused)) __launch_bounds__(1024) void k_argmax(const float* logits, uint32_t n, int32_t* state,
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
    if (advance) advance_state(state, tokens, bi, advance);
  }
}
