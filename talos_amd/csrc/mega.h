// mega.h -- one persistent kernel per decode step.
//
// The whole token (src/model/llama.rs:96-183 plus the output projection and
// the greedy argmax of src/sample.rs:7-14) runs in one launch of one
// 512-thread workgroup per CU (one fits per CU and the grid is the CU count,
// so all are resident at once).  Phases per layer:
//   qkv (rmsnorm + q/k/v + RoPE + K/V append) | attention | o + residual |
//   rmsnorm + gate/up + SwiGLU | down + residual
// then rmsnorm + output projection with a fused argmax.  A grid barrier
// (coherent.h), or a wait on the arrival flags of just the workgroups that
// produced a phase's input, separates dependent phases.  A phase loads the
// parts of its input that are final before the wait, waits, loads the rest,
// and issues its first weight loads right behind those staging loads.
// Activations cross workgroups only through coherent loads/stores.
#pragma once
#include "coherent.h"
#include "kernels.h"
#include "mfma.h"

#define MEGA_NT 512
#define MEGA_NW (MEGA_NT / 64)

// Slots of the device state block (int32), after ST_STEP.
enum { ST_ERR = 8 };

struct MegaLayer {
  DevMat q, k, v, o, g, u, d;
  const float* attn_norm;
  const float* ffn_norm;
  float* kc;
  float* vc;
};

struct MegaParams {
  const MegaLayer* layers;
  uint32_t n_layer;
  DevMat out_w;
  const float* out_norm;
  DevMat embd;
  uint32_t n, ff, kv_dim, hd, group, n_kv, vocab;
  float eps, scale;
  const float* rope;
  float* x;        // layer-0 input when the host supplies the embedding
  float* act;      // per-layer activation slots (MEGA_ACT_*), lstride floats per layer
  uint32_t np;     // n rounded up to 64: the stride of the n-sized slots
  uint32_t lstride;
  float* logits;
  float* hidden;
  float* part;     // per-layer attention slice partials, pstride floats per layer
  size_t pstride;
  uint32_t* count;
  int32_t* state;
  int32_t* tokens;
  uint32_t* sync;  // mega_sync_words(nblocks) words, laid out as that function describes
  uint32_t nsplit, max_chunk;
  int attn_direct;  // sequences up to this length: one attention item per q head
  int attn_wait;    // attention blocks wait for their q/k/v producers only, not a grid barrier
  int dsplit;       // down-projection in MEGA_DSPLIT column parts (int8-plane x): 1 the
                    // parts on the waves of a team, 2 on different workgroups
  int embed;   // 1: x = embedding row of the state token, looked up on the device
  int hidden_only;
  int argmax;  // 0: none, 1: argmax into state, 2: + greedy advance, 3: + feed advance (advance_state)
  int prefetch;  // issue each matvec phase's first weight loads before its barrier wait
  uint64_t* timeline;  // optional: [nblocks][MEGA_TL_SLOTS] wall-clock marks
  uint32_t spin_limit; // polls before a bounded wait gives up (then ST_ERR is set)
  int one_hop;         // grid barriers: every block reads all arrivals (no release word)
};

// Read-only tables read through the constant address space compile to
// scalar loads.
#define TALOS_CONST __attribute__((address_space(4)))
__device__ __forceinline__ DevMat const_mat(const TALOS_CONST DevMat* p) {
  DevMat m;
  m.q = p->q;
  m.d = p->d;
  m.sc = p->sc;
  m.rows = p->rows;
  m.cols = p->cols;
  m.fmt = p->fmt;
  m.nchunk = p->nchunk;
  return m;
}

// Activation slots of one layer.  Every slot is written once per launch and
// read only after the barrier that follows the write, so consumers read it
// with ordinary cached loads (coherent.h).
// The down-projection output is slot D, or, when its column quarters run on
// different workgroups (MegaParams::dsplit 2), the quarter sums: quarter 0
// in slot D, quarters 1..3 in three slots per layer after the last layer's
// (the layer stride stays that of five slots and h).
enum { MEGA_ACT_BASE = 0, MEGA_ACT_O = 1, MEGA_ACT_D = 2, MEGA_ACT_Q = 3, MEGA_ACT_ATTY = 4, MEGA_ACT_H = 5 };
static inline __host__ __device__ uint32_t mega_np(uint32_t n) { return (n + 63) & ~63u; }
static inline __host__ __device__ uint32_t mega_lstride(uint32_t n, uint32_t ff) {
  return 5 * mega_np(n) + mega_np(ff);
}
// floats of the activation area: n_layer strides, then the quarter slots
static inline __host__ __device__ size_t mega_act_floats(uint32_t n_layer, uint32_t n, uint32_t ff) {
  return (size_t)n_layer * (mega_lstride(n, ff) + 3 * mega_np(n));
}
__device__ __forceinline__ float* mega_act(const MegaParams& P, uint32_t l, int slot) {
  return P.act + (size_t)l * P.lstride + (size_t)slot * P.np;
}
// quarter q's slot of layer l's down-projection sums
__device__ __forceinline__ float* mega_dq(const MegaParams& P, uint32_t l, uint32_t q) {
  return q == 0 ? mega_act(P, l, MEGA_ACT_D)
                : P.act + (size_t)P.n_layer * P.lstride + ((size_t)l * 3 + q - 1) * P.np;
}
// Residual base of layer l: the host-supplied x for layer 0 unless the
// embedding is looked up on the device.
__device__ __forceinline__ float* mega_base(const MegaParams& P, uint32_t l) {
  return (l == 0 && !P.embed) ? P.x : mega_act(P, l, MEGA_ACT_BASE);
}

// Phase timeline: per layer 20 marks (qkv staged/end, attention barrier/end,
// o staged/end, gate-up staged/end, down staged/end, one spare, five inside
// the block's first attention item: inputs loaded, softmax done, PV reduced,
// slice published, item done; then the barrier-passed marks of the qkv, o,
// gate-up and down phases), then head.
#define MEGA_TL_PER_LAYER 20
#define MEGA_TL_ATTN 11
#define MEGA_TL_BAR 16
#define MEGA_TL_SLOTS(n_layer) ((n_layer) * MEGA_TL_PER_LAYER + 8)
#define MEGA_MARK(P, slot)                                                                   \
  do {                                                                                       \
    if ((P).timeline && threadIdx.x == 0)                                                    \
      (P).timeline[(size_t)blockIdx.x * MEGA_TL_SLOTS((P).n_layer) + (slot)] = wall_clock64(); \
  } while (0)

// [nblocks * 16 flags][go @+0][epoch base @+16][done @+32][argmax pairs @+64,
// 2 * nblocks words][packed arrivals, nblocks words rounded up to 4]
static inline size_t mega_sync_words(uint32_t nblocks) {
  return (size_t)nblocks * 16 + 64 + 2 * nblocks + ((nblocks + 3) & ~3u) + 64;
}

// Stage n floats into the LDS layouts, optionally as rmsnorm(x)*w
// (src/math/ops.rs:5-12), with every load of the block (x and the norm
// weights) issued in one batch (one memory round trip).  `after()` runs
// right after that batch is issued: loads it issues complete after the
// staging loads (a wave's vector memory operations complete in order), so the
// matvec's first weight loads go there.  src(e) yields x[e..e+3] for
// e % 4 == 0; the block also publishes the staged raw values of
// [pub_lo, pub_hi) to `pub`.  Requires n % 4 == 0 and n <= MEGA_STAGE_MAX.
// VPT float4 per thread: the caller picks the smallest that covers n
// (mega_stage below).
#define MEGA_VPT 8
#define MEGA_STAGE_MAX (MEGA_VPT * MEGA_NT * 4)

template <int MEGA_VPT_N, class Src, class After, class Wait>
__device__ __forceinline__ void mega_stage_v(Src src, int n, const float* __restrict__ w, float eps, bool norm,
                                             const XStage& X, int need, float* pub, int pub_lo, int pub_hi,
                                             After after, Wait wait) {
#undef MEGA_VPT
#define MEGA_VPT MEGA_VPT_N
  // Opaque copy of the thread index: keeps the compiler from hoisting this
  // index arithmetic out of the layer loop (which would keep it live, and
  // spilled, across every phase).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int n4 = ((n + 15) & ~15) >> 2;
  const int nr = n >> 2;  // real float4 groups
  f4 v[MEGA_VPT];
  // Loads are unconditional (index clamped) so they issue as one batch;
  // out-of-range groups are zeroed afterwards.  The summands of x are added
  // only after every load (norm weights included) is out.
  f4 wv[MEGA_VPT];
  SrcRaw<Src> raw[MEGA_VPT];
#pragma unroll
  for (int i = 0; i < MEGA_VPT; ++i) {
    const int e4 = i * MEGA_NT + tid;
    src_load_early(src, (e4 < nr ? e4 : nr - 1) * 4, raw[i]);
  }
  if (norm) {
#pragma unroll
    for (int i = 0; i < MEGA_VPT; ++i) {
      const int e4 = i * MEGA_NT + tid;
      wv[i] = gld4(w + (e4 < nr ? e4 : nr - 1) * 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  wait();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < MEGA_VPT; ++i) {
    const int e4 = i * MEGA_NT + tid;
    src_load_late(src, (e4 < nr ? e4 : nr - 1) * 4, raw[i]);
  }
  constexpr bool kSumFirst = Src::kParts >= 5;  // as in stage_xq
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kSumFirst) after();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < MEGA_VPT; ++i) v[i] = src_sum<Src>(raw[i]);
  if constexpr (kSumFirst) after();
#pragma unroll
  for (int i = 0; i < MEGA_VPT; ++i)
    if (i * MEGA_NT + tid >= nr) v[i] = f4{0.f, 0.f, 0.f, 0.f};
  float scale = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < MEGA_VPT; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = block_sum(ss, X.red, MEGA_NW);
    scale = 1.0f / sqrtf(ss / (float)n + eps);
  }
#pragma unroll
  for (int i = 0; i < MEGA_VPT; ++i) {
    const int e4 = i * MEGA_NT + tid;
    f4 x = v[i];
    if (e4 < n4) {
      if (pub && e4 < nr && e4 * 4 >= pub_lo && e4 * 4 < pub_hi) st_coh4(pub + e4 * 4, x);
      if (norm && e4 < nr) {
        const f4 ww = wv[i];
        x.x = x.x * scale * ww.x;
        x.y = x.y * scale * ww.y;
        x.z = x.z * scale * ww.z;
        x.w = x.w * scale * ww.w;
      }
      if (need & 1) *reinterpret_cast<f4*>(X.xs[0] + xidx<0>(e4 * 4)) = x;
      if (need & 2) *reinterpret_cast<f4*>(X.xs[1] + xidx<1>(e4 * 4)) = x;
    }
    float s = (x.x + x.y) + (x.z + x.w);
    s = quad_sum(s);
    if (e4 < n4 && (tid & 3) == 0) X.xsum[e4 >> 2] = s;
  }
  __syncthreads();
#undef MEGA_VPT
#define MEGA_VPT 8
}

template <class Src, class After, class Wait>
__device__ __forceinline__ void mega_stage(Src src, int n, const float* __restrict__ w, float eps, bool norm,
                                           const XStage& X, int need, float* pub, int pub_lo, int pub_hi,
                                           After after, Wait wait) {
  if (n <= 2 * MEGA_NT * 4)
    mega_stage_v<2>(src, n, w, eps, norm, X, need, pub, pub_lo, pub_hi, after, wait);
  else
    mega_stage_v<MEGA_VPT>(src, n, w, eps, norm, X, need, pub, pub_lo, pub_hi, after, wait);
}

// Groups per block the matrix-core phases may need (LDS partial sums).
#define MEGA_GPB 8
// Column parts of the split down-projection and the most rows a team of
// MEGA_DSPLIT waves may own.
#define MEGA_DSPLIT 4
#define MEGA_DSPLIT_ROWS 16
// Items in flight in the gate/up and split down-projection streams of the
// int8-plane layers (Q4_0 and Q8_0; with Q8_0 the third item makes the
// kernel spill ~92 bytes per lane, which slows its attention by ~1.5 us per
// layer at 16k positions, less than the two streams gain).
#ifndef MEGA_DEPTH_GU
#define MEGA_DEPTH_GU 3
#endif
#ifndef MEGA_DEPTH_D
#define MEGA_DEPTH_D 2
#endif
// ... and in the down-projection with its quarters on different workgroups
// (four units per wave, each block staging only its quarter)
#ifndef MEGA_DEPTH_DQ
#define MEGA_DEPTH_DQ 3
#endif

// stage_xq with the fewest rounds of 8 elements per thread covering n.
template <class Src, class After, class Wait>
__device__ __forceinline__ void stage_xq_n(Src src, int n, const float* w, float eps, bool norm, const XQ& X,
                                           float* pub, int pub_lo, int pub_hi, After after, Wait wait) {
  const int n8 = n >> 3;
  if (n8 <= MEGA_NT)
    stage_xq<1, MEGA_NT>(src, n, w, eps, norm, X, pub, pub_lo, pub_hi, after, wait);
  else if (n8 <= 2 * MEGA_NT)
    stage_xq<2, MEGA_NT>(src, n, w, eps, norm, X, pub, pub_lo, pub_hi, after, wait);
  else
    stage_xq<4, MEGA_NT>(src, n, w, eps, norm, X, pub, pub_lo, pub_hi, after, wait);
}

// Matvec modes of the persistent kernel: f32 x on the vector ALUs, Q4_0 on
// the matrix cores (mfma.h), or int8-plane x with v_dot4 on the vector ALUs
// (mv_compute for XI; Q4_0 / Q8_0 layers).
enum { MEGA_MM_F32 = 0, MEGA_MM_MFMA = 1, MEGA_MM_DOT4 = 2 };

// The staged x of a vector-ALU matvec phase: f32 (carve_x / mega_stage) or
// int8 planes (carve_xq / stage_xq with the bank-conflict-free layout).
template <bool IQ>
struct MegaX {
  XStage X;
  int need;
  __device__ __forceinline__ MegaX(float* smem, int n, int need_) : X(carve_x(smem, n, need_)), need(need_) {}
  // (the f32 staging applies the rmsnorm factor itself: returns 1)
  template <bool DEFER = false, class Src, class After, class Wait>
  __device__ __forceinline__ float stage(Src src, int n, const float* w, float eps, bool norm, float* pub, int lo,
                                         int hi, After after, Wait wait) const {
    mega_stage(src, n, w, eps, norm, X, need, pub, lo, hi, after, wait);
    return 1.f;
  }
  __device__ __forceinline__ XF src(int layout) const { return XF{X.xs[layout], X.xsum}; }
};
template <>
struct MegaX<true> {
  XQ X;
  __device__ __forceinline__ MegaX(float* smem, int n, int) : X(carve_xq(smem, n, MEGA_GPB, MEGA_NW)) {}
  // DEFER: returns the rmsnorm factor for the caller to apply to each row
  // result (stage_xq); otherwise 1.
  template <bool DEFER = false, class Src, class After, class Wait>
  __device__ __forceinline__ float stage(Src src, int n, const float* w, float eps, bool norm, float* pub, int lo,
                                         int hi, After after, Wait wait) const {
    const int n8 = n >> 3;
    if (n8 <= MEGA_NT)
      return stage_xq<1, MEGA_NT, true, DEFER>(src, n, w, eps, norm, X, pub, lo, hi, after, wait);
    else if (n8 <= 2 * MEGA_NT)
      return stage_xq<2, MEGA_NT, true, DEFER>(src, n, w, eps, norm, X, pub, lo, hi, after, wait);
    else
      return stage_xq<4, MEGA_NT, true, DEFER>(src, n, w, eps, norm, X, pub, lo, hi, after, wait);
  }
  __device__ __forceinline__ XI src(int) const {
    return XI{reinterpret_cast<const uint8_t*>(X.pl), X.bs, X.nb, 0};
  }
};

// x[e..e+3] of one array, of a + b, or of (a + b) + c: the residual stream
// is kept as the layer's base plus the o-projection and down-projection
// outputs, summed in the order of src/model/llama.rs:159-161, 174-176.
// A source is loaded as kParts raw float4 (part) and summed (sum) once all
// loads of the stage are out; kParts == 0: operator() yields the value.
struct Src1 {
  static constexpr int kParts = 1, kEarly = 0;
  const float* a;
  __device__ __forceinline__ f4 part(int, int e) const { return gld4(a + e); }
  __device__ __forceinline__ static f4 sum(const f4* p) { return p[0]; }
};
struct Src2 {  // the layer's residual base (final early) + the o-projection
  static constexpr int kParts = 2, kEarly = 1;
  const float *a, *b;
  __device__ __forceinline__ f4 part(int s, int e) const { return gld4((s == 0 ? a : b) + e); }
  __device__ __forceinline__ static f4 sum(const f4* p) {
    return f4{p[0].x + p[1].x, p[0].y + p[1].y, p[0].z + p[1].z, p[0].w + p[1].w};
  }
};
struct Src3 {  // base and o-projection (final early) + the down-projection
  static constexpr int kParts = 3, kEarly = 2;
  const float *a, *b, *c;
  __device__ __forceinline__ f4 part(int s, int e) const { return gld4((s == 0 ? a : (s == 1 ? b : c)) + e); }
  __device__ __forceinline__ static f4 sum(const f4* p) {
    return f4{(p[0].x + p[1].x) + p[2].x, (p[0].y + p[1].y) + p[2].y, (p[0].z + p[1].z) + p[2].z,
              (p[0].w + p[1].w) + p[2].w};
  }
};

// base + o-projection (final early, added as they are loaded: fewer
// registers held across the barrier) + the four column-quarter sums of the
// down-projection, added in quarter order first (as the sum of one
// workgroup's quarters would be)
struct Src6 {
  static constexpr int kParts = 5, kEarly = 1;
  const float *a, *b, *c0, *c1, *c2, *c3;
  __device__ __forceinline__ f4 part(int s, int e) const {
    if (s == 0) {
      const f4 x = gld4(a + e), y = gld4(b + e);
      return f4{x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w};
    }
    return gld4((s == 1 ? c0 : s == 2 ? c1 : s == 3 ? c2 : c3) + e);
  }
  __device__ __forceinline__ static f4 sum(const f4* p) {
    const f4 d{((p[1].x + p[2].x) + p[3].x) + p[4].x, ((p[1].y + p[2].y) + p[3].y) + p[4].y,
               ((p[1].z + p[2].z) + p[3].z) + p[4].z, ((p[1].w + p[2].w) + p[3].w) + p[4].w};
    return f4{p[0].x + d.x, p[0].y + d.y, p[0].z + d.z, p[0].w + d.w};
  }
};

struct EmbSrc {
  static constexpr int kParts = 0, kEarly = 0;
  DevMat M;
  uint32_t tok;
  __device__ __forceinline__ f4 operator()(int e) const {
    return f4{dq_elem(M, tok, e), dq_elem(M, tok, e + 1), dq_elem(M, tok, e + 2), dq_elem(M, tok, e + 3)};
  }
};

// silu(g) * u (src/math/ops.rs:28-37) with exp2 and the reciprocal on the
// transcendental unit: a few ulp from g / (1 + expf(-g)) * u, in 5 VALU
// instructions instead of ~20 (an epilogue every gate/up item pays).
// g -> -inf: 1 + exp2(+inf) = inf, rcp -> 0, the result -0 * u as with the
// division.
__device__ __forceinline__ float mega_swiglu(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Element i of a layer's down-projection output (slots D..D+3 when its
// column quarters ran on different workgroups).
__device__ __forceinline__ float mega_down(const MegaParams& P, uint32_t l, uint32_t i) {
  if (P.dsplit != 2) return gld(mega_act(P, l, MEGA_ACT_D) + i);
  return ((gld(mega_dq(P, l, 0) + i) + gld(mega_dq(P, l, 1) + i)) + gld(mega_dq(P, l, 2) + i)) +
         gld(mega_dq(P, l, 3) + i);
}

// Strided unit count for global wave gw of tw.
__device__ __forceinline__ int mega_nunits(uint32_t total, uint32_t gw, uint32_t tw) {
  return gw < total ? (int)((total - gw + tw - 1) / tw) : 0;
}

// One attention work item: KV head j, q heads hq0..hq0+ng-1 (ng <=
// MEGA_ATTN_HG), positions [t0, t1) of one slice (src/model/llama.rs:139-155
// for those heads).  The slice is split into 8 contiguous ranges, one per
// wave, and each wave runs its own online softmax with no block barrier:
// steps of MEGA_ATTN_STEP positions, 16 lanes per position holding DPL
// dimensions of its K row and of its V row, the next step's rows loaded
// while this one computes (two register buffers; loads unconditional with
// clamped rows, so the wait counts stay exact).  Scores are kept in log2
// units (q.k * scale * log2 e), so every exponential is one exp2; row sums
// use a mirror butterfly that leaves identical bits in all 16 lanes.  The
// waves' (m, l, o) meet in LDS and are merged in wave order; with nsp > 1
// slices the block publishes the slice partial and the last block to finish
// for KV head j merges the slices in slice order.  q, the K/V row at `pos`
// and the slice partials are written once per launch (coherent stores) and
// read after the barrier or the slice counter that follows the write.
// Short sequences (seq <= P.attn_direct) run one item per q head over all
// positions (ng = 1, nsp = 1): no slice merge, and the group's K/V rows,
// read by the group's items on one XCD, come from its L2.
#define MEGA_ATTN_HG 4
#ifndef MEGA_ATTN_STEP
#define MEGA_ATTN_STEP 4
#endif

// Positions per slice: ceil(seq * n_kv / nblocks) rounded up to 16 (at
// least 16), so that the items (KV head x slice) cover about one per block.
// As chunk >= seq * n_kv / nblocks, the slice count ceil(seq / chunk) is at
// most ceil(nblocks / n_kv).
static inline __host__ __device__ int mega_attn_chunk(int seq, uint32_t n_kv, uint32_t nblocks) {
  int c = (int)(((uint64_t)seq * n_kv + nblocks - 1) / nblocks);
  c = (c + 15) & ~15;
  return c < 16 ? 16 : c;
}
static inline uint32_t mega_attn_max_splits(uint32_t n_kv, uint32_t nblocks) { return (nblocks + n_kv - 1) / n_kv; }
// LDS floats: per wave and head its m and l, and its o row.
static inline size_t mega_attn_lds_floats(uint32_t hd, uint32_t group) {
  return (size_t)MEGA_NW * group * (hd + 2) + 64;
}

// Sum of the 16 lanes of a DPP row, the same bits in every lane (xor 1,
// xor 2, half-mirror, mirror: each step adds two equal-bits halves).
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141
__device__ __forceinline__ float row_allsum16(float v) {
  v += dpp_f<DPP_QUAD_1032>(0.f, v);
  v += dpp_f<DPP_QUAD_2301>(0.f, v);
  v += dpp_f<DPP_ROW_HALF_MIRROR>(0.f, v);
  v += dpp_f<DPP_ROW_MIRROR>(0.f, v);
  return v;
}

template <int DPL>
__device__ __forceinline__ void mega_attn_item(const MegaParams& P, const float* kc, const float* vc, const float* qv,
                                               float* atty, float* part, uint32_t j, uint32_t hq0, uint32_t ng,
                                               int split, int nsp, int chunk, int pos, float* smem, int tls) {
#define ATTN_MARK(k)                  \
  do {                                \
    if (tls >= 0) MEGA_MARK(P, tls + (k)); \
  } while (0)
  constexpr int HD = 16 * DPL;  // head_dim
  constexpr int HG = MEGA_ATTN_HG;
  constexpr int RS = MEGA_ATTN_STEP / 4;  // rounds of 4 positions per step
  constexpr float kLog2e = 1.4426950408889634f;
  const uint32_t group = ng;
  float* mw = smem;                    // [NW][group]
  float* lw = mw + MEGA_NW * group;    // [NW][group]
  float* ow = lw + MEGA_NW * group;    // [NW][group][HD]
  __shared__ int am_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int dl = lane & 15, g = lane >> 4;
  const int seq = pos + 1;
  const int t0 = split * chunk;
  const int t1 = min(seq, t0 + chunk);  // t1 > t0: split < nsp = ceil(seq / chunk)
  const int len = t1 - t0;
  const int pw = (len + MEGA_NW - 1) / MEGA_NW;
  const int w0 = t0 + wave * pw, w1 = min(t1, w0 + pw);  // this wave's positions (maybe none)
  const int nsteps = w1 > w0 ? (w1 - w0 + MEGA_ATTN_STEP - 1) / MEGA_ATTN_STEP : 0;
  const size_t hoff = (size_t)j * HD + (size_t)dl * DPL;
  const float qscale = P.scale * kLog2e;

  float qr[HG][DPL];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    const float* qp = qv + ((size_t)hq0 + (h < (int)ng ? h : 0)) * HD + dl * DPL;
    if constexpr (DPL % 4 == 0) {
#pragma unroll
      for (int i = 0; i < DPL; i += 4) {
        const f4 v = gld4(qp + i);
        qr[h][i] = v.x * qscale;
        qr[h][i + 1] = v.y * qscale;
        qr[h][i + 2] = v.z * qscale;
        qr[h][i + 3] = v.w * qscale;
      }
    } else {
#pragma unroll
      for (int i = 0; i < DPL; ++i) qr[h][i] = gld(qp + i) * qscale;
    }
  }
  // rows of step s (clamped into the slice: out-of-range lanes reload a row
  // of it and are masked)
  auto load = [&](float (&kr)[RS][DPL], float (&vr)[RS][DPL], int s) {
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      const int t = min(w0 + s * MEGA_ATTN_STEP + r * 4 + g, t1 - 1);
      const float* kp = kc + (size_t)t * P.kv_dim + hoff;
      const float* vp = vc + (size_t)t * P.kv_dim + hoff;
      if constexpr (DPL % 4 == 0) {
#pragma unroll
        for (int i = 0; i < DPL; i += 4) {
          const f4 a = gld4(kp + i), b = gld4(vp + i);
          kr[r][i] = a.x;
          kr[r][i + 1] = a.y;
          kr[r][i + 2] = a.z;
          kr[r][i + 3] = a.w;
          vr[r][i] = b.x;
          vr[r][i + 1] = b.y;
          vr[r][i + 2] = b.z;
          vr[r][i + 3] = b.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          kr[r][i] = gld(kp + i);
          vr[r][i] = gld(vp + i);
        }
      }
    }
  };
  float m[HG], l[HG], acc[HG][DPL];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[h][i] = 0.f;
  }
  auto compute = [&](const float (&kr)[RS][DPL], const float (&vr)[RS][DPL], int s) {
    float sc[HG][RS];
    bool ok[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) ok[r] = w0 + s * MEGA_ATTN_STEP + r * 4 + g < w1;
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        float d = 0.f;
        if (h < (int)ng) {
#pragma unroll
          for (int i = 0; i < DPL; ++i) d = __builtin_fmaf(qr[h][i], kr[r][i], d);
          d = row_allsum16(d);
        }
        sc[h][r] = ok[r] ? d : -INFINITY;
      }
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      if (h >= (int)ng) continue;
      float mx = sc[h][0];
#pragma unroll
      for (int r = 1; r < RS; ++r) mx = fmaxf(mx, sc[h][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, TALOS_WAVE));
      mx = fmaxf(mx, __shfl_xor(mx, 32, TALOS_WAVE));
      const float mn = fmaxf(m[h], mx);
      const float a = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[h] - mn);
      m[h] = mn;
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[h][i] *= a;
#pragma unroll
      for (int r = 0; r < RS; ++r) {
        const float p = ok[r] ? __builtin_amdgcn_exp2f(sc[h][r] - mn) : 0.f;
        ps += p;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[h][i] = __builtin_fmaf(p, vr[r][i], acc[h][i]);
      }
      l[h] = __builtin_fmaf(l[h], a, ps);
    }
  };

  float kA[RS][DPL], vA[RS][DPL], kB[RS][DPL], vB[RS][DPL];
  load(kA, vA, 0);
  ATTN_MARK(0);
  for (int s = 0; s < nsteps; s += 2) {
    load(kB, vB, s + 1);
    compute(kA, vA, s);
    if (s + 1 >= nsteps) break;
    load(kA, vA, s + 2);
    compute(kB, vB, s + 1);
  }
  ATTN_MARK(1);
  // this wave's (m, l, o): l and o summed over the 4 row groups in a fixed
  // order (the xor butterfly leaves the same bits in every lane)
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    if (h >= (int)ng) continue;
    float lt = l[h];
    lt += __shfl_xor(lt, 16, TALOS_WAVE);
    lt += __shfl_xor(lt, 32, TALOS_WAVE);
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      float o = acc[h][i];
      o += __shfl_xor(o, 16, TALOS_WAVE);
      o += __shfl_xor(o, 32, TALOS_WAVE);
      acc[h][i] = o;
    }
    if (g == 0) {
#pragma unroll
      for (int i = 0; i < DPL; ++i) ow[((size_t)wave * group + h) * HD + dl * DPL + i] = acc[h][i];
    }
    if (lane == 0) {
      mw[wave * group + h] = m[h];
      lw[wave * group + h] = lt;
    }
  }
  __syncthreads();
  ATTN_MARK(2);
  // merge the waves in wave order
  float O = 0.f, M = -INFINITY, L = 0.f;
  const int oi = tid;
  const bool mine = oi < (int)(group * HD);
  const int oh = mine ? oi / HD : 0, od = oi % HD;
  if (mine) {
#pragma unroll
    for (int w = 0; w < MEGA_NW; ++w) M = fmaxf(M, mw[w * group + oh]);
#pragma unroll
    for (int w = 0; w < MEGA_NW; ++w) {
      const float mv = mw[w * group + oh];
      const float e = mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - M);
      L = __builtin_fmaf(lw[w * group + oh], e, L);
      O = __builtin_fmaf(ow[((size_t)w * group + oh) * HD + od], e, O);
    }
  }
  if (nsp == 1) {
    if (mine) st_coh(atty + ((size_t)hq0 + oh) * HD + od, O / L);
    __syncthreads();
    ATTN_MARK(4);
    return;
  }

  const size_t pstride = HD + 2;
  float* mypart = part + ((size_t)j * P.nsplit + split) * group * pstride;
  if (mine) {
    st_coh(mypart + oh * pstride + od, O);
    if (od == 0) {
      st_coh(mypart + oh * pstride + HD, M);
      st_coh(mypart + oh * pstride + HD + 1, L);
    }
  }
  wait_mem();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(P.count + j, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    am_last = old == (uint32_t)nsp - 1;
  }
  __syncthreads();
  ATTN_MARK(3);
  if (am_last) {
    const float* parts = part + (size_t)j * P.nsplit * group * pstride;
    // One memory round trip per MB slices: each thread loads its element's
    // partials with the slices' (m, l) and folds them in slice order under
    // a running max (clamped loads; only live slices count).
    constexpr int MB = 16;
    for (uint32_t i = tid; i < group * HD; i += MEGA_NT) {
      const uint32_t h = i / HD, dd = i % HD;
      float Ms = -INFINITY, Ls = 0.f, Os = 0.f;
      for (int s0 = 0; s0 < nsp; s0 += MB) {
        float ov[MB], mv[MB], lv[MB];
#pragma unroll
        for (int r = 0; r < MB; ++r) {
          const float* ps = parts + ((size_t)min(s0 + r, nsp - 1) * group + h) * pstride;
          ov[r] = gld(ps + dd);
          mv[r] = gld(ps + HD);
          lv[r] = gld(ps + HD + 1);
        }
        float Mb = Ms;
#pragma unroll
        for (int r = 0; r < MB; ++r)
          if (s0 + r < nsp) Mb = fmaxf(Mb, mv[r]);
        const float a = Ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(Ms - Mb);  // 0 for the first batch
        Ls *= a;
        Os *= a;
#pragma unroll
        for (int r = 0; r < MB; ++r)
          if (s0 + r < nsp) {
            const float w = __builtin_amdgcn_exp2f(mv[r] - Mb);
            Ls = __builtin_fmaf(lv[r], w, Ls);
            Os = __builtin_fmaf(ov[r], w, Os);
          }
        Ms = Mb;
      }
      st_coh(atty + ((size_t)hq0 + h) * HD + dd, Os / Ls);
    }
    if (tid == 0) st_coh_u(P.count + j, 0u);
  }
  __syncthreads();
  ATTN_MARK(4);
#undef ATTN_MARK
}

// MF: the layer matvecs (Q4_0) run on the matrix cores (mfma.h); UN and UF
// are then the tiles per wave of the n- and ff-wide rows (cols / 1024).
template <uint32_t LF, uint32_t OF, int UN, int UF, int UO, int DPL, int MM>
__global__ __launch_bounds__(MEGA_NT) void k_mega(MegaParams P) {
  extern __shared__ float smem[];
  constexpr bool MF = MM == MEGA_MM_MFMA;
  constexpr bool IQ = MM == MEGA_MM_DOT4;
  constexpr bool IQO = IQ && (OF == TALOS_FMT_Q4_0 || OF == TALOS_FMT_Q8_0);  // the head too
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform: scalar registers
  const uint32_t nb = gridDim.x;
  const uint32_t gw = blockIdx.x * MEGA_NW + wave, tw = nb * MEGA_NW;
  GridSync G;
  G.flags = P.sync;
  G.go = P.sync + nb * 16;
  G.err = reinterpret_cast<uint32_t*>(P.state + ST_ERR);
  G.nblocks = nb;
  G.spin = P.spin_limit;
  G.packed = P.sync + nb * 16 + 64 + 2 * nb;
  G.one_hop = P.one_hop;
  uint32_t* epoch_p = P.sync + nb * 16 + 16;
  uint32_t* done = P.sync + nb * 16 + 32;
  int32_t* amx = reinterpret_cast<int32_t*>(P.sync + nb * 16 + 64);
  uint32_t ep = ld_coh_u(epoch_p);
  const int pos = P.state[ST_POS];
  const uint32_t tok = (uint32_t)P.state[ST_TOKEN];
  const uint32_t half = P.hd / 2;
  constexpr int RL = mv_rows(LF), RO = mv_rows(OF);
  // gate/up waves take contiguous runs of row pairs (int8-plane Q4_0 layers)
  constexpr bool GU_RUNS = IQ && LF == TALOS_FMT_Q4_0;
  constexpr int LL = MvT<LF>::L, LO = MvT<OF>::L;
  const int need_l = 1 << LL, need_o = 1 << LO;
  // each matvec phase issues its first weight loads right behind its staging
  // loads
  const bool pre = P.prefetch != 0;
  // this block's slice of the residual base it publishes each layer
  const int slice = (((int)P.n + (int)nb - 1) / (int)nb + 7) & ~7;
  const int pub_lo = (int)blockIdx.x * slice, pub_hi = pub_lo + slice;
  auto arrive = [&] { grid_arrive(G, ep + 1); };
  auto wait = [&] { grid_wait(G, ++ep); };

  // The layer table is read-only for the launch: reading it through the
  // constant address space gives scalar loads.
  typedef const TALOS_CONST MegaLayer* LayerTab;
  const LayerTab layer_tab = (LayerTab)P.layers;
  for (uint32_t l = 0; l < P.n_layer; ++l) {
    const auto LP = layer_tab + l;  // fields are copied out where used
    float* base = mega_base(P, l);
    float* q = mega_act(P, l, MEGA_ACT_Q);
    float* atty = mega_act(P, l, MEGA_ACT_ATTY);
    float* o_out = mega_act(P, l, MEGA_ACT_O);
    float* h = mega_act(P, l, MEGA_ACT_H);
    float* d_out = mega_act(P, l, MEGA_ACT_D);
    // ---- qkv: rmsnorm(x) -> q/k/v -> RoPE -> q, K/V row at pos
    if constexpr (MF) {
      const XQ X = carve_xq(smem, P.n, MEGA_GPB, MEGA_NW);
      const int g_q = (int)P.n / 16, g_kv = (int)P.kv_dim / 16, ngr = g_q + 2 * g_kv;
      const int gpb = (ngr + (int)nb - 1) / (int)nb;
      auto seg = [&](int gi, int& s, uint32_t& row0) {
        s = gi < g_q ? 0 : (gi < g_q + g_kv ? 1 : 2);
        row0 = (uint32_t)(s == 0 ? gi : (s == 1 ? gi - g_q : gi - g_q - g_kv)) * 16;
      };
      auto grp = [&](int gi, DevMat& M0, DevMat& M1, uint32_t& row0) {
        int s;
        seg(gi, s, row0);
        M0 = s == 0 ? const_mat(&LP->q) : (s == 1 ? const_mat(&LP->k) : const_mat(&LP->v));
        M1 = M0;
      };
      auto arr = [&] {
        if (l > 0) arrive();
      };
      auto stage = [&](auto&& pf) {
        if (l > 0) {
          // x = (base + attproj) + down of the previous layer; publish it
          Src3 src{mega_base(P, l - 1), mega_act(P, l - 1, MEGA_ACT_O), mega_act(P, l - 1, MEGA_ACT_D)};
          stage_xq_n(src, P.n, LP->attn_norm, P.eps, true, X, base, pub_lo, pub_hi, pf, [&] {
            wait();
            MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 0);
          });
        } else if (P.embed) {
          EmbSrc src{P.embd, tok};
          stage_xq_n(src, P.n, LP->attn_norm, P.eps, true, X, base, pub_lo, pub_hi, pf, [] {});
        } else {
          Src1 src{P.x};
          stage_xq_n(src, P.n, LP->attn_norm, P.eps, true, X, nullptr, 0, 0, pf, [] {});
        }
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 0);
      };
      auto fin = [&](int gi, int jj, float y0, float y1) {
        int s;
        uint32_t row0;
        seg(gi, s, row0);
        const uint32_t row = row0 + 2 * jj;
        const uint32_t i = (row % P.hd) / 2;
        const float c = P.rope[((size_t)pos * half + i) * 2 + 0];
        const float sn = P.rope[((size_t)pos * half + i) * 2 + 1];
        if (s < 2) {
          float* dst = s == 0 ? q + row : LP->kc + (size_t)pos * P.kv_dim + row;
          st_coh(dst, y0 * c - y1 * sn);
          st_coh(dst + 1, y0 * sn + y1 * c);
        } else {
          st_coh(LP->vc + (size_t)pos * P.kv_dim + row, y0);
          st_coh(LP->vc + (size_t)pos * P.kv_dim + row + 1, y1);
        }
      };
      mq_phase<mq_item_tiles(UN * 2), UN * 2, 4, false, MEGA_NW>(ngr, gpb, grp, arr, stage, fin, X, lane, wave);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 1);
    } else {
      const MegaX<IQ> X(smem, P.n, need_l);
      const uint32_t u0 = P.n / RL, u1 = P.kv_dim / RL, total = u0 + 2 * u1;
      auto seg = [&](uint32_t u, int& s, uint32_t& p) {
        s = u < u0 ? 0 : (u < u0 + u1 ? 1 : 2);
        p = s == 0 ? u : (s == 1 ? u - u0 : u - u0 - u1);
      };
      auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
        int s;
        uint32_t p;
        seg(gw + (uint32_t)k * tw, s, p);
        A0 = s == 0 ? const_mat(&LP->q) : (s == 1 ? const_mat(&LP->k) : const_mat(&LP->v));
        A1 = A0;
        r0 = p * RL;
        rmax = A0.rows;
      };
      auto arr = [&] {
        if (l > 0) arrive();
      };
      float rs = 1.f;  // rmsnorm factor of the staged x, applied per row
      auto stage = [&](auto&& pf) {
        if (l > 0) {
          // x = (base + attproj) + down of the previous layer; publish it
          auto w = [&] {
            wait();
            MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 0);
          };
          bool done = false;
          if constexpr (IQ) {  // quarter sums: int8-plane kernels only
            if (P.dsplit == 2) {
              Src6 src{mega_base(P, l - 1), mega_act(P, l - 1, MEGA_ACT_O), mega_dq(P, l - 1, 0),
                       mega_dq(P, l - 1, 1),   mega_dq(P, l - 1, 2),              mega_dq(P, l - 1, 3)};
              rs = X.template stage<true>(src, P.n, LP->attn_norm, P.eps, true, base, pub_lo, pub_hi, pf, w);
              done = true;
            }
          }
          if (!done) {
            Src3 src{mega_base(P, l - 1), mega_act(P, l - 1, MEGA_ACT_O), mega_act(P, l - 1, MEGA_ACT_D)};
            rs = X.template stage<true>(src, P.n, LP->attn_norm, P.eps, true, base, pub_lo, pub_hi, pf, w);
          }
        } else if (P.embed) {
          EmbSrc src{P.embd, tok};
          rs = X.template stage<true>(src, P.n, LP->attn_norm, P.eps, true, base, pub_lo, pub_hi, pf, [] {});
        } else {
          Src1 src{P.x};
          rs = X.template stage<true>(src, P.n, LP->attn_norm, P.eps, true, nullptr, 0, 0, pf, [] {});
        }
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 0);
      };
      auto epi = [&](int k, const float(&y)[RL]) {
        if (lane != 0) return;
        int s;
        uint32_t p;
        seg(gw + (uint32_t)k * tw, s, p);
        const uint32_t r0 = p * RL;
#pragma unroll
        for (int r = 0; r < RL; r += 2) {
          const uint32_t row = r0 + r;
          const float y0 = y[r] * rs, y1 = y[r + 1] * rs;
          // (loaded for v rows too: a load under the branch would cost the
          // streaming loop its exact wait counts)
          const uint32_t i = (row % P.hd) / 2;
          const float c = P.rope[((size_t)pos * half + i) * 2 + 0];
          const float sn = P.rope[((size_t)pos * half + i) * 2 + 1];
          if (s < 2) {
            float* dst = s == 0 ? q + row : LP->kc + (size_t)pos * P.kv_dim + row;
            st_coh(dst, y0 * c - y1 * sn);
            st_coh(dst + 1, y0 * sn + y1 * c);
          } else {
            st_coh(LP->vc + (size_t)pos * P.kv_dim + row, y0);
            st_coh(LP->vc + (size_t)pos * P.kv_dim + row + 1, y1);
          }
        }
      };
      mv_stream<LF, RL, UN, false, IQ>(mega_nunits(total, gw, tw), unit, arr, stage, epi, X.src(LL), lane,
                                   pre && l > 0);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 1);
    }
    // ---- attention over positions 0..pos
    uint32_t o_prod = nb;  // the blocks [0, o_prod) write the attention output
    {
      // slices of >= 16 positions, sized so that the items (KV head x
      // slice) cover about one per block
      const int seq = pos + 1;
      const int chunk = mega_attn_chunk(seq, P.n_kv, nb);
      const int nsp = (seq + chunk - 1) / chunk;
      // direct: item b is q head (b % n_kv) * group + b / n_kv of KV head
      // b % n_kv (a group's items sit on blocks congruent mod n_kv), over
      // all positions; otherwise item b is slice b / n_kv of KV head b % n_kv
      const bool direct = seq <= P.attn_direct;
      const uint32_t items = direct ? P.n_kv * P.group : P.n_kv * (uint32_t)nsp;
      if (!MF && P.attn_wait && direct) o_prod = items < nb ? items : nb;
      if (!MF && P.attn_wait) {
        // Every block arrives; a block with attention items then waits only
        // for the blocks that computed their q, k and v rows (qkv unit u
        // runs on wave u % tw), the others go on to the o-projection's
        // barrier.
        grid_arrive(G, ep + 1);
        ++ep;
        __syncthreads();  // barrier_skip() as thread 0 read it
        if (blockIdx.x < items && !barrier_skip()) {
          for (uint32_t it = blockIdx.x; it < items; it += nb) {
            const uint32_t jj = it % P.n_kv, hq0 = jj * P.group + (direct ? it / P.n_kv : 0);
            const uint32_t ng = direct ? 1 : P.group, hu = P.hd / RL;  // units per head
            const uint32_t nq = ng * hu, uq0 = hq0 * hu, uk0 = P.n / RL + jj * hu, uv0 = uk0 + P.kv_dim / RL;
            for (uint32_t t = threadIdx.x; t < nq + 2 * hu; t += MEGA_NT) {
              const uint32_t u = t < nq ? uq0 + t : (t < nq + hu ? uk0 + (t - nq) : uv0 + (t - nq - hu));
              const uint32_t b = (u % tw) / MEGA_NW;
              uint32_t k = 0;
              while ((int32_t)(ld_coh_u(G.flags + b * 16) - ep) < 0) {
                if (++k > G.spin) {
                  st_coh_u(G.err, 1u);
                  break;
                }
              }
            }
          }
        }
        __syncthreads();
      } else {
        grid_barrier(G, ++ep);
      }
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 2);
      if (!direct && nsp > (int)P.nsplit) {
        if (threadIdx.x == 0) st_coh_u(G.err, 1u);  // host sized the partials too small
      } else {
        float* part = P.part + (size_t)l * P.pstride;
        for (uint32_t it = blockIdx.x; it < items; it += nb) {
          const uint32_t jj = it % P.n_kv, r = it / P.n_kv;
          mega_attn_item<DPL>(P, LP->kc, LP->vc, q, atty, part, jj, jj * P.group + (direct ? r : 0),
                              direct ? 1 : P.group, direct ? 0 : (int)r, direct ? 1 : nsp, direct ? seq : chunk, pos,
                              smem, it == blockIdx.x ? (int)(l * MEGA_TL_PER_LAYER + MEGA_TL_ATTN) : -1);
        }
      }
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 3);
    }
    // ---- o-projection (the residual add happens where x is next read)
    if constexpr (MF) {
      const XQ X = carve_xq(smem, P.n, MEGA_GPB, MEGA_NW);
      const int ngr = (int)P.n / 16, gpb = (ngr + (int)nb - 1) / (int)nb;
      auto grp = [&](int gi, DevMat& M0, DevMat& M1, uint32_t& row0) {
        M0 = const_mat(&LP->o);
        M1 = M0;
        row0 = (uint32_t)gi * 16;
      };
      auto stage = [&](auto&& pf) {
        Src1 src{atty};
        stage_xq_n(src, P.n, nullptr, 0.f, false, X, nullptr, 0, 0, pf, [&] {
          wait();
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 1);
        });
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 4);
      };
      auto fin = [&](int gi, int jj, float y0, float y1) {
        const uint32_t row = (uint32_t)gi * 16 + 2 * jj;
        st_coh(o_out + row, y0);
        st_coh(o_out + row + 1, y1);
      };
      mq_phase<mq_item_tiles(UN), UN, MEGA_NW, false, MEGA_NW>(ngr, gpb, grp, arrive, stage, fin, X, lane, wave);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 5);
    } else {
      // with x in registers, two rows per unit: the n rows spread over every
      // wave of the grid (4096 rows, 2048 waves)
      constexpr int RP = IQ ? 2 : RL;
      const MegaX<IQ> X(smem, P.n, need_l);
      const uint32_t total = P.n / RP;
      auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
        A0 = const_mat(&LP->o);
        A1 = A0;
        r0 = (gw + (uint32_t)k * tw) * RP;
        rmax = LP->o.rows;
      };
      auto stage = [&](auto&& pf) {
        Src1 src{atty};
        X.stage(src, P.n, nullptr, 0.f, false, nullptr, 0, 0, pf, [&] {
          if (o_prod < nb) {
            // short sequences: only the item blocks [0, o_prod) wrote the
            // attention output; wait for their arrival flags directly
            ++ep;
            __syncthreads();
            if (!barrier_skip() && threadIdx.x < o_prod) {
              uint32_t k = 0;
              while ((int32_t)(ld_coh_u(G.flags + threadIdx.x * 16) - ep) < 0) {
                if (++k > G.spin) {
                  st_coh_u(G.err, 1u);
                  break;
                }
              }
            }
            __syncthreads();
          } else {
            wait();
          }
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 1);
        });
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 4);
      };
      auto epi = [&](int k, const float(&y)[RP]) {
        if (lane != 0) return;
        const uint32_t r0 = (gw + (uint32_t)k * tw) * RP;
#pragma unroll
        for (int r = 0; r < RP; ++r) st_coh(o_out + r0 + r, y[r]);
      };
      mv_stream<LF, RP, UN, false, IQ>(mega_nunits(total, gw, tw), unit, arrive, stage, epi, X.src(LL), lane,
                                   pre);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 5);
    }
    // ---- rmsnorm(base + attproj) + gate/up + SwiGLU
    if constexpr (MF) {
      const XQ X = carve_xq(smem, P.n, MEGA_GPB, MEGA_NW);
      const int ngr = (int)P.ff / 8, gpb = (ngr + (int)nb - 1) / (int)nb;
      auto grp = [&](int gi, DevMat& M0, DevMat& M1, uint32_t& row0) {
        M0 = const_mat(&LP->g);
        M1 = const_mat(&LP->u);
        row0 = (uint32_t)gi * 8;
      };
      auto stage = [&](auto&& pf) {
        Src2 src{base, o_out};
        stage_xq_n(src, P.n, LP->ffn_norm, P.eps, true, X, nullptr, 0, 0, pf, [&] {
          wait();
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 2);
        });
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 6);
      };
      auto fin = [&](int gi, int jj, float g, float u) {
        st_coh(h + (size_t)gi * 8 + jj, mega_swiglu(g, u));
      };
      mq_phase<mq_item_tiles(UN * MEGA_NW), UN * MEGA_NW, 1, true, MEGA_NW>(ngr, gpb, grp, arrive, stage, fin, X, lane, wave);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 7);
    } else {
      // with x in registers, one row pair per unit: 14336 pairs give each of
      // the 2048 waves of a 256-CU grid exactly 7
      constexpr int RG = IQ ? 2 : RL, PR = RG / 2;
      const MegaX<IQ> X(smem, P.n, need_l);
      const uint32_t total = (P.ff + PR - 1) / PR;
      // With the down rows' column quarters on different workgroups and
      // producer-only waits, wave gw takes the contiguous run of pairs
      // [gw * upw, +upw): a quarter of the SwiGLU output then comes from one
      // contiguous range of blocks, which the down staging waits for alone.
      // Q4_0 only: with Q8_0 rows the runs slow the gate/up streaming by
      // more than the wait saves.
      const bool gu_run = GU_RUNS && P.dsplit == 2 && P.attn_wait;
      const uint32_t upw = (total + tw - 1) / tw;
      auto pair0 = [&](int k) { return gu_run ? gw * upw + (uint32_t)k : gw + (uint32_t)k * tw; };
      const int gu_units = gu_run ? (gw * upw < total ? (int)min(upw, total - gw * upw) : 0)
                                  : mega_nunits(total, gw, tw);
      auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
        A0 = const_mat(&LP->g);
        A1 = const_mat(&LP->u);
        r0 = pair0(k) * PR;
        rmax = LP->g.rows;
      };
      float rs = 1.f;  // rmsnorm factor of the staged x, applied per row
      auto stage = [&](auto&& pf) {
        Src2 src{base, o_out};
        rs = X.template stage<true>(src, P.n, LP->ffn_norm, P.eps, true, nullptr, 0, 0, pf, [&] {
          wait();
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 2);
        });
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 6);
      };
      auto epi = [&](int k, const float(&y)[RG]) {
        if (lane != 0) return;
        const uint32_t p0 = pair0(k) * PR;
#pragma unroll
        for (int r = 0; r < PR; ++r) {
          if (p0 + r < P.ff) {
            const float g = y[2 * r] * rs, u = y[2 * r + 1] * rs;
            st_coh(h + p0 + r, mega_swiglu(g, u));
          }
        }
      };
      constexpr int DG = IQ ? MEGA_DEPTH_GU : 2;
      mv_stream<LF, RG, UN, true, IQ, DG>(gu_units, unit, arrive, stage, epi, X.src(LL), lane, pre);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 7);
    }
    // ---- down-projection (2-row units keep the long rows' double buffer in
    // registers)
    if constexpr (MF) {
      const XQ X = carve_xq(smem, P.ff, MEGA_GPB, MEGA_NW);
      const int ngr = (int)P.n / 16, gpb = (ngr + (int)nb - 1) / (int)nb;
      auto grp = [&](int gi, DevMat& M0, DevMat& M1, uint32_t& row0) {
        M0 = const_mat(&LP->d);
        M1 = M0;
        row0 = (uint32_t)gi * 16;
      };
      auto stage = [&](auto&& pf) {
        Src1 src{h};
        stage_xq_n(src, P.ff, nullptr, 0.f, false, X, nullptr, 0, 0, pf, [&] {
          wait();
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 3);
        });
        MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 8);
      };
      auto fin = [&](int gi, int jj, float y0, float y1) {
        const uint32_t row = (uint32_t)gi * 16 + 2 * jj;
        st_coh(d_out + row, y0);
        st_coh(d_out + row + 1, y1);
      };
      mq_phase<mq_item_tiles(UF), UF, MEGA_NW, false, MEGA_NW>(ngr, gpb, grp, arrive, stage, fin, X, lane, wave);
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 9);
    } else {
      auto whole_rows = [&] {
        // two rows per unit: the n = 4096 rows give each of the 2048 waves of
        // a 256-CU grid one unit (UF chunk-steps per item keep the bytes in
        // flight per wave up)
        constexpr int RD = 2;
        const MegaX<IQ> X(smem, P.ff, need_l);
        const uint32_t total = P.n / RD;
        auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
          A0 = const_mat(&LP->d);
          A1 = A0;
          r0 = (gw + (uint32_t)k * tw) * RD;
          rmax = LP->d.rows;
        };
        auto stage = [&](auto&& pf) {
          Src1 src{h};
          X.stage(src, P.ff, nullptr, 0.f, false, nullptr, 0, 0, pf, [&] {
            wait();
            MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 3);
          });
          MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 8);
        };
        auto epi = [&](int k, const float(&y)[RD]) {
          if (lane != 0) return;
          const uint32_t r0 = (gw + (uint32_t)k * tw) * RD;
  #pragma unroll
          for (int r = 0; r < RD; ++r) st_coh(d_out + r0 + r, y[r]);
        };
        mv_stream<LF, RD, UF, false>(mega_nunits(total, gw, tw), unit, arrive, stage, epi, X.src(LL), lane,
                                     pre);
            };
      if constexpr (IQ) {
        if (P.dsplit == 2) {
          // The down rows in column quarters on different workgroups: block
          // b takes quarter b % 4 of the columns of rows [(b / 4) * rpb, +rpb),
          // rpb / 8 rows per wave in two-row units, and stages only its
          // quarter of x (a quarter of the loads and the conversion); the
          // quarter sums go to four slots that the next staging adds in
          // quarter order.
          constexpr int KS = MEGA_DSPLIT, RD = 2;
          const uint32_t part = blockIdx.x % KS, grp = blockIdx.x / KS;
          const uint32_t qn = LP->d.nchunk / KS;  // chunks per quarter
          const uint32_t rpb = P.n / (nb / KS), rpw = rpb / MEGA_NW;
          const MegaX<IQ> X(smem, (int)qn * 32, need_l);
          const uint32_t row0 = grp * rpb + (uint32_t)wave * rpw;
          auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
            A0 = const_mat(&LP->d);
            A0.q += (size_t)part * qn * fmt_chunk_qbytes(LF);
            A0.d += (size_t)part * qn;
            A0.nchunk = qn;
            A1 = A0;
            r0 = row0 + (uint32_t)k * RD;
            rmax = LP->d.rows;
          };
          auto stage = [&](auto&& pf) {
            Src1 src{h + (size_t)part * qn * 32};
            X.stage(src, (int)qn * 32, nullptr, 0.f, false, nullptr, 0, 0, pf, [&] {
              if (GU_RUNS && P.attn_wait) {
                // gate/up wave gw wrote the SwiGLU outputs [gw * upw, +upw):
                // wait for the arrival flags of the blocks that wrote this
                // quarter [e0, e1) only
                ++ep;
                __syncthreads();
                const uint32_t upw = (P.ff + tw - 1) / tw, e0 = part * qn * 32, e1 = e0 + qn * 32;
                const uint32_t b0 = e0 / upw / MEGA_NW, b1 = (e1 - 1) / upw / MEGA_NW;
                if (!barrier_skip()) {
                  for (uint32_t b = b0 + threadIdx.x; b <= b1 && b < nb; b += MEGA_NT) {
                    uint32_t k = 0;
                    while ((int32_t)(ld_coh_u(G.flags + b * 16) - ep) < 0) {
                      if (++k > G.spin) {
                        st_coh_u(G.err, 1u);
                        break;
                      }
                    }
                  }
                }
                __syncthreads();
              } else {
                wait();
              }
              MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 3);
            });
            MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 8);
          };
          float* dq = mega_dq(P, l, part);
          auto epi = [&](int k, const float(&y)[RD]) {
            if (lane != 0) return;
            const uint64_t v2 = (uint64_t)__float_as_uint(y[0]) | ((uint64_t)__float_as_uint(y[1]) << 32);
            __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(dq + row0 + (uint32_t)k * RD)), v2, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);  // the unit's two rows in one store
          };
          constexpr int DD = MEGA_DEPTH_DQ;
          mv_stream<LF, RD, UN, false, true, DD>((int)(rpw / RD), unit, arrive, stage, epi, X.src(LL), lane, pre);
        } else if (P.dsplit) {
          // The down rows in column quarters: the four waves of a team (waves
          // 4t..4t+3 of a block) each take one quarter of the columns of the
          // team's rows, two rows per unit, with the x of their quarter held in
          // registers; the four quarter sums of a row meet in LDS and are added
          // in quarter order.
          constexpr int KS = MEGA_DSPLIT, RD = 2, TEAMS = MEGA_NW / KS;
          __shared__ float dpart[TEAMS][KS][MEGA_DSPLIT_ROWS];
          const MegaX<IQ> X(smem, P.ff, need_l);
          const int part = wave % KS, tm = wave / KS;
          const uint32_t rpt = P.n / (nb * TEAMS);  // rows per team
          const uint32_t team = blockIdx.x * TEAMS + tm;
          const uint32_t qn = LP->d.nchunk / KS;  // chunks per quarter
          auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
            A0 = const_mat(&LP->d);
            A0.q += (size_t)part * qn * fmt_chunk_qbytes(LF);
            A0.d += (size_t)part * qn;
            A0.nchunk = qn;
            A1 = A0;
            r0 = team * rpt + (uint32_t)k * RD;
            rmax = LP->d.rows;
          };
          auto stage = [&](auto&& pf) {
            Src1 src{h};
            X.stage(src, P.ff, nullptr, 0.f, false, nullptr, 0, 0, pf, [&] {
              wait();
              MEGA_MARK(P, l * MEGA_TL_PER_LAYER + MEGA_TL_BAR + 3);
            });
            MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 8);
          };
          auto epi = [&](int k, const float(&y)[RD]) {
            if (lane != 0) return;
#pragma unroll
            for (int r = 0; r < RD; ++r) dpart[tm][part][k * RD + r] = y[r];
          };
          XI xq = X.src(LL);
          xq.c0 = part * (int)qn;
          constexpr int DD = LF == TALOS_FMT_Q4_0 ? MEGA_DEPTH_D : 2;
          mv_stream<LF, RD, UN, false, true, DD>((int)(rpt / RD), unit, arrive, stage, epi, xq, lane, pre);
          __syncthreads();
          if (threadIdx.x < TEAMS * rpt) {
            const uint32_t t = threadIdx.x / rpt, r = threadIdx.x % rpt;
            const float v = ((dpart[t][0][r] + dpart[t][1][r]) + dpart[t][2][r]) + dpart[t][3][r];
            st_coh(d_out + (blockIdx.x * TEAMS + t) * rpt + r, v);
          }
        } else {
          whole_rows();
        }
      } else {
        whole_rows();
      }
      MEGA_MARK(P, l * MEGA_TL_PER_LAYER + 9);
    }
  }

  // ---- head: final rmsnorm of (base + attproj) + down, then logits (+
  // argmax) or the hidden state
  const uint32_t ll = P.n_layer - 1;
  const float* last = mega_base(P, ll);
  const float* last_o = mega_act(P, ll, MEGA_ACT_O);
  const float* last_d = mega_act(P, ll, MEGA_ACT_D);
  __shared__ int32_t wk[MEGA_NW], wi[MEGA_NW];
  int32_t bk = INT32_MIN, bi = -1;
  if (P.hidden_only) {
    grid_barrier(G, ++ep);
    if (blockIdx.x == 0) {
      float ss = 0.f;
      for (uint32_t i = threadIdx.x; i < P.n; i += MEGA_NT) {
        const float v = (gld(last + i) + gld(last_o + i)) + mega_down(P, ll, i);
        ss += v * v;
      }
      ss = block_sum(ss, smem, MEGA_NW);
      const float scale = 1.0f / sqrtf(ss / (float)P.n + P.eps);
      for (uint32_t i = threadIdx.x; i < P.n; i += MEGA_NT) {
        const float v = (gld(last + i) + gld(last_o + i)) + mega_down(P, ll, i);
        P.hidden[i] = v * scale * P.out_norm[i];
      }
    }
  } else {
    const MegaX<IQO> X(smem, P.n, need_o);
    const uint32_t total = (P.vocab + RO - 1) / RO;
    auto unit = [&](int k, DevMat& A0, DevMat& A1, uint32_t& r0, uint32_t& rmax) {
      A0 = P.out_w;
      A1 = P.out_w;
      r0 = (gw + (uint32_t)k * tw) * RO;
      rmax = P.out_w.rows;
    };
    auto stage = [&](auto&& pf) {
      bool done = false;
      if constexpr (IQ) {
        if (P.dsplit == 2) {
          Src6 src{last, last_o, mega_dq(P, ll, 0), mega_dq(P, ll, 1), mega_dq(P, ll, 2), mega_dq(P, ll, 3)};
          X.stage(src, P.n, P.out_norm, P.eps, true, nullptr, 0, 0, pf, [&] { wait(); });
          done = true;
        }
      }
      if (!done) {
        Src3 src{last, last_o, last_d};
        X.stage(src, P.n, P.out_norm, P.eps, true, nullptr, 0, 0, pf, [&] { wait(); });
      }
      MEGA_MARK(P, P.n_layer * MEGA_TL_PER_LAYER + 0);
    };
    auto epi = [&](int k, const float(&y)[RO]) {
      if (lane != 0) return;
      const uint32_t r0 = (gw + (uint32_t)k * tw) * RO;
#pragma unroll
      for (int r = 0; r < RO; ++r) {
        if (r0 + r < P.vocab) {
          P.logits[r0 + r] = y[r];
          const int32_t key = total_key(y[r]);
          if (key > bk || (key == bk && (int32_t)(r0 + r) > bi)) {
            bk = key;
            bi = (int32_t)(r0 + r);
          }
        }
      }
    };
    mv_stream<OF, RO, UO, false>(mega_nunits(total, gw, tw), unit, arrive, stage, epi, X.src(LO), lane, pre);
    MEGA_MARK(P, P.n_layer * MEGA_TL_PER_LAYER + 1);
  }
  // per-block best, then the last block to finish reduces and advances state
  if (lane == 0) {
    wk[wave] = bk;
    wi[wave] = bi;
  }
  __syncthreads();
  __shared__ int am_last;
  if (threadIdx.x == 0) {
    for (int w = 0; w < MEGA_NW; ++w)
      if (wk[w] > bk || (wk[w] == bk && wi[w] > bi)) {
        bk = wk[w];
        bi = wi[w];
      }
    st_coh_i(amx + 2 * blockIdx.x, bk);
    st_coh_i(amx + 2 * blockIdx.x + 1, bi);
    wait_mem();
    const uint32_t old = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    am_last = old == nb - 1;
  }
  __syncthreads();
  if (am_last && threadIdx.x == 0) {
    int32_t k = INT32_MIN, i = -1;
    for (uint32_t b = 0; b < nb; ++b) {
      const int32_t kb = ld_coh_i(amx + 2 * b), ib = ld_coh_i(amx + 2 * b + 1);
      if (kb > k || (kb == k && ib > i)) {
        k = kb;
        i = ib;
      }
    }
    if (P.argmax) {
      P.state[ST_ARGMAX] = i;
      if (P.argmax >= 2) advance_state(P.state, P.tokens, i, P.argmax);
    }
    st_coh_u(epoch_p, ep);
    st_coh_u(done, 0u);
  }
}
