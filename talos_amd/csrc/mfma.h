// mfma.h -- Q4_0 matvec on the matrix cores (v_mfma_i32_16x16x64_i8) for the
// persistent decode kernel.
//
// Batch-1 decode is bandwidth-bound, but the Q4_0 dequant-dot on the vector
// ALUs costs ~2 VALU ops per weight, as much time as the weight bytes take
// to arrive.  Here the integer work moves to the matrix cores and stays
// exact:
//  * x (f32) is staged per 32-element block b as three int8 planes with a
//    scale: x ~= s_b * (a + b'/254 + c/254^2), a, b', c in [-127, 127]
//    (error <= 2^-24 * max|x_b|: f32-level), plus each plane's integer sum
//    over b;
//  * a wave owns 16 weight rows (the MFMA's 16 columns).  In one MFMA lane
//    group g (lanes 16g..16g+15) supplies 16 quants of its own Q4_0 block
//    (the low or the high nibbles, as unsigned bytes 0..15), and the A
//    operand rows 4g..4g+2 hold that block's three x planes (zero in the
//    other groups' k ranges), so D rows 4g..4g+2 are the block's three exact
//    integer piece dots, in the registers of the lanes that own the block;
//  * each lane then applies the block's scales in f32:
//    acc += d * s * (D0' + D1'/254 + D2'/254^2), Dp' = Dp - 8 * (plane sum)
//    (the -8 offset of Q4_0, src/gguf/dtype.rs:83-90, exact in integers).
// The K dimension of a row group is split over the block's 8 waves; partial
// row sums meet in LDS and are added in wave order (deterministic).
#pragma once
#include "coherent.h"
#include "matvec.h"

typedef int v4i __attribute__((ext_vector_type(4)));

// LDS of the int8-plane staging (carve_xq).
struct XQ {
  int8_t* pl;     // [3][nb][32]
  XBlk* bs;       // [nb]
  int8_t* zero;   // 16 zero bytes (A rows that carry no plane)
  float* part;    // [MEGA_NW][gpb][16] per-wave partial row sums
  float* red;     // block-reduction scratch
  int nb;
};

static inline __host__ __device__ size_t xq_lds_bytes(int n, int gpb_max, int nwaves) {
  const size_t nb = (size_t)n / 32;
  return nb * 96 + nb * sizeof(XBlk) + 16 + (size_t)nwaves * gpb_max * 16 * 4 + 64 + 64;
}

__device__ __forceinline__ XQ carve_xq(float* smem, int n, int gpb_max, int nwaves) {
  XQ X;
  X.nb = n / 32;
  uint8_t* p = reinterpret_cast<uint8_t*>(smem);
  X.pl = reinterpret_cast<int8_t*>(p);
  p += (size_t)X.nb * 96;
  X.bs = reinterpret_cast<XBlk*>(p);
  p += (size_t)X.nb * sizeof(XBlk);
  X.zero = reinterpret_cast<int8_t*>(p);
  p += 16;
  X.part = reinterpret_cast<float*>(p);
  p += (size_t)nwaves * gpb_max * 16 * 4;
  X.red = reinterpret_cast<float*>(p);
  return X;
}

// Stage x (n floats, n % 32 == 0, n <= NR*512*8) as int8 planes, optionally
// as rmsnorm(x)*w (src/math/ops.rs:5-12).  Thread t owns 8 consecutive
// elements per round (4 threads = one block).  The loads of the parts of x
// that are final before the barrier (and of w) are issued first, then
// wait() (the barrier), then the other loads, then after() (the matvec's
// first weight loads), then the arithmetic.  The block publishes its raw x
// slice [pub_lo, pub_hi) to `pub` (coherent).
// Plane layout: [3][nb][32] bytes, or with SPLIT [3][2][nb] 16-byte words
// (word h of block b at (h * nb + b) * 16: a wave reading one block per lane
// touches consecutive words, free of LDS bank conflicts).
// DEFER (with norm): the planes are those of x*w, and the returned factor
// 1/sqrt(mean(x^2) + eps) is left for the caller to apply to each matvec
// result (the planes of a block do not depend on a common factor, so the
// sum of squares shares the staging's last block sync instead of taking two
// of its own).  Otherwise the planes are of (x*r)*w and the factor is 1.
template <int NR, int NT, bool SPLIT = false, bool DEFER = false, class Src, class After, class Wait>
__device__ __forceinline__ float stage_xq(Src src, int n, const float* __restrict__ w, float eps, bool norm,
                                          const XQ& X, float* pub, int pub_lo, int pub_hi, After after, Wait wait) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int n8 = n >> 3;
  f4 v[NR][2], wv[NR][2];
  SrcRaw<Src> raw[NR][2];  // summed once every load of the stage is out
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int g8 = r * NT + tid;
    const int gg = g8 < n8 ? g8 : n8 - 1;
    src_load_early(src, gg * 8, raw[r][0]);
    src_load_early(src, gg * 8 + 4, raw[r][1]);
  }
  if (norm) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int g8 = r * NT + tid;
      const int gg = g8 < n8 ? g8 : n8 - 1;
      wv[r][0] = gld4(w + gg * 8);
      wv[r][1] = gld4(w + gg * 8 + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  wait();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int g8 = r * NT + tid;
    const int gg = g8 < n8 ? g8 : n8 - 1;
    src_load_late(src, gg * 8, raw[r][0]);
    src_load_late(src, gg * 8 + 4, raw[r][1]);
  }
  // A source of many parts (Src6) takes its sums before the first weight
  // loads are issued: its loads and those loads would not fit the registers
  // together.
  constexpr bool kSumFirst = Src::kParts >= 5;
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kSumFirst) after();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    v[r][0] = src_sum<Src>(raw[r][0]);
    v[r][1] = src_sum<Src>(raw[r][1]);
  }
  if constexpr (kSumFirst) after();
#pragma unroll
  for (int r = 0; r < NR; ++r)
    if (r * NT + tid >= n8) v[r][0] = v[r][1] = f4{0.f, 0.f, 0.f, 0.f};
  float scale = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        ss += v[r][h].x * v[r][h].x + v[r][h].y * v[r][h].y + v[r][h].z * v[r][h].z + v[r][h].w * v[r][h].w;
    if constexpr (DEFER) {
      ss = wave_sum(ss);
      if ((tid & 63) == 0) X.red[tid >> 6] = ss;  // read after the closing sync
    } else {
      ss = block_sum(ss, X.red, NT / 64);
      scale = 1.0f / sqrtf(ss / (float)n + eps);
    }
  }
  if (tid < 4) reinterpret_cast<uint32_t*>(X.zero)[tid] = 0u;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int g8 = r * NT + tid;
    const bool ok = g8 < n8;
    float x[8] = {v[r][0].x, v[r][0].y, v[r][0].z, v[r][0].w, v[r][1].x, v[r][1].y, v[r][1].z, v[r][1].w};
    if (pub && ok && g8 * 8 >= pub_lo && g8 * 8 < pub_hi) {
      st_coh4(pub + g8 * 8, v[r][0]);
      st_coh4(pub + g8 * 8 + 4, v[r][1]);
    }
    if (norm) {
      const float wx[8] = {wv[r][0].x, wv[r][0].y, wv[r][0].z, wv[r][0].w,
                           wv[r][1].x, wv[r][1].y, wv[r][1].z, wv[r][1].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = x[k] * scale * wx[k];
    }
    float am = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) am = fmaxf(am, fabsf(x[k]));
    // the block is the quad of threads 4m..4m+3
    am = fmaxf(am, dpp_f<DPP_QUAD_1032>(am, am));
    am = fmaxf(am, dpp_f<DPP_QUAD_2301>(am, am));
    const float inv = am > 0.f ? 127.f / am : 0.f;
    uint32_t pa[2], pb[2], pc[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma clang fp contract(off)
      // r = t + 1.5 * 2^23 (|t| <= 127.5) rounds t to the nearest integer
      // (ties to even) and holds it, two's complement, in r's low byte;
      // -254 * (r - 1.5 * 2^23) = fma(r, -254, 254 * 1.5 * 2^23) exactly.
      // t - a is exact, so fma(t, 254, -254 a) is (t - a) * 254 rounded once.
      constexpr float kM = 12582912.f, k254M = 254.f * 12582912.f;
      uint32_t ra[4], rb[4], rc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float t = x[hh * 4 + k] * inv;
        const float fa = t + kM;
        const float t2 = __builtin_fmaf(t, 254.f, __builtin_fmaf(fa, -254.f, k254M));
        const float fb = t2 + kM;
        const float fc = __builtin_fmaf(t2, 254.f, __builtin_fmaf(fb, -254.f, k254M)) + kM;
        ra[k] = __float_as_uint(fa);
        rb[k] = __float_as_uint(fb);
        rc[k] = __float_as_uint(fc);
      }
      // low bytes of four words into one (v_perm_b32: 0-3 pick the second
      // operand's bytes, 4-7 the first's, 0x0c gives 0)
      auto pack = [](const uint32_t (&r)[4]) {
        const uint32_t lo = __builtin_amdgcn_perm(r[1], r[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(r[3], r[2], 0x0c0c0400u);
        return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
      };
      pa[hh] = pack(ra);
      pb[hh] = pack(rb);
      pc[hh] = pack(rc);
    }
    // plane sums over the block: integers below 2^12, exact in f32
    auto bsum = [](const uint32_t (&p)[2]) {
      return (float)__builtin_amdgcn_sdot4((int)p[0], 0x01010101, __builtin_amdgcn_sdot4((int)p[1], 0x01010101, 0,
                                                                                             false), false);
    };
    const float sa = quad_sum(bsum(pa)), sb = quad_sum(bsum(pb)), sc = quad_sum(bsum(pc));
    if (ok) {
      const int blk = g8 >> 2, off = (g8 & 3) * 8;
      const size_t plane = (size_t)X.nb * 32;
      const size_t at = SPLIT ? ((size_t)(off >> 4) * X.nb + blk) * 16 + (off & 15) : (size_t)blk * 32 + off;
      *reinterpret_cast<uint2*>(X.pl + at) = uint2{pa[0], pa[1]};
      *reinterpret_cast<uint2*>(X.pl + plane + at) = uint2{pb[0], pb[1]};
      *reinterpret_cast<uint2*>(X.pl + 2 * plane + at) = uint2{pc[0], pc[1]};
      if ((g8 & 3) == 0) X.bs[blk] = XBlk{am / 127.f, (int)sa, (int)sb, (int)sc};
    }
  }
  __syncthreads();
  if (!DEFER || !norm) return 1.f;
  float t = 0.f;  // block_sum's order
  for (int k = 0; k < NT / 64; ++k) t += X.red[k];
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(1.0f / sqrtf(t / (float)n + eps))));
}

// One item: U tiles of 4 consecutive Q4_0 blocks of one 16-row group.  Lane
// (j = lane & 15, g = lane >> 4) holds, for tile u, block blk0 + 4u + g of
// row j and its f16 scale: each load instruction reads 64 contiguous bytes
// of each of the 16 rows.
template <int U>
struct MqBuf {
  u4 q[U];
  uint32_t sc[U];
};

template <int U, bool PAIR>
__device__ __forceinline__ void mq_load(MqBuf<U>& B, const DevMat& M0, const DevMat& M1, uint32_t row0, int blk0,
                                        int lane) {
  const int j = lane & 15, g = lane >> 4;
  const bool second = PAIR && j >= 8;
  const uint8_t* q = second ? M1.q : M0.q;
  const uint16_t* d = second ? M1.d : M0.d;
  const size_t nb = M0.nchunk;
  const uint32_t row = PAIR ? row0 + (j & 7) : row0 + j;
  const size_t b = (size_t)row * nb + blk0 + g;
#pragma unroll
  for (int u = 0; u < U; ++u) B.q[u] = ldg4(q + (b + 4 * u) * 16);
#pragma unroll
  for (int u = 0; u < U; ++u) B.sc[u] = gld(d + b + 4 * u);
}

__device__ __forceinline__ v4i nib_lo(u4 q) {
  return v4i{(int)(q.x & 0x0F0F0F0Fu), (int)(q.y & 0x0F0F0F0Fu), (int)(q.z & 0x0F0F0F0Fu), (int)(q.w & 0x0F0F0F0Fu)};
}
__device__ __forceinline__ v4i nib_hi(u4 q) {
  return v4i{(int)((q.x >> 4) & 0x0F0F0F0Fu), (int)((q.y >> 4) & 0x0F0F0F0Fu), (int)((q.z >> 4) & 0x0F0F0F0Fu),
             (int)((q.w >> 4) & 0x0F0F0F0Fu)};
}

// acc += this lane's blocks of the item (see the header comment).
template <int U>
__device__ __forceinline__ float mq_compute(const MqBuf<U>& B, const XQ& X, int blk0, int lane, float acc) {
  const int j = lane & 15, g = lane >> 4;
  const int p = j - 4 * g;
  const bool has = p >= 0 && p < 3;
  const int b = blk0 + g;
  const int8_t* abase = X.pl + (size_t)(has ? p : 0) * X.nb * 32;
  constexpr float k1 = 1.0f / 254.0f, k2 = 1.0f / 64516.0f;
  const v4i zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int blk = b + 4 * u;
    const int8_t* alo = has ? abase + (size_t)blk * 32 : X.zero;
    const int8_t* ahi = has ? alo + 16 : X.zero;
    const v4i a0 = *reinterpret_cast<const v4i*>(alo);
    const v4i a1 = *reinterpret_cast<const v4i*>(ahi);
    v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, nib_lo(B.q[u]), zero4, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, nib_hi(B.q[u]), D, 0, 0, 0);
    const XBlk sx = X.bs[blk];
    const float f = __builtin_fmaf((float)(D[2] - 8 * sx.sc), k2,
                                   __builtin_fmaf((float)(D[1] - 8 * sx.sb), k1, (float)(D[0] - 8 * sx.sa)));
    const float d = f16_to_f32((uint16_t)B.sc[u]);
    acc = __builtin_fmaf(d, sx.s * f, acc);
  }
  return acc;
}

// Sum over the 4 lane groups of each of the 16 rows (lanes j, j+16, j+32,
// j+48); lanes 0..15 receive their row's total.
__device__ __forceinline__ float group_sum4(float v) {
  v += __shfl_xor(v, 16, TALOS_WAVE);
  v += __shfl_xor(v, 32, TALOS_WAVE);
  return v;
}

// Tiles per item for a wave range of tpw tiles: the largest divisor <= 8
// (two items in flight stay within the register budget).
static inline __host__ __device__ constexpr int mq_item_tiles(int tpw) {
  int u = tpw < 8 ? tpw : 8;
  while (tpw % u) --u;
  return u;
}

// One matvec phase of the persistent kernel on the matrix cores.
//   ngroups 16-row groups; grp(gi, M0, M1, row0) describes group gi (with
//   PAIR: rows row0..row0+7 of M0 in lanes 0-7 and of M1 in lanes 8-15);
//   block b owns groups [b*gpb, b*gpb + gpb).  Its NW waves form NW/WPG
//   teams; team t takes the block's groups t, t + NW/WPG, ...; wave k of a
//   team covers the TPW tiles (4 blocks each) [k*TPW, (k+1)*TPW) of the
//   group's rows (so cols == WPG * TPW * 128), in items of U tiles, two
//   items in flight;
//   arrive(), stage(pf): as mv_stream (pf issues the first item's loads);
//   fin(gi, jj, ya, yb): the finished rows -- without PAIR rows 2jj and
//   2jj+1 of the group, with PAIR row jj of M0 and of M1 -- called by one
//   thread each after the team's partial sums are added in wave order.
template <int U, int TPW, int WPG, bool PAIR, int NW, class GrpFn, class ArriveFn, class StageFn, class FinFn>
__device__ __forceinline__ void mq_phase(int ngroups, int gpb, GrpFn grp, ArriveFn arrive, StageFn stage, FinFn fin,
                                         const XQ& X, int lane, int wave) {
  static_assert(TPW % U == 0 && NW % WPG == 0, "items must tile the wave's K range");
  constexpr int IPG = TPW / U;    // items per group
  constexpr int NTEAM = NW / WPG;
  const int team = wave / WPG, kw = wave % WPG;
  const int g0 = (int)blockIdx.x * gpb;
  const int ng = g0 < ngroups ? min(gpb, ngroups - g0) : 0;
  const int ngt = team < ng ? (ng - team + NTEAM - 1) / NTEAM : 0;  // this team's groups
  const int nit = ngt * IPG;
  const int wblk = kw * 4 * TPW;
  auto lgroup = [&](int it) { return team + (it / IPG) * NTEAM; };  // block-local group
  auto iblk = [&](int it) { return wblk + (it % IPG) * 4 * U; };
  // Items past the last (and idle waves) load the wave's first blocks of
  // row 0 -- a small region that stays in L2 -- so every load is
  // unconditional and the compiler's wait counts stay exact.
  auto load = [&](MqBuf<U>& B, int it) {
    DevMat M0, M1;
    uint32_t row0;
    const bool live = it < nit;
    const int gi = live ? g0 + lgroup(it) : 0;
    grp(gi, M0, M1, row0);
    mq_load<U, PAIR>(B, M0, M1, live ? row0 : 0u, live ? iblk(it) : wblk, lane);
  };
  MqBuf<U> b0, b1;
  arrive();
  auto pf = [&] { load(b0, 0); };
  stage(pf);
  float acc = 0.f;
  auto step = [&](const MqBuf<U>& B, int it) {
    acc = mq_compute<U>(B, X, iblk(it), lane, acc);
    if (it % IPG == IPG - 1) {
      const float r = group_sum4(acc);
      if (lane < 16) X.part[((size_t)kw * gpb + lgroup(it)) * 16 + lane] = r;
      acc = 0.f;
    }
  };
  for (int it = 0; it < nit; it += 2) {
    load(b1, it + 1);
    step(b0, it);
    if (it + 1 >= nit) break;
    load(b0, it + 2);
    step(b1, it + 1);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < ng * 8; t += NW * 64) {
    const int g = t >> 3, jj = t & 7;
    const int ra = PAIR ? jj : 2 * jj, rb = PAIR ? jj + 8 : 2 * jj + 1;
    float ya = 0.f, yb = 0.f;
#pragma unroll
    for (int w = 0; w < WPG; ++w) {
      ya += X.part[((size_t)w * gpb + g) * 16 + ra];
      yb += X.part[((size_t)w * gpb + g) * 16 + rb];
    }
    fin(g0 + g, jj, ya, yb);
  }
}
