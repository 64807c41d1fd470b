// prefill.h -- batched prompt processing on the matrix cores.
//
// The reference feeds a prompt one Model::step per token (src/main.rs:
// 88-94).  Here a chunk of T prompt tokens goes through each layer together
// (src/model/llama.rs:96-176 for T rows at once), so every weight byte is
// read once per chunk instead of once per token:
//   rows: x_t = dequant_row(token_embd, tok_t); per layer
//   rmsnorm -> q, k, v = GEMMs -> RoPE, K/V rows into the cache ->
//   causal attention -> x += GEMM(o) -> rmsnorm -> gate, up = GEMMs ->
//   SwiGLU -> x += GEMM(down).
// Q4_0 / Q8_0 GEMMs and the attention run on f16 matrix cores with operands
// split into hi + lo halves (k_pf_gemm16, k_pf_attn16: f32-level products,
// f32 sums); F32 and Q6_K matrices, head_dim not a multiple of 32 and
// TALOS_HIP_PF16=0 take the f32 matrix-core kernels (k_pf_gemm, k_pf_attn:
// f32 products and sums, the dequantized weight in f32, exactly the weight
// the reference multiplies).  Only the chunk's last row goes on to the
// final norm and the output projection.
//
// v_mfma_f32_16x16x4_f32 (one wave): D[16][16] += A[16][4] B[4][16] with
// lane l supplying A[l % 16][l / 16] and B[l / 16][l % 16], and holding
// D[4 (l / 16) + r][l % 16] in result register r (checked on the device).
#pragma once
#include "kernels.h"

typedef float pf4 __attribute__((ext_vector_type(4)));

// The split-f16 GEMM's X: per row, groups of 8 elements as 8 hi halves then
// 8 lo halves (hi = f16(x), lo = f16(x - hi)); element k of row t has its hi
// at ((t K + (k & ~7)) * 2 + (k & 7)) and its lo 8 halves later.  The empty
// asm statement pins x as the rounded f32 value its producer computed:
// otherwise the compiler may fold a product feeding the conversion into
// v_fma_mixlo_f16 (the exact product rounded once to f16) for the hi that lo
// is computed from while converting the rounded f32 value for the hi it
// stores, and where the two roundings differ (an f32 value on an f16
// rounding midpoint) hi + lo is off by an f16 ulp.
__device__ __forceinline__ void pf16_split_bits(float v, uint16_t& hi, uint16_t& lo) {
  asm volatile("" : "+v"(v));
  const _Float16 h = (_Float16)v;
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
}
__device__ __forceinline__ size_t pf16_x_at(size_t row_start, uint32_t k) {
  return (row_start + (k & ~7u)) * 2 + (k & 7u);
}

__device__ __forceinline__ pf4 mfma16x4(float a, float b, pf4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// x_t = dequant_row(token_embd, tok_t) (src/model/weights.rs:58-62).
__global__ __launch_bounds__(256) void k_pf_embed(DevMat M, const int32_t* __restrict__ toks, uint32_t n,
                                                  float* __restrict__ X) {
  const uint32_t t = blockIdx.x, tok = (uint32_t)toks[t];
  for (uint32_t e = threadIdx.x; e < n; e += 256) X[(size_t)t * n + e] = dq_elem(M, tok, e);
}

// Xn_t = rmsnorm(x_t) * w (src/math/ops.rs:5-12), one row per block; with
// X16 also in the split-f16 GEMM's interleaved halves.  n % 8 == 0: each
// thread takes 8-element groups with 16-byte loads and stores, a group's 8
// hi and 8 lo halves as two 16-byte words (the sum of squares in another
// order than the scalar loop's, within f32 rounding of it).
__global__ __launch_bounds__(256) void k_pf_rmsnorm(const float* __restrict__ X, const float* __restrict__ w,
                                                    float eps, uint32_t n, float* __restrict__ Xn,
                                                    uint16_t* __restrict__ X16) {
  __shared__ float red[8];
  const size_t ro = (size_t)blockIdx.x * n;
  const float* x = X + ro;
  if (n % 8 == 0) {
    const uint32_t n8 = n / 8;
    const f4* x4 = reinterpret_cast<const f4*>(x);
    float ss = 0.f;
    for (uint32_t gi = threadIdx.x; gi < n8; gi += 256) {
      const f4 a = x4[2 * gi], b = x4[2 * gi + 1];
      ss += ((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w)) + ((b.x * b.x + b.y * b.y) + (b.z * b.z + b.w * b.w));
    }
    ss = block_sum(ss, red, 4);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    const f4* w4 = reinterpret_cast<const f4*>(w);
    f4* y4 = reinterpret_cast<f4*>(Xn + ro);
    for (uint32_t gi = threadIdx.x; gi < n8; gi += 256) {
      const f4 a = x4[2 * gi], b = x4[2 * gi + 1], wa = w4[2 * gi], wb = w4[2 * gi + 1];
      const float v[8] = {a.x * scale * wa.x, a.y * scale * wa.y, a.z * scale * wa.z, a.w * scale * wa.w,
                          b.x * scale * wb.x, b.y * scale * wb.y, b.z * scale * wb.z, b.w * scale * wb.w};
      y4[2 * gi] = f4{v[0], v[1], v[2], v[3]};
      y4[2 * gi + 1] = f4{v[4], v[5], v[6], v[7]};
      if (X16) {
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pf16_split_bits(v[k], hi[k], lo[k]);
        auto pack = [](const uint16_t(&h)[8]) {
          return u4{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                    (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16)};
        };
        u4* d = reinterpret_cast<u4*>(X16 + pf16_x_at(ro, 8 * gi));
        d[0] = pack(hi);
        d[1] = pack(lo);
      }
    }
    return;
  }
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss += x[i] * x[i];
  ss = block_sum(ss, red, 4);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += 256) {
    const float v = x[i] * scale * w[i];
    Xn[ro + i] = v;
    if (X16) {
      const size_t at = pf16_x_at(ro, i);
      pf16_split_bits(v, X16[at], X16[at + 8]);
    }
  }
}

// ------------------------------------------------------------- the GEMM --
// Y_s[t][r] (+)= sum_k X[t][k] W_s[r][k] for t < T and the rows r of up to
// three matrices W_s sharing X (q/k/v, gate/up: one launch).  Block: 8
// waves, a tile of 64 tokens x 128 rows of one matrix; wave w owns rows
// [128 tile + 16 w, +16) for all 64 tokens (four 16 x 16 MFMA tiles).  Per
// 64-wide K chunk the block stages X transposed in LDS, [k][token] with a
// pitch of 80 floats (the 64 lanes of one A read hit 64 distinct banks),
// double buffered; each lane dequantizes its row's elements k = 4 s + l / 16
// of every 32-element block straight from the repacked layout.  The next
// chunk's weight and X loads are issued before the current chunk's MFMAs
// (all unconditional, clamped addresses, so the wait counts stay exact).
// Per output the products are summed in K order, chunk by chunk.
#define PF_KC 64
#define PF_AP 80
#define PF_TOK 64
#define PF_ROWS 128
#define PF_NT 512

struct PfSeg {
  DevMat W;
  float* Y;       // [T][ldy]
  uint32_t ldy;
  uint32_t tiles;  // ceil(W.rows / PF_ROWS)
  // W's tiled copy (k_pf_tile; Q4_0 / Q8_0 with rows % 16 == 0 and
  // cols % 64 == 0), or null: the split-f16 GEMM then reads W itself
  const uint8_t* tq;
  const uint32_t* td;
};

struct PfGemm {
  PfSeg S[3];
  uint32_t nseg;
  const float* X;  // [T][K], K % 4 == 0
  const uint16_t* X16;  // X in interleaved halves (pf16_x_at; k_pf_gemm16)
  uint32_t T, K;
  int accumulate;
  // k_pf_gemm16<FMT, true>: S[0] gate and S[1] up (same rows); a block
  // owns 64 rows of each and writes H = silu(gate) * up ([T][ldh], and its
  // interleaved halves H16) instead of Y
  float* H;
  uint16_t* H16;
  uint32_t ldh;
};

// One lane's weights of a 64-wide K chunk: two 32-element blocks of its row.
template <uint32_t FMT>
struct PfW {
  u4 q[2][FMT == TALOS_FMT_Q8_0 ? 2 : 1];
  uint32_t d;  // the two blocks' f16 scales
};
template <>
struct PfW<TALOS_FMT_F32> {
  float v[2][8];
};
// Q6_K: a 64-wide K chunk is two quarters (32-element runs) of one half
// super-block, held by the two 16-byte layout chunks g2 = 0, 1 of that half
// (elements 16 g2 .. +15 of each quarter): their low-nibble planes a, b, the
// high-bit plane h and the four int8 sub-scales, and the super-block's d.
template <>
struct PfW<TALOS_FMT_Q6_K> {
  u4 a[2], b[2], h[2];
  uint32_t sc[2];
  float d;
};

template <uint32_t FMT>
__device__ __forceinline__ void pf_load_w(PfW<FMT>& F, const DevMat& W, uint32_t rowc, uint32_t k0, uint32_t K,
                                          int g) {
  if constexpr (FMT == TALOS_FMT_F32) {
    const float* wr = reinterpret_cast<const float*>(W.q) + (size_t)rowc * W.nchunk * 4;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const uint32_t k = k0 + 32 * blk + 4 * s + g;
        F.v[blk][s] = wr[k < K ? k : K - 1];
      }
  } else if constexpr (FMT == TALOS_FMT_Q6_K) {
    // K % 256 == 0, so k0 < K is inside the row
    const uint32_t nc = W.nchunk, sb = k0 / 256, c0 = sb * 4 + ((k0 % 256) / 128) * 2;
    const uint8_t* base = W.q + (size_t)rowc * nc * 48;
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const size_t c = c0 + g2;
      F.a[g2] = *reinterpret_cast<const u4*>(base + c * 16);
      F.b[g2] = *reinterpret_cast<const u4*>(base + (size_t)nc * 16 + c * 16);
      F.h[g2] = *reinterpret_cast<const u4*>(base + (size_t)nc * 32 + c * 16);
      F.sc[g2] = W.sc[(size_t)rowc * nc + c];
    }
    F.d = f16_to_f32(W.d[(size_t)rowc * (nc / 4) + sb]);
  } else {
    const uint32_t nb = K / 32;
    uint32_t dd[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const uint32_t bi0 = (k0 + 32 * blk) / 32, bi = bi0 < nb ? bi0 : nb - 1;
      const size_t ci = (size_t)rowc * nb + bi;
      if constexpr (FMT == TALOS_FMT_Q4_0) {
        F.q[blk][0] = *reinterpret_cast<const u4*>(W.q + ci * 16);
      } else {
        F.q[blk][0] = *reinterpret_cast<const u4*>(W.q + ci * 32);
        F.q[blk][1] = *reinterpret_cast<const u4*>(W.q + ci * 32 + 16);
      }
      if (nb % 2) dd[blk] = W.d[ci];
    }
    // the two scales as one aligned word when the row's block count is even
    F.d = nb % 2 ? dd[0] | (dd[1] << 16) : *reinterpret_cast<const uint32_t*>(W.d + (size_t)rowc * nb + k0 / 32);
  }
}

// b[s] = W[row][kb + 4 s + g] for block blk of the chunk (kb = its first
// element; zero past K).
template <uint32_t FMT>
__device__ __forceinline__ void pf_dequant(const PfW<FMT>& F, int blk, uint32_t kb, uint32_t K, int g,
                                           float (&b)[8]) {
  if constexpr (FMT == TALOS_FMT_F32) {
#pragma unroll
    for (int s = 0; s < 8; ++s) b[s] = kb + 4 * s + g < K ? F.v[blk][s] : 0.f;
  } else if constexpr (FMT == TALOS_FMT_Q6_K) {
    // element j = 4 s + g of quarter qt (src/gguf/dtype.rs:98-118): byte
    // j % 16 of layout chunk j / 16 -- the low nibble of plane a (quarter 0)
    // or b (1), the high nibble of a (2) or b (3), and bits 2 qt, 2 qt + 1
    // of plane h above it; y = d * sub-scale * (q - 32)
    const uint32_t qt = (kb % 128) / 32;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int g2 = s >> 2, w = s & 3;  // j / 16, (j % 16) / 4
      const uint32_t lw = (qt & 1) ? F.b[g2][w] : F.a[g2][w];
      const uint32_t by = (lw >> (8 * g)) & 0xFFu, hb = (F.h[g2][w] >> (8 * g + 2 * qt)) & 3u;
      const int q = (int)((qt < 2 ? by & 0x0Fu : by >> 4) | (hb << 4)) - 32;
      const float sub = (float)(int8_t)((F.sc[g2] >> (8 * qt)) & 0xFFu);
      b[s] = F.d * sub * (float)q;
    }
  } else {
    const float d = f16_to_f32((uint16_t)(F.d >> (16 * blk)));
    if constexpr (FMT == TALOS_FMT_Q4_0) {
      const uint32_t w4[4] = {F.q[blk][0].x, F.q[blk][0].y, F.q[blk][0].z, F.q[blk][0].w};
      // element e = 4 s + g: byte e & 15, low nibble for e < 16
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int e = 4 * s + g, by = e & 15;
        const uint32_t v = (w4[by >> 2] >> (8 * (by & 3))) & 0xFFu;
        const int nib = e < 16 ? (int)(v & 15u) : (int)(v >> 4);
        b[s] = kb < K ? d * (float)(nib - 8) : 0.f;
      }
    } else {
      const uint32_t w8[8] = {F.q[blk][0].x, F.q[blk][0].y, F.q[blk][0].z, F.q[blk][0].w,
                              F.q[blk][1].x, F.q[blk][1].y, F.q[blk][1].z, F.q[blk][1].w};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int e = 4 * s + g;
        const uint32_t v = ((w8[e >> 2] >> (8 * (e & 3))) & 0xFFu) ^ 0x80u;
        b[s] = kb < K ? d * (float)(int8_t)v : 0.f;
      }
    }
  }
}

// X[tb .. +64][k0 .. +64]: float4 e = tid + 512 j holds token e % 64,
// elements k0 + 4 (e / 64) .. +3 (zero past T and K).
struct PfX {
  f4 v[2];
};
__device__ __forceinline__ void pf_load_x(PfX& P, const float* __restrict__ X, uint32_t T, uint32_t K, uint32_t tb,
                                          uint32_t k0, int tid) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid + PF_NT * j;
    const uint32_t t = tb + (uint32_t)(e & 63), k = k0 + 4u * (uint32_t)(e >> 6);
    const uint32_t tc = t < T ? t : T - 1, kc = k < K ? k : K - 4;
    const f4 x = *reinterpret_cast<const f4*>(X + (size_t)tc * K + kc);
    P.v[j] = (t < T && k < K) ? x : f4{0.f, 0.f, 0.f, 0.f};
  }
}
__device__ __forceinline__ void pf_store_x(const PfX& P, float* As, int tid) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = tid + PF_NT * j, tt = e & 63, k4 = e >> 6;
    As[(4 * k4 + 0) * PF_AP + tt] = P.v[j].x;
    As[(4 * k4 + 1) * PF_AP + tt] = P.v[j].y;
    As[(4 * k4 + 2) * PF_AP + tt] = P.v[j].z;
    As[(4 * k4 + 3) * PF_AP + tt] = P.v[j].w;
  }
}

template <uint32_t FMT>
__global__ __launch_bounds__(PF_NT) void k_pf_gemm(PfGemm G) {
  __shared__ float As[2][PF_KC * PF_AP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  // this block's matrix and row tile
  uint32_t tile = blockIdx.y, s = 0;
  while (s + 1 < G.nseg && tile >= G.S[s].tiles) tile -= G.S[s++].tiles;
  const PfSeg& S = G.S[s];
  const uint32_t M = S.W.rows;
  const uint32_t tb = blockIdx.x * PF_TOK;
  const uint32_t row = tile * PF_ROWS + (uint32_t)wave * 16 + li;
  const uint32_t rowc = row < M ? row : M - 1;
  pf4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = pf4{0.f, 0.f, 0.f, 0.f};
  const int nchunks = (int)((G.K + PF_KC - 1) / PF_KC);
  PfW<FMT> wc, wn;
  PfX xc, xn;
  pf_load_w<FMT>(wc, S.W, rowc, 0, G.K, g);
  pf_load_x(xc, G.X, G.T, G.K, tb, 0, tid);
  for (int c = 0; c < nchunks; ++c) {
    float* A = As[c & 1];
    pf_store_x(xc, A, tid);
    __syncthreads();
    // the next chunk's loads (the last chunk again when there is none)
    const uint32_t k0 = (uint32_t)c * PF_KC, kn = (uint32_t)(c + 1 < nchunks ? c + 1 : c) * PF_KC;
    pf_load_w<FMT>(wn, S.W, rowc, kn, G.K, g);
    pf_load_x(xn, G.X, G.T, G.K, tb, kn, tid);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      float b[8];
      pf_dequant<FMT>(wc, blk, k0 + 32 * blk, G.K, g, b);
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        const int kk = blk * 32 + 4 * s8 + g;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma16x4(A[kk * PF_AP + 16 * t + li], b[s8], acc[t]);
      }
    }
    wc = wn;
    xc = xn;
  }
  // D[4 g + r][li] of tile t: token tb + 16 t + 4 g + r, weight row `row`
  if (row < M) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t tok = tb + 16 * t + 4 * g + r;
        if (tok < G.T) {
          float* y = S.Y + (size_t)tok * S.ldy + row;
          *y = G.accumulate ? *y + acc[t][r] : acc[t][r];
        }
      }
  }
}

// ------------------------------------------------- the split-f16 GEMM --
// The same product for Q4_0 / Q8_0 weights on v_mfma_f32_16x16x32_f16.  A
// quantized weight is an integer (Q8_0 q in [-128, 127], Q4_0 nib - 8 in
// [-8, 7]) times its block's f16 scale d, and the integers are exact in f16;
// x is split as hi = f16(x), lo = f16(x - hi), which carries x to within
// 2^-22 of itself (f32 level).  Per 32-element block one MFMA pair forms
// sum_k q_k (hi_k + lo_k) exactly in f32 (f16 products are exact), and the
// block adds d times it to the f32 accumulator: the reference's f32 products
// d q x summed in another order, so within f32 rounding of it.  One MFMA
// covers one quant block (K = 32): lane l supplies A[token l % 16][k = 8
// (l / 16) .. +7] and B[k = 8 (l / 16) .. +7][row l % 16], the same k set in
// both, and holds D[token 4 (l / 16) + r][row l % 16] in register r.
// Tile, waves and pipelining as k_pf_gemm.  X arrives split: its producer
// (rmsnorm, attention, SwiGLU) writes the hi and lo halves beside the f32
// rows once (pf16_x_at), instead of every row tile converting it; they are
// staged in LDS as [token][k] halves with a pitch of 72.
typedef _Float16 pfh8 __attribute__((ext_vector_type(8)));
typedef _Float16 pfh2 __attribute__((ext_vector_type(2)));
#define PF_HP 72

__device__ __forceinline__ pf4 mfma16x32h(pfh8 a, pfh8 b, pf4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// hi + lo halves of v = a * b rounded to f32 (pf16_split_bits: the product
// pinned before it is split).
__device__ __forceinline__ void pf16_split_product(float a, float b, _Float16& hi, _Float16& lo) {
  uint16_t hb, lb;
  pf16_split_bits(a * b, hb, lb);
  hi = __builtin_bit_cast(_Float16, hb);
  lo = __builtin_bit_cast(_Float16, lb);
}

// This lane's 8 weights of each of the chunk's two blocks as raw bytes (8
// per block: Q8_0 quants q + 128, or Q4_0 bytes whose low or high nibbles
// are the elements), with the two blocks' f16 scales.
struct PfW16 {
  uint32_t q[2][2];
  uint32_t d;
};
template <uint32_t FMT>
__device__ __forceinline__ void pf16_load_w(PfW16& F, const DevMat& W, uint32_t rowc, uint32_t k0, uint32_t K,
                                            int g) {
  const uint32_t nb = K / 32;
  if (FMT == TALOS_FMT_Q8_0 && nb % 2 == 0) {
    // the chunk's 64 quant bytes (blocks k0 / 32 and + 1, contiguous) as four
    // 16-byte pieces, piece g in lane group g; pf16_swap_q8 then gives every
    // lane 8 bytes of each block
    const size_t ci = (size_t)rowc * nb + k0 / 32;
    const u4 v = *reinterpret_cast<const u4*>(W.q + ci * 32 + 16 * g);
    F.q[0][0] = v.x;
    F.q[0][1] = v.y;
    F.q[1][0] = v.z;
    F.q[1][1] = v.w;
    F.d = *reinterpret_cast<const uint32_t*>(W.d + ci);
    return;
  }
  if (FMT == TALOS_FMT_Q4_0 && nb % 2 == 0) {
    // the chunk's 32 quant bytes as four 8-byte pieces, piece g in lane
    // group g (groups 0, 1: block 0; groups 2, 3: block 1); pf16_swap_q4
    // then gives every lane 8 bytes of each block
    const size_t ci = (size_t)rowc * nb + k0 / 32;
    const uint2 v = *reinterpret_cast<const uint2*>(W.q + ci * 16 + 8 * g);
    F.q[0][0] = v.x;
    F.q[0][1] = v.y;
    F.d = *reinterpret_cast<const uint32_t*>(W.d + ci);
    return;
  }
  uint32_t dd[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const uint32_t bi0 = (k0 + 32 * blk) / 32, bi = bi0 < nb ? bi0 : nb - 1;
    const size_t ci = (size_t)rowc * nb + bi;
    // Q8_0: elements 8 g .. +7 are bytes 8 g .. +7; Q4_0: bytes 8 (g & 1) .. +7,
    // low nibbles for g < 2 (elements j), high for g >= 2 (elements j + 16)
    const uint8_t* src = FMT == TALOS_FMT_Q8_0 ? W.q + ci * 32 + 8 * g : W.q + ci * 16 + 8 * (g & 1);
    const uint2 v = *reinterpret_cast<const uint2*>(src);
    F.q[blk][0] = v.x;
    F.q[blk][1] = v.y;
    if (nb % 2) dd[blk] = W.d[ci];
  }
  // With an even block count per row the chunk's two scales are one aligned
  // 4-byte word: one load instead of two (each load of a wave touches 16
  // rows' lines, and the address unit is what these loads run short of:
  // 14 % off the 1024-token gate/up GEMM)
  F.d = nb % 2 ? dd[0] | (dd[1] << 16) : *reinterpret_cast<const uint32_t*>(W.d + (size_t)rowc * nb + k0 / 32);
}
// The tiled copy of a Q4_0 / Q8_0 matrix (rows % 16 == 0, cols % 64 == 0):
// piece t = ((r / 16) * (cols / 64) + c) * 16 + r % 16 holds row r's
// 64-element chunk c, its two blocks' quant bytes (QB = 64 for Q8_0, 32 for
// Q4_0) at tq + QB t and their two f16 scales as one word td[t].  A wave's
// 16 rows of a chunk are then one contiguous run (1 KB for Q8_0): each load
// instruction of pf16_load_w touches 8 (Q8_0) or 4 (Q4_0) whole lines
// instead of a part of 16 rows' lines each, and the address unit, which the
// split-f16 GEMM's loads run short of, makes half the passes or fewer.
template <uint32_t FMT>
constexpr uint32_t pf_tile_qb() {
  return FMT == TALOS_FMT_Q8_0 ? 64u : 32u;
}
static inline __host__ __device__ size_t pf_tile_bytes(uint32_t fmt, size_t rows, size_t cols) {
  return rows * (cols / 64) * ((fmt == TALOS_FMT_Q8_0 ? 64 : 32) + 4);
}
// One thread per piece, consecutive threads writing consecutive pieces.
template <uint32_t FMT>
__global__ __launch_bounds__(256) void k_pf_tile(DevMat W, uint8_t* __restrict__ tq, uint32_t* __restrict__ td) {
  constexpr uint32_t QB = pf_tile_qb<FMT>();
  const uint32_t nch = W.cols / 64, nb = W.cols / 32;
  const size_t total = (size_t)W.rows * nch;
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const uint32_t li = (uint32_t)(t % 16);
  const size_t rc = t / 16;  // (r / 16) * nch + c
  const uint32_t r = (uint32_t)(rc / nch) * 16 + li, c = (uint32_t)(rc % nch);
  const size_t ci = (size_t)r * nb + 2 * c;  // the chunk's first block
  const u4* src = reinterpret_cast<const u4*>(W.q + ci * (QB / 2));
  u4* dst = reinterpret_cast<u4*>(tq + t * QB);
#pragma unroll
  for (uint32_t i = 0; i < QB / 16; ++i) dst[i] = src[i];
  td[t] = *reinterpret_cast<const uint32_t*>(W.d + ci);
}
// pf16_load_w from the tiled copy (same lane contents).
template <uint32_t FMT>
__device__ __forceinline__ void pf16_load_w_tiled(PfW16& F, const PfSeg& S, uint32_t rowc, uint32_t k0, uint32_t K,
                                                  int g) {
  const size_t t = ((size_t)(rowc >> 4) * (K / 64) + k0 / 64) * 16 + (rowc & 15);
  if (FMT == TALOS_FMT_Q8_0) {
    const u4 v = *reinterpret_cast<const u4*>(S.tq + t * 64 + 16 * g);
    F.q[0][0] = v.x;
    F.q[0][1] = v.y;
    F.q[1][0] = v.z;
    F.q[1][1] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(S.tq + t * 32 + 8 * g);
    F.q[0][0] = v.x;
    F.q[0][1] = v.y;
  }
  F.d = S.td[t];
}
// (TILED a template parameter, not a test of S.tq: a load under a branch
// would leave the compiler waiting for every load in flight where the
// branches meet, the next chunk's weights included)
template <uint32_t FMT, bool TILED>
__device__ __forceinline__ void pf16_load_seg(PfW16& F, const PfSeg& S, uint32_t rowc, uint32_t k0, uint32_t K,
                                              int g) {
  if constexpr (TILED)
    pf16_load_w_tiled<FMT>(F, S, rowc, k0, K, g);
  else
    pf16_load_w<FMT>(F, S.W, rowc, k0, K, g);
}

// After the one-load fetch of a Q8_0 chunk, lane group g holds bytes
// 16 g .. +15 of the chunk (groups 0, 1: block 0; groups 2, 3: block 1).
// v_permlane32_swap trades the upper 32 lanes of its first operand for the
// lower 32 of its second, so swapping words 0, 1 (upper half: groups 2, 3)
// with words 2, 3 (lower half: groups 0, 1) leaves words 0, 1 of every lane
// on block 0 and words 2, 3 on block 1: group g then holds bytes 8 s(g) ..
// +7 of each block, s = (0, 2, 1, 3), the k order its X fragments are read
// in.
__device__ __forceinline__ void pf16_swap_q8(PfW16& F) {
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const auto r = __builtin_amdgcn_permlane32_swap(F.q[0][w], F.q[1][w], false, false);
    F.q[0][w] = r[0];
    F.q[1][w] = r[1];
  }
}

// After the one-load fetch of a Q4_0 chunk, lane group g holds bytes 8 g ..
// +7 of the chunk.  Swapping a word with itself copies the lower 32 lanes'
// value into the upper ones (first result) and the upper lanes' into the
// lower (second): every lane then holds bytes 8 (g & 1) .. +7 of block 0 and
// of block 1 -- exactly what the direct two-load fetch gives it (groups 0, 1
// take the low nibbles, 2, 3 the high).
__device__ __forceinline__ void pf16_swap_q4(PfW16& F) {
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const auto r = __builtin_amdgcn_permlane32_swap(F.q[0][w], F.q[0][w], false, false);
    F.q[0][w] = r[0];
    F.q[1][w] = r[1];
  }
}

// The 8 weights of block blk as f16 integers (zero past K): each byte b
// (a Q8_0 q + 128, or a Q4_0 nibble) becomes the half 1024 + b by placing
// 0x64 above it, then the offset is subtracted (exact in f16).
template <uint32_t FMT>
__device__ __forceinline__ pfh8 pf16_weights(const PfW16& F, int blk, int g, bool live) {
  const float off = FMT == TALOS_FMT_Q8_0 ? 1152.f : 1032.f;
  const pfh2 o2{(_Float16)off, (_Float16)off};
  pfh8 r;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    uint32_t v = F.q[blk][w];
    if (FMT == TALOS_FMT_Q4_0) v = (g >= 2 ? v >> 4 : v) & 0x0F0F0F0Fu;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u);
    const pfh2 a = __builtin_bit_cast(pfh2, lo) - o2, b = __builtin_bit_cast(pfh2, hi) - o2;
    r[4 * w + 0] = a[0];
    r[4 * w + 1] = a[1];
    r[4 * w + 2] = b[0];
    r[4 * w + 3] = b[1];
  }
  return live ? r : pfh8{0, 0, 0, 0, 0, 0, 0, 0};
}

// X[tb .. +64][k0 .. +64] from the interleaved halves: thread t holds token
// t / 8, elements k0 + 8 (t % 8) .. +7 as 8 hi and 8 lo halves (zero past T
// and K).
struct PfX16 {
  u4 h, l;
};
__device__ __forceinline__ void pf16_load_x(PfX16& P, const uint16_t* __restrict__ X16, uint32_t T, uint32_t K,
                                            uint32_t tb, uint32_t k0, int tid) {
  const uint32_t t = tb + (uint32_t)(tid >> 3), k = k0 + 8u * (uint32_t)(tid & 7);
  const uint32_t tc = t < T ? t : T - 1, kc = k < K ? k : K - 8;
  const u4* p = reinterpret_cast<const u4*>(X16 + pf16_x_at((size_t)tc * K, kc));
  const u4 h = p[0], l = p[1];
  const bool ok = t < T && k < K;
  const u4 z{0u, 0u, 0u, 0u};
  P.h = ok ? h : z;
  P.l = ok ? l : z;
}
__device__ __forceinline__ void pf16_store_x(const PfX16& P, _Float16* Xh, _Float16* Xl, int tid) {
  const int tt = tid >> 3, k8 = tid & 7;
  *reinterpret_cast<u4*>(Xh + tt * PF_HP + 8 * k8) = P.h;
  *reinterpret_cast<u4*>(Xl + tt * PF_HP + 8 * k8) = P.l;
}

template <uint32_t FMT, bool SWIGLU = false, bool TILED = false>
__global__ __launch_bounds__(PF_NT) void k_pf_gemm16(PfGemm G) {
  static_assert(FMT == TALOS_FMT_Q4_0 || FMT == TALOS_FMT_Q8_0, "integer weights only");
  __shared__ __align__(16) _Float16 Xs[2][2][64 * PF_HP];  // [buffer][hi, lo][token][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  uint32_t tile = blockIdx.y, s = 0;
  if (SWIGLU) {
    s = (uint32_t)wave >> 2;  // waves 0-3: gate rows, 4-7: the same up rows
  } else {
    while (s + 1 < G.nseg && tile >= G.S[s].tiles) tile -= G.S[s++].tiles;
  }
  const PfSeg& S = G.S[s];
  const uint32_t M = S.W.rows;
  const uint32_t tb = blockIdx.x * 64;
  const uint32_t row = SWIGLU ? tile * (PF_ROWS / 2) + (uint32_t)(wave & 3) * 16 + li
                              : tile * PF_ROWS + (uint32_t)wave * 16 + li;
  const uint32_t rowc = row < M ? row : M - 1;
  pf4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = pf4{0.f, 0.f, 0.f, 0.f};
  const int nchunks = (int)((G.K + PF_KC - 1) / PF_KC);
  // Q8_0 rows of an even block count take the one-load fetch: lane group g
  // then holds elements 8 s(g) .. +7 of each block (pf16_swap_q8), and its X
  // fragments are read in that k order
  const bool one = (G.K / 32) % 2 == 0;  // the one-load fetch (Q8_0 and Q4_0)
  const bool q8one = FMT == TALOS_FMT_Q8_0 && one;
  const int kg = q8one ? ((g & 1) << 1) | (g >> 1) : g;
  PfW16 wc, wn;
  PfX16 xc, xn;
  pf16_load_seg<FMT, TILED>(wc, S, rowc, 0, G.K, g);
  pf16_load_x(xc, G.X16, G.T, G.K, tb, 0, tid);
  for (int c = 0; c < nchunks; ++c) {
    _Float16* Xh = Xs[c & 1][0];
    _Float16* Xl = Xs[c & 1][1];
    const uint32_t k0 = (uint32_t)c * PF_KC, kn = (uint32_t)(c + 1 < nchunks ? c + 1 : c) * PF_KC;
    // the next chunk's X loads go out before this chunk's X is staged (the
    // staging waits for the older loads only), its weights after the sync
    pf16_load_x(xn, G.X16, G.T, G.K, tb, kn, tid);
    pf16_store_x(xc, Xh, Xl, tid);
    __syncthreads();
    pf16_load_seg<FMT, TILED>(wn, S, rowc, kn, G.K, g);
    if (q8one) pf16_swap_q8(wc);
    if (FMT == TALOS_FMT_Q4_0 && one) pf16_swap_q4(wc);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const bool live = k0 + 32 * blk < G.K;
      const pfh8 b = pf16_weights<FMT>(wc, blk, g, live);
      const float d = f16_to_f32((uint16_t)(wc.d >> (16 * blk)));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int off = (16 * t + li) * PF_HP + 32 * blk + 8 * kg;
        const pfh8 ah = *reinterpret_cast<const pfh8*>(Xh + off);
        const pfh8 al = *reinterpret_cast<const pfh8*>(Xl + off);
        pf4 blkacc = mfma16x32h(ah, b, pf4{0.f, 0.f, 0.f, 0.f});
        blkacc = mfma16x32h(al, b, blkacc);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(d, blkacc[r], acc[t][r]);
      }
    }
    wc = wn;
    xc = xn;
  }
  if constexpr (SWIGLU) {
    // gate and up tiles meet in LDS ([gate, up][64 rows][64 tokens], pitch
    // 65), then each thread forms 8 of the block's h = silu(g) * u (the same
    // f32 operations as k_pf_swiglu), rows fastest for the stores
    __syncthreads();  // every wave is done with the X tiles
    float* E = reinterpret_cast<float*>(&Xs[0][0][0]);
    {
      const int rl = (wave & 3) * 16 + li;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) E[(s * 64 + rl) * 65 + 16 * t + 4 * g + r] = acc[t][r];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int idx = tid + PF_NT * k, rl = idx & 63, tk = idx >> 6;
      const uint32_t hrow = tile * (PF_ROWS / 2) + (uint32_t)rl, tok = tb + (uint32_t)tk;
      if (hrow < M && tok < G.T) {
        const float gv = E[rl * 65 + tk], uv = E[(64 + rl) * 65 + tk];
        const float hv = (gv / (1.0f + expf(-gv))) * uv;
        G.H[(size_t)tok * G.ldh + hrow] = hv;
        const size_t at = pf16_x_at((size_t)tok * G.ldh, hrow);
        pf16_split_bits(hv, G.H16[at], G.H16[at + 8]);
      }
    }
    return;
  }
  if (row < M) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t tok = tb + 16 * t + 4 * g + r;
        if (tok < G.T) {
          float* y = S.Y + (size_t)tok * S.ldy + row;
          *y = G.accumulate ? *y + acc[t][r] : acc[t][r];
        }
      }
  }
}

// RoPE of the raw q and k rows of T tokens at positions p0 + t, the K and V
// rows into the cache: four consecutive elements (two rotation pairs of one
// head) per thread with 16-byte loads and stores, head_dim % 4 == 0 (the
// batched prefill takes head_dim % 16 == 0); rope_elem's arithmetic.
__global__ __launch_bounds__(256) void k_pf_rope_kv(const float* __restrict__ Qr, const float* __restrict__ Kr,
                                                    const float* __restrict__ Vr, float* __restrict__ Q,
                                                    float* __restrict__ kc, float* __restrict__ vc,
                                                    const float* __restrict__ rope, uint32_t p0, uint32_t n,
                                                    uint32_t n_head, uint32_t hd, uint32_t kv_dim) {
  const uint32_t t = blockIdx.y, i = (blockIdx.x * 256 + threadIdx.x) * 4;
  const int pos = (int)(p0 + t);
  const uint32_t half = hd / 2;
  // pairs p, p + 1 of the head (p even, so the table's 4 floats are aligned)
  auto rot = [&](const f4 v) {
    const uint32_t p = (i % hd) / 2;
    const f4 cs = *reinterpret_cast<const f4*>(rope + ((size_t)pos * half + p) * 2);
    return f4{v.x * cs.x - v.y * cs.y, v.x * cs.y + v.y * cs.x, v.z * cs.z - v.w * cs.w, v.z * cs.w + v.w * cs.z};
  };
  if (i < n) {
    const f4 v = *reinterpret_cast<const f4*>(Qr + (size_t)t * n + i);
    *reinterpret_cast<f4*>(Q + (size_t)t * n + i) = i < n_head * hd ? rot(v) : v;
  }
  if (i < kv_dim) {
    *reinterpret_cast<f4*>(kc + (size_t)pos * kv_dim + i) = rot(*reinterpret_cast<const f4*>(Kr + (size_t)t * kv_dim + i));
    *reinterpret_cast<f4*>(vc + (size_t)pos * kv_dim + i) = *reinterpret_cast<const f4*>(Vr + (size_t)t * kv_dim + i);
  }
}

// h = silu(g) * u row-wise over T rows of ff (src/math/ops.rs:28-37); with
// H16 (ff % 8 == 0) also in the split-f16 GEMM's interleaved halves.
__global__ __launch_bounds__(256) void k_pf_swiglu(const float* __restrict__ Gt, const float* __restrict__ Ut,
                                                   float* __restrict__ H, uint16_t* __restrict__ H16,
                                                   size_t count) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const float v = (Gt[i] / (1.0f + expf(-Gt[i]))) * Ut[i];
  H[i] = v;
  if (H16) {
    const size_t at = (i & ~(size_t)7) * 2 + (i & 7);
    pf16_split_bits(v, H16[at], H16[at + 8]);
  }
}

// ---------------------------------------------------- flash attention --
// ATT[t][h hd ..] = softmax_j(<q_t,h, K_j> / sqrt(hd)) V_j over positions
// j <= p0 + t (src/model/llama.rs:135-155 for T queries).  Block: KV head
// kvh, 16 queries, one wave per q head of the group (HPB waves); K/V tiles of
// 64 positions staged in LDS and shared by the waves.  Per wave and tile:
//   S^T = K Q^T on the matrix cores, the K rows of each 16-position
//   sub-tile taken in the order pi(i) = 4 (i % 4) + i / 4, so that result
//   register r of lane l holds position 4 r + l / 16 for query l % 16 --
//   exactly the B operand of step r of the next product;
//   online softmax per query in log2 units;
//   O^T += V^T P^T on the matrix cores (hd / 16 tiles of 16 dimensions).
// Requires head_dim % 16 == 0 (<= 256) and a group of at most 8 (waves).
#define PF_ATT_Q 16
#define PF_ATT_KT 64

struct PfAttn {
  const float* Q;    // [T][n] (rotated)
  const float* kc;   // this layer's cache [ctx][kv_dim]
  const float* vc;
  float* out;        // [T][n]
  uint16_t* out16;   // with it, out in the split-f16 GEMM's interleaved halves too (or null)
  uint32_t T, p0, n, kv_dim, hd, group;
  float scale;       // 1 / sqrt(hd)
};

// The attention's output row for one query and head: this lane's O^T
// registers (tile i, register r: dim 16 i + 4 g + r) times inv into
// out[row + col0 ..] and, with out16, as interleaved hi and lo halves.
template <int HD>
__device__ __forceinline__ void pf_attn_store(const pf4 (&o)[HD / 16], float inv, float* out, uint16_t* out16,
                                              size_t row, uint32_t col0, int g) {
#pragma unroll
  for (int i = 0; i < HD / 16; ++i) {
    const uint32_t col = col0 + 16 * i + 4 * g;
    const f4 v{o[i][0] * inv, o[i][1] * inv, o[i][2] * inv, o[i][3] * inv};
    *reinterpret_cast<f4*>(out + row + col) = v;
    if (out16) {
      uint16_t hb[4], lb[4];
      pf16_split_bits(v.x, hb[0], lb[0]);
      pf16_split_bits(v.y, hb[1], lb[1]);
      pf16_split_bits(v.z, hb[2], lb[2]);
      pf16_split_bits(v.w, hb[3], lb[3]);
      uint16_t* d = out16 + pf16_x_at(row, col);  // col % 4 == 0: four elements of one group
      *reinterpret_cast<uint2*>(d) = uint2{hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16)};
      *reinterpret_cast<uint2*>(d + 8) = uint2{lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16)};
    }
  }
}

// NT threads (max(4, group) waves, rounded to 4 or 8); the block's K/V tile
// for positions j0 .. j0 + 63 is fetched as float4 (16 per position and
// array at HD = 64 ...), C per thread, into registers one tile ahead of the
// tile being computed, then written to LDS between two block syncs.
template <int HD, int NT>
__global__ __launch_bounds__(NT) void k_pf_attn(PfAttn A) {
  constexpr int KP = HD + 4, VP = HD + 16;  // LDS pitches: conflict-free A reads of K and of V
  constexpr int F4 = PF_ATT_KT * HD / 4;    // float4 per tile and array
  constexpr int C = (F4 + NT - 1) / NT;     // per thread
  extern __shared__ float sm[];
  float* Ks = sm;                   // [64][KP]
  float* Vs = sm + PF_ATT_KT * KP;  // [64][VP]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  // the latest queries (the longest causal loops) go out first
  const uint32_t kvh = blockIdx.x, t0 = (gridDim.y - 1 - blockIdx.y) * PF_ATT_Q;
  const uint32_t h = kvh * A.group + (uint32_t)wave;  // this wave's q head
  const bool live = (uint32_t)wave < A.group;
  const uint32_t tq = t0 + li;                         // this lane's query (B column)
  const int qpos = (int)(A.p0 + (tq < A.T ? tq : A.T - 1));
  constexpr float kLog2e = 1.4426950408889634f;
  // Q^T fragments: lane l supplies Q[query li][d = 4 s + g] for step s
  float qf[HD / 4];
  {
    const float* qrow = A.Q + (size_t)(tq < A.T ? tq : A.T - 1) * A.n + (size_t)(live ? h : 0) * HD;
#pragma unroll
    for (int s = 0; s < HD / 4; ++s) qf[s] = qrow[4 * s + g] * (A.scale * kLog2e);
  }
  pf4 o[HD / 16];
#pragma unroll
  for (int i = 0; i < HD / 16; ++i) o[i] = pf4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  // positions 0 .. last, last = the block's largest query position
  const int last = (int)(A.p0 + min(t0 + PF_ATT_Q, A.T) - 1);
  const float* kbase = A.kc + (size_t)kvh * HD;
  const float* vbase = A.vc + (size_t)kvh * HD;
  f4 kr[C], vr[C];
  // float4 e of a tile: position e / (HD / 4), dims 4 (e % (HD / 4)) .. +3;
  // positions past `last` (and e past the tile) read a clamped row and are
  // zeroed when stored
  auto fetch = [&](int j0) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int e = tid + NT * c, pj = e / (HD / 4), d4 = e % (HD / 4);
      const int j = min(j0 + min(pj, PF_ATT_KT - 1), last);
      kr[c] = *reinterpret_cast<const f4*>(kbase + (size_t)j * A.kv_dim + 4 * d4);
      vr[c] = *reinterpret_cast<const f4*>(vbase + (size_t)j * A.kv_dim + 4 * d4);
    }
  };
  auto put = [&](int j0) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int e = tid + NT * c, pj = e / (HD / 4), d4 = e % (HD / 4);
      if (e < F4) {
        const bool ok = j0 + pj <= last;
        const f4 z{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f4*>(Ks + pj * KP + 4 * d4) = ok ? kr[c] : z;
        *reinterpret_cast<f4*>(Vs + pj * VP + 4 * d4) = ok ? vr[c] : z;
      }
    }
  };
  fetch(0);
  for (int j0 = 0; j0 <= last; j0 += PF_ATT_KT) {
    __syncthreads();  // the previous tile's reads of Ks / Vs are done
    put(j0);
    __syncthreads();
    fetch(j0 + PF_ATT_KT <= last ? j0 + PF_ATT_KT : j0);  // the next tile's rows in flight
    if (!live) continue;
    // S^T for the four 16-position sub-tiles
    pf4 st[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      st[u] = pf4{0.f, 0.f, 0.f, 0.f};
      const int prow = 16 * u + 4 * (li % 4) + li / 4;  // pi(li) within sub-tile u
#pragma unroll
      for (int s = 0; s < HD / 4; ++s) st[u] = mfma16x4(Ks[prow * KP + 4 * s + g], qf[s], st[u]);
    }
    // causal mask and the tile's max per query (lanes li, li+16, li+32, li+48)
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + 16 * u + 4 * r + g;
        if (j > qpos) st[u][r] = -INFINITY;
        mx = fmaxf(mx, st[u][r]);
      }
    mx = xor32_max(xor16_max(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = st[u][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st[u][r] - mn);
        st[u][r] = p;
        ps += p;
      }
    ps = xor32_sum(xor16_sum(ps));
    l = l * alpha + ps;
#pragma unroll
    for (int i = 0; i < HD / 16; ++i) o[i] *= alpha;
    // O^T[dim][query] += V^T P^T: step r of sub-tile u covers positions
    // 16 u + 4 r + (0..3); lane l supplies V[16 u + 4 r + g][16 i + li] and
    // P[query li][16 u + 4 r + g] = st[u][r]
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pj = 16 * u + 4 * r + g;
#pragma unroll
        for (int i = 0; i < HD / 16; ++i) o[i] = mfma16x4(Vs[pj * VP + 16 * i + li], st[u][r], o[i]);
      }
  }
  // O^T tile i, register r: dim 16 i + 4 g + r of query li
  if (live && tq < A.T) {
    pf_attn_store<HD>(o, 1.0f / l, A.out, A.out16, (size_t)tq * A.n, (uint32_t)h * HD, g);
  }
}

// ------------------------------------------ split-f16 flash attention --
// k_pf_attn on v_mfma_f32_16x16x32_f16 (head_dim a multiple of 32): K, V, q
// and the probabilities split as hi + lo halves, each product as three
// MFMAs (hi hi, hi lo, lo hi; the lo lo term is below 2^-22 of the product),
// f32 accumulation.
//
// K and V come split already: k_pf_kv16 converts the layer's cached rows
// [0, R) once per chunk into a shadow -- per KV head, K as [position][hd]
// and V transposed in 64-position tiles, [tile][hd][64], hi and lo arrays,
// rows R .. next multiple of 64 zero -- so that a tile of either is one
// contiguous 16-byte-per-lane read, instead of every query block converting
// every tile it reads.  V^T's positions are permuted within each
// 32-position block: slot
// 8 g + 4 e + r holds position 16 e + 4 g + r (g < 4, e < 2, r < 4).  S^T
// sub-tile u (positions 16 u .. +15, natural K rows) leaves the scores of
// positions 16 u + 4 (l / 16) + r in register r of lane l, so over sub-tiles
// 2 b and 2 b + 1 lane l holds exactly slots 8 (l / 16) .. +7 of P^T's
// 32-position step b -- its B fragment for the P.V MFMA, whose A fragment
// (V^T in slot order) is one 16-byte LDS read.
struct PfKv16 {
  const float* kc;  // this layer's cache [ctx][kv_dim]
  const float* vc;
  uint16_t* kh;     // [n_head_kv][cap][hd]
  uint16_t* kl;
  uint16_t* vh;     // [n_head_kv][cap / 64][hd][64]
  uint16_t* vl;
  uint32_t R, kv_dim, hd, cap;
};

__device__ __forceinline__ void pf16_split(float v, _Float16& hi, _Float16& lo) {
  hi = (_Float16)v;
  lo = (_Float16)(v - (float)hi);
}

__device__ __forceinline__ uint32_t pf16_bits(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Block: 64 positions x 64 channels of K and V (grid: kv_dim / 64 rounded
// up, cap-rounded rows / 64).
__global__ __launch_bounds__(256) void k_pf_kv16(PfKv16 P) {
  __shared__ float Vt[64][65];  // [position][channel]
  const int tid = threadIdx.x;
  const uint32_t c0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int e = tid + 256 * it, r = e >> 4, q = e & 15;  // row r, channels 4 q .. + 3
    const uint32_t pos = j0 + r, ch = c0 + 4 * q;
    f4 k{0.f, 0.f, 0.f, 0.f}, v{0.f, 0.f, 0.f, 0.f};
    if (pos < P.R && ch < P.kv_dim) {
      k = *reinterpret_cast<const f4*>(P.kc + (size_t)pos * P.kv_dim + ch);
      v = *reinterpret_cast<const f4*>(P.vc + (size_t)pos * P.kv_dim + ch);
    }
    if (ch < P.kv_dim) {
      const size_t at = ((size_t)(ch / P.hd) * P.cap + pos) * P.hd + ch % P.hd;
      _Float16 h[4], l[4];
      pf16_split(k.x, h[0], l[0]);
      pf16_split(k.y, h[1], l[1]);
      pf16_split(k.z, h[2], l[2]);
      pf16_split(k.w, h[3], l[3]);
      *reinterpret_cast<uint2*>(P.kh + at) = uint2{pf16_bits(h[0], h[1]), pf16_bits(h[2], h[3])};
      *reinterpret_cast<uint2*>(P.kl + at) = uint2{pf16_bits(l[0], l[1]), pf16_bits(l[2], l[3])};
    }
    Vt[r][4 * q] = v.x;
    Vt[r][4 * q + 1] = v.y;
    Vt[r][4 * q + 2] = v.z;
    Vt[r][4 * q + 3] = v.w;
  }
  __syncthreads();
  // V^T: channel tid / 4, slots 16 (tid % 4) .. + 15 of the 64-position tile
  const int cc = tid >> 2, piece = tid & 3;
  if (c0 + cc >= P.kv_dim) return;
  uint32_t hw[8], lw[8];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    _Float16 h[2], l[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const int k = 16 * piece + i + w;                                       // slot
      const int p = (k & 32) | (16 * ((k >> 2) & 1) + 4 * ((k >> 3) & 3) + (k & 3));  // its position
      pf16_split(Vt[p][cc], h[w], l[w]);
    }
    hw[i / 2] = pf16_bits(h[0], h[1]);
    lw[i / 2] = pf16_bits(l[0], l[1]);
  }
  const uint32_t ch = c0 + cc;
  const size_t at = (((size_t)(ch / P.hd) * (P.cap / 64) + j0 / 64) * P.hd + ch % P.hd) * 64 + 16 * piece;
  uint4* dh = reinterpret_cast<uint4*>(P.vh + at);
  uint4* dl = reinterpret_cast<uint4*>(P.vl + at);
  dh[0] = uint4{hw[0], hw[1], hw[2], hw[3]};
  dh[1] = uint4{hw[4], hw[5], hw[6], hw[7]};
  dl[0] = uint4{lw[0], lw[1], lw[2], lw[3]};
  dl[1] = uint4{lw[4], lw[5], lw[6], lw[7]};
}

struct PfAttn16 {
  const float* Q;      // [T][n] (rotated)
  const uint16_t* kh;  // k_pf_kv16's shadow of this layer's rows
  const uint16_t* kl;
  const uint16_t* vh;
  const uint16_t* vl;
  float* out;          // [T][n]
  uint16_t* out16;     // with it, out in the split-f16 GEMM's interleaved halves too (or null)
  uint32_t T, p0, n, group, cap;
  float scale;         // 1 / sqrt(hd)
};

// NT threads (one wave per q head of the group, 4 or 8 waves); the K and V
// tile for positions j0 .. j0 + 63 (hi and lo) is fetched as 16-byte pieces
// into registers one tile ahead of the tile being computed, then written to
// LDS between two block syncs.  At most 256 registers per lane, so that two
// waves share each SIMD (two 4-wave blocks per CU: 13.8k against 12.4k
// tok/s at the 7B shape's 16k prompt, where the unbounded build took 259).
template <int HD, int NT, int QG = 1>
__global__ __launch_bounds__(NT, 2) void k_pf_attn16(PfAttn16 A) {
  static_assert(HD % 32 == 0 && (16 * HD) % NT == 0, "head_dim a multiple of 32");
  constexpr int WPQ = NT / 64 / QG;   // waves per group of 16 queries
  constexpr int KP = HD + 8;          // K halves pitch (conflict-free row reads)
  constexpr int VP = PF_ATT_KT + 8;   // V^T halves pitch
  constexpr int PC = 16 * HD / NT;    // 16-byte pieces per thread, each of K and V
  extern __shared__ float sm[];
  _Float16* Kh = reinterpret_cast<_Float16*>(sm);
  _Float16* Kl = Kh + PF_ATT_KT * KP;
  _Float16* Vh = Kl + PF_ATT_KT * KP;  // [HD][VP]
  _Float16* Vl = Vh + HD * VP;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  // QG groups of 16 queries per block, each with one wave per q head (the
  // K/V tile in LDS serves QG times the matrix work)
  const int qg = wave / WPQ, hw = wave % WPQ;
  const uint32_t kvh = blockIdx.x, t0 = (gridDim.y - 1 - blockIdx.y) * (PF_ATT_Q * QG);
  const uint32_t h = kvh * A.group + (uint32_t)hw;
  const bool live = (uint32_t)hw < A.group;
  const uint32_t tq = t0 + PF_ATT_Q * qg + li;
  const int qpos = (int)(A.p0 + (tq < A.T ? tq : A.T - 1));
  constexpr float kLog2e = 1.4426950408889634f;
  // Q^T fragments of step s: Q[query li][32 s + 8 g .. +7], pre-scaled, split
  pfh8 qh[HD / 32], ql[HD / 32];
  {
    const float* qrow = A.Q + (size_t)(tq < A.T ? tq : A.T - 1) * A.n + (size_t)(live ? h : 0) * HD;
    const float sc = A.scale * kLog2e;
#pragma unroll
    for (int s = 0; s < HD / 32; ++s) {
      const f4 a = *reinterpret_cast<const f4*>(qrow + 32 * s + 8 * g);
      const f4 b = *reinterpret_cast<const f4*>(qrow + 32 * s + 8 * g + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        _Float16 hi, lo;
        pf16_split_product(v[i], sc, hi, lo);
        qh[s][i] = hi;
        ql[s][i] = lo;
      }
    }
  }
  pf4 o[HD / 16];
#pragma unroll
  for (int i = 0; i < HD / 16; ++i) o[i] = pf4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const int first = (int)(A.p0 + t0);  // the block's earliest query position
  const int last = (int)(A.p0 + min(t0 + PF_ATT_Q * QG, A.T) - 1);
  u4 kr[PC], vr[PC];
  // K piece e: array e / (8 HD) (hi, lo), position (e / (HD / 8)) % 64,
  // channels 8 (e % (HD / 8)) .. +7; V piece e: array e / (8 HD), channel
  // (e / 8) % HD, slots 8 (e % 8) .. +7.
  auto fetch = [&](int j0) {
#pragma unroll
    for (int c = 0; c < PC; ++c) {
      const int e = tid + NT * c, hl = e / (8 * HD), r = e % (8 * HD);
      const int pj = r / (HD / 8), ck = r % (HD / 8);
      const uint16_t* src = hl ? A.kl : A.kh;
      kr[c] = *reinterpret_cast<const u4*>(src + ((size_t)kvh * A.cap + j0 + pj) * HD + 8 * ck);
      const int d = r / 8, cv = r % 8;
      const uint16_t* vsrc = hl ? A.vl : A.vh;
      vr[c] = *reinterpret_cast<const u4*>(vsrc + (((size_t)kvh * (A.cap / 64) + j0 / 64) * HD + d) * 64 + 8 * cv);
    }
  };
  auto put = [&]() {
#pragma unroll
    for (int c = 0; c < PC; ++c) {
      const int e = tid + NT * c, hl = e / (8 * HD), r = e % (8 * HD);
      const int pj = r / (HD / 8), ck = r % (HD / 8);
      *reinterpret_cast<u4*>((hl ? Kl : Kh) + pj * KP + 8 * ck) = kr[c];
      const int d = r / 8, cv = r % 8;
      *reinterpret_cast<u4*>((hl ? Vl : Vh) + d * VP + 8 * cv) = vr[c];
    }
  };
  fetch(0);
  for (int j0 = 0; j0 <= last; j0 += PF_ATT_KT) {
    __syncthreads();
    put();
    __syncthreads();
    fetch(j0 + PF_ATT_KT <= last ? j0 + PF_ATT_KT : j0);
    if (!live) continue;
    pf4 st[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      st[u] = pf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < HD / 32; ++s) {
        const pfh8 kh = *reinterpret_cast<const pfh8*>(Kh + (16 * u + li) * KP + 32 * s + 8 * g);
        const pfh8 kl = *reinterpret_cast<const pfh8*>(Kl + (16 * u + li) * KP + 32 * s + 8 * g);
        st[u] = mfma16x32h(kh, qh[s], st[u]);
        st[u] = mfma16x32h(kh, ql[s], st[u]);
        st[u] = mfma16x32h(kl, qh[s], st[u]);
      }
    }
    // register r of sub-tile u: position j0 + 16 u + 4 g + r; only a tile
    // reaching past the block's earliest query holds positions to mask
    if (j0 + PF_ATT_KT - 1 > first) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (j0 + 16 * u + 4 * g + r > qpos) st[u][r] = -INFINITY;
    }
    // Position 0 is in every query's first tile, so m is finite from then on
    // and exp2 of a masked score is 0.
    float mx = st[0][0];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[u][r]);
    mx = xor32_max(xor16_max(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(st[u][r] - mn);
        st[u][r] = pv;
        ps += pv;
      }
    ps = xor32_sum(xor16_sum(ps));
    l = l * alpha + ps;
#pragma unroll
    for (int i = 0; i < HD / 16; ++i) o[i] *= alpha;
    // O^T[dim][query] += V^T P^T over the two 32-position steps
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      pfh8 ph, pl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        _Float16 hi, lo;
        pf16_split(st[2 * b + (i >> 2)][i & 3], hi, lo);
        ph[i] = hi;
        pl[i] = lo;
      }
#pragma unroll
      for (int i = 0; i < HD / 16; ++i) {
        const pfh8 vh = *reinterpret_cast<const pfh8*>(Vh + (16 * i + li) * VP + 32 * b + 8 * g);
        const pfh8 vl = *reinterpret_cast<const pfh8*>(Vl + (16 * i + li) * VP + 32 * b + 8 * g);
        o[i] = mfma16x32h(vh, ph, o[i]);
        o[i] = mfma16x32h(vh, pl, o[i]);
        o[i] = mfma16x32h(vl, ph, o[i]);
      }
    }
  }
  if (live && tq < A.T) {
    pf_attn_store<HD>(o, 1.0f / l, A.out, A.out16, (size_t)tq * A.n, (uint32_t)h * HD, g);
  }
}

static inline size_t pf_attn16_lds_bytes(uint32_t hd) {
  return ((size_t)PF_ATT_KT * (hd + 8) * 2 + (size_t)hd * (PF_ATT_KT + 8) * 2) * 2;
}
