// layout.h -- device-resident weight layouts (shared by host repack code and
// the kernels).
//
// GGUF block formats (src/gguf/dtype.rs:1-9) are repacked once at upload into
// structure-of-arrays planes so that every lane of a 64-wide wavefront issues
// one 128-bit coalesced load per quant block and the f16 scales stream from a
// separate contiguous plane.  A "chunk" is the unit one lane consumes per
// K-step:
//
//   F32   chunk =  4 elements: q = float[rows][cols]
//   Q8_0  chunk = 32 elements: q = u8[rows][nblk][32] holding (int8 q) ^ 0x80,
//                              d = f16[rows][nblk]
//   Q4_0  chunk = 32 elements: q = u8[rows][nblk][16], the block's 16 packed
//                              bytes unchanged (low nibble -> j, high -> j+16),
//                              d = f16[rows][nblk]
//   Q6_K  chunk = 64 elements, a quarter super-block (half n, 16-group g):
//                              q  = u8[rows][3][nchunk][16]; plane 0 holds
//                                   ql[n*64+g*16 ..+16], plane 1 ql[n*64+32+
//                                   g*16 ..+16], plane 2 qh[n*32+g*16 ..+16];
//                              sc = u32[rows][nchunk], the four int8 sub-scales
//                                   sc[n*8+g+{0,2,4,6}] that chunk reads;
//                              d  = f16[rows][nchunk/4]
#pragma once
#include <stdint.h>

enum : uint32_t {
  TALOS_FMT_F32 = 0,
  TALOS_FMT_Q4_0 = 2,
  TALOS_FMT_Q8_0 = 8,
  TALOS_FMT_Q6_K = 14,
};

struct DevMat {
  const uint8_t* q;    // quant plane
  const uint16_t* d;   // f16 scales (Q8_0, Q4_0, Q6_K)
  const uint32_t* sc;  // Q6_K sub-scale words
  uint32_t rows, cols;
  uint32_t fmt;
  uint32_t nchunk;     // chunks per row
};

// Elements per lane chunk.
static inline __host__ __device__ uint32_t fmt_chunk_elems(uint32_t fmt) {
  return fmt == TALOS_FMT_F32 ? 4u : fmt == TALOS_FMT_Q6_K ? 64u : 32u;
}
// Quant-plane bytes per chunk.
static inline __host__ __device__ uint32_t fmt_chunk_qbytes(uint32_t fmt) {
  return fmt == TALOS_FMT_F32 ? 16u : fmt == TALOS_FMT_Q8_0 ? 32u : fmt == TALOS_FMT_Q4_0 ? 16u : 48u;
}
// LDS layout of x each format reads: 0 = 16-B pad per 32 floats, 1 = per 64.
static inline __host__ __device__ int fmt_xlayout(uint32_t fmt) {
  return fmt == TALOS_FMT_Q6_K ? 1 : 0;
}
