/*
 * talos_oracle.c -- plain-C restatement of Talos's CPU decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend and the CPU
 * baseline.  The product library never links it.  Build flags (Makefile):
 * -O2 -ffp-contract=off -fno-fast-math -fopenmp, so every multiply and add
 * rounds separately, as Rust's non-FMA x86-64 build does.
 *
 * Reference files restated (Tsuskov/talos):
 *   src/gguf/dtype.rs     block formats and dequantize
 *   src/gguf/reader.rs    GGUF v3 parse, tensor_raw / tensor_f32
 *   src/math/matmul.rs    8-lane dot, row-parallel matvec
 *   src/math/quant.rs     per-block dequant + dot, row-parallel
 *   src/math/ops.rs       rmsnorm, softmax, silu, swiglu, rope
 *   src/model/config.rs   hyper-parameters from llama.* metadata
 *   src/model/weights.rs  tensor names and shapes
 *   src/model/llama.rs    forward / forward_hidden
 *   src/kv_cache.rs       per-layer append-only K/V rows
 *   src/sample.rs         argmax (ties -> last index)
 *
 * Bit-level notes (what the reference's third-party crates decide and this
 * file cannot pin without running Rust): `wide::f32x8::mul_add` is taken as
 * an unfused multiply then add (x86-64 default target has no FMA), and
 * `reduce_add` as a left-to-right sum of the eight lanes.  Parity against the
 * GPU is to tolerance, which these choices are far inside.
 */
#include "talos_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void seterr(char *err, size_t errlen, const char *fmt, ...) {
  if (!err || !errlen) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

/* ------------------------------------------------------------------ f16 -- */

float tor_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      float v = (float)man * 5.9604644775390625e-8f; /* man * 2^-24, exact */
      return sign ? -v : v;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t tor_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0));
  int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m24 = man | 0x800000u;
    int shift = 14 - e;
    uint32_t hm = m24 >> shift;
    uint32_t rem = m24 & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------ dtype.rs:30-121 formats -- */

int tor_type_supported(uint32_t tag) {
  return tag == TOR_F32 || tag == TOR_Q4_0 || tag == TOR_Q8_0 || tag == TOR_Q6_K;
}

size_t tor_block_elems(int type) { /* dtype.rs:44-50 */
  switch (type) {
    case TOR_F32: return 1;
    case TOR_Q8_0:
    case TOR_Q4_0: return 32;
    case TOR_Q6_K: return 256;
  }
  return 0;
}

size_t tor_block_bytes(int type) { /* dtype.rs:53-60 */
  switch (type) {
    case TOR_F32: return 4;
    case TOR_Q8_0: return 34;
    case TOR_Q4_0: return 18;
    case TOR_Q6_K: return 210;
  }
  return 0;
}

/* dtype.rs:64-121 */
void tor_dequantize(int type, const uint8_t *raw, float *out, size_t n) {
  switch (type) {
    case TOR_F32:
      memcpy(out, raw, n * 4);
      return;
    case TOR_Q8_0: /* dtype.rs:69-78 */
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t *b = raw + blk * 34;
        float d = tor_f16_to_f32(rd16(b));
        for (int j = 0; j < 32; ++j) out[blk * 32 + j] = d * (float)(int8_t)b[2 + j];
      }
      return;
    case TOR_Q4_0: /* dtype.rs:79-92 */
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t *b = raw + blk * 18;
        float d = tor_f16_to_f32(rd16(b));
        const uint8_t *qs = b + 2;
        float *chunk = out + blk * 32;
        for (int j = 0; j < 16; ++j) {
          int lo = (int)(qs[j] & 0x0F) - 8;
          int hi = (int)(qs[j] >> 4) - 8;
          chunk[j] = d * (float)lo;
          chunk[j + 16] = d * (float)hi;
        }
      }
      return;
    case TOR_Q6_K: /* dtype.rs:93-118 */
      for (size_t sb = 0; sb < n / 256; ++sb) {
        const uint8_t *b = raw + sb * 210;
        float d = tor_f16_to_f32(rd16(b + 208));
        for (int h = 0; h < 2; ++h) {
          const uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
          const int8_t *sc = (const int8_t *)(b + 192 + h * 8);
          float *y = out + sb * 256 + h * 128;
          for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 0x03) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 0x03) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
          }
        }
      }
      return;
  }
}

/* -------------------------------------------------------- quantizers -- */

/* src/math/metal/mod.rs:553-561 (quant_q8_0). */
void tor_quantize_q8_0(const float *x, uint8_t *out, size_t n) {
  for (size_t blk = 0; blk < n / 32; ++blk) {
    const float *v = x + blk * 32;
    uint8_t *o = out + blk * 34;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    float d = amax / 127.0f;
    uint16_t dh = tor_f32_to_f16(d);
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; ++j) {
      float q = 0.0f;
      if (d != 0.0f) {
        q = roundf(v[j] / d);
        if (q < -128.0f) q = -128.0f;
        if (q > 127.0f) q = 127.0f;
      }
      o[2 + j] = (uint8_t)(int8_t)q;
    }
  }
}

/* src/math/metal/mod.rs:564-574 (quant_q4_0). */
void tor_quantize_q4_0(const float *x, uint8_t *out, size_t n) {
  for (size_t blk = 0; blk < n / 32; ++blk) {
    const float *v = x + blk * 32;
    uint8_t *o = out + blk * 18;
    float max = 0.0f;
    for (int j = 0; j < 32; ++j)
      if (fabsf(v[j]) > fabsf(max)) max = v[j];
    float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = tor_f32_to_f16(d);
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 16; ++j) {
      int xi0 = (int)truncf(v[j] * id + 8.5f);
      int xi1 = (int)truncf(v[j + 16] * id + 8.5f);
      xi0 = xi0 < 0 ? 0 : (xi0 > 15 ? 15 : xi0);
      xi1 = xi1 < 0 ? 0 : (xi1 > 15 ? 15 : xi1);
      o[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
  }
}

/* Q6_K quantizer (the build's own; the reference only decodes Q6_K).
 * Sub-block j of 16 elements (element e belongs to j = e/16, which is the
 * sub-scale index dtype.rs:107-115 reads for it): s_j = signed max / -32.
 * Super scale d = signed max of s_j / -128, stored f16; sub-scale codes
 * sc_j = round(s_j / d) in [-128, 127]; elements re-quantized against the
 * decoded scale d16*sc_j, q = round(v / (d16*sc_j)) in [-32, 31], stored as
 * q+32 in the ql/qh bit layout of dtype.rs:103-116. */
void tor_quantize_q6_k(const float *x, uint8_t *out, size_t n) {
  for (size_t sb = 0; sb < n / 256; ++sb) {
    const float *v = x + sb * 256;
    uint8_t *b = out + sb * 210;
    float s[16];
    for (int j = 0; j < 16; ++j) {
      float m = 0.0f;
      for (int e = 0; e < 16; ++e)
        if (fabsf(v[j * 16 + e]) > fabsf(m)) m = v[j * 16 + e];
      s[j] = m / -32.0f;
    }
    float smax = 0.0f;
    for (int j = 0; j < 16; ++j)
      if (fabsf(s[j]) > fabsf(smax)) smax = s[j];
    float d = smax / -128.0f;
    uint16_t dh = tor_f32_to_f16(d);
    float d16 = tor_f16_to_f32(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; ++j) {
      float c = d16 != 0.0f ? roundf(s[j] / d16) : 0.0f;
      if (c < -128.0f) c = -128.0f;
      if (c > 127.0f) c = 127.0f;
      sc[j] = (int8_t)c;
    }
    uint8_t q[256];
    for (int e = 0; e < 256; ++e) {
      float es = d16 * (float)sc[e / 16];
      float qq = es != 0.0f ? roundf(v[e] / es) : 0.0f;
      if (qq < -32.0f) qq = -32.0f;
      if (qq > 31.0f) qq = 31.0f;
      q[e] = (uint8_t)((int)qq + 32);
    }
    memset(b, 0, 210);
    for (int h = 0; h < 2; ++h) {
      uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
      const uint8_t *qq = q + h * 128;
      for (int l = 0; l < 32; ++l) {
        ql[l] = (uint8_t)((qq[l] & 0xF) | ((qq[l + 64] & 0xF) << 4));
        ql[l + 32] = (uint8_t)((qq[l + 32] & 0xF) | ((qq[l + 96] & 0xF) << 4));
        qh[l] = (uint8_t)((qq[l] >> 4) | ((qq[l + 32] >> 4) << 2) |
                          ((qq[l + 64] >> 4) << 4) | ((qq[l + 96] >> 4) << 6));
      }
    }
    for (int j = 0; j < 16; ++j) b[192 + j] = (uint8_t)sc[j];
    b[208] = (uint8_t)(dh & 0xFF);
    b[209] = (uint8_t)(dh >> 8);
  }
}

/* --------------------------------------------------------------- math -- */

/* src/math/matmul.rs:15-30: eight accumulators, lane j takes k = j mod 8,
 * acc = a*b + acc, then the lanes are summed, then the scalar tail. */
float tor_dot(const float *a, const float *b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t n8 = n / 8 * 8;
  for (size_t i = 0; i < n8; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] = a[i + j] * b[i + j] + acc[j];
  float sum = 0.0f;
  for (int j = 0; j < 8; ++j) sum += acc[j];
  for (size_t i = n8; i < n; ++i) sum += a[i] * b[i];
  return sum;
}

/* src/math/matmul.rs:34-47: out[m] = dot(row m, x), parallel over rows. */
void tor_matvec_f32(const float *w, const float *x, float *out, size_t rows,
                    size_t cols, int nthreads) {
  long r;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (r = 0; r < (long)rows; ++r) out[r] = tor_dot(w + (size_t)r * cols, x, cols);
}

/* src/math/quant.rs:18-51: per row, dequantize one block into a stack
 * buffer, dot it with x's block, sum serially over blocks. */
void tor_matvec_quant(const uint8_t *bytes, int type, const float *x,
                      float *out, size_t rows, size_t cols, int nthreads) {
  if (type == TOR_F32) {
    tor_matvec_f32((const float *)bytes, x, out, rows, cols, nthreads);
    return;
  }
  size_t be = tor_block_elems(type), bb = tor_block_bytes(type);
  size_t row_bytes = cols / be * bb;
  long r;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (r = 0; r < (long)rows; ++r) {
    const uint8_t *row = bytes + (size_t)r * row_bytes;
    float buf[256];
    float sum = 0.0f;
    for (size_t blk = 0; blk < cols / be; ++blk) {
      tor_dequantize(type, row + blk * bb, buf, be);
      sum += tor_dot(buf, x + blk * be, be);
    }
    out[r] = sum;
  }
}

/* src/math/ops.rs:5-12 */
void tor_rmsnorm(const float *x, const float *w, float eps, float *out,
                 size_t n) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
  float mean_sq = ss / (float)n;
  float scale = 1.0f / sqrtf(mean_sq + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* src/math/ops.rs:15-25 */
void tor_softmax(float *x, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - max);
    sum += x[i];
  }
  for (size_t i = 0; i < n; ++i) x[i] /= sum;
}

/* src/math/ops.rs:28-30 */
float tor_silu(float x) { return x / (1.0f + expf(-x)); }

/* src/math/ops.rs:33-37 */
void tor_swiglu(const float *gate, const float *up, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = tor_silu(gate[i]) * up[i];
}

/* src/math/ops.rs:48-61: interleaved pairs (2i, 2i+1) within each head,
 * theta = pos * base^(-2i/head_dim) in f32 via powf, then sinf/cosf. */
void tor_rope(float *v, size_t pos, size_t n_head, size_t head_dim,
              float freq_base) {
  size_t half = head_dim / 2;
  for (size_t h = 0; h < n_head; ++h) {
    size_t base = h * head_dim;
    for (size_t i = 0; i < half; ++i) {
      float expo = (-2.0f * (float)i) / (float)head_dim;
      float theta = (float)pos * powf(freq_base, expo);
      float s = sinf(theta), c = cosf(theta);
      float a = v[base + 2 * i], b = v[base + 2 * i + 1];
      v[base + 2 * i] = a * c - b * s;
      v[base + 2 * i + 1] = a * s + b * c;
    }
  }
}

/* src/sample.rs:7-14: max by f32::total_cmp; Iterator::max_by returns the
 * last of equal maxima. */
static inline int32_t total_key(float f) {
  int32_t i;
  memcpy(&i, &f, 4);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}
uint32_t tor_argmax(const float *logits, size_t n) {
  uint32_t best = 0;
  int32_t bk = total_key(logits[0]);
  for (size_t i = 1; i < n; ++i) {
    int32_t k = total_key(logits[i]);
    if (k >= bk) {
      bk = k;
      best = (uint32_t)i;
    }
  }
  return best;
}

/* ------------------------------------------------ sample.rs:19-76 -- */

typedef struct {
  int32_t key;
  uint32_t idx;
} tor_rank;

/* descending total_cmp; equal logits in descending index order (the
 * reference's sort_unstable_by leaves the order of equal logits open; this
 * order makes top-1 the argmax, whose ties go to the last index). */
static int cmp_desc(const void *a, const void *b) {
  const tor_rank *x = (const tor_rank *)a, *y = (const tor_rank *)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx > y->idx ? -1 : (x->idx < y->idx ? 1 : 0);
}

/* sample(logits, temperature, top_k, top_p, rng) with the draw
 * rng.gen::<f32>() passed in as `u` (in [0, 1)); top_k == 0 is None,
 * has_top_p == 0 is None.  Every step in f32, sums sequential, as the
 * reference. */
uint32_t tor_sample(const float *logits, size_t n, float temperature, size_t top_k, int has_top_p, float top_p,
                    float u) {
  if (temperature <= 0.0f) return tor_argmax(logits, n);
  tor_rank *idx = (tor_rank *)malloc(n * sizeof(tor_rank));
  float *probs = (float *)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; ++i) {
    idx[i].key = total_key(logits[i]);
    idx[i].idx = (uint32_t)i;
  }
  qsort(idx, n, sizeof(tor_rank), cmp_desc);
  size_t keep = top_k == 0 ? n : (top_k < 1 ? 1 : (top_k > n ? n : top_k));
  const float maxv = logits[idx[0].idx];
  float sum = 0.0f;
  for (size_t j = 0; j < keep; ++j) {
    probs[j] = expf((logits[idx[j].idx] - maxv) / temperature);
  }
  for (size_t j = 0; j < keep; ++j) sum += probs[j];
  for (size_t j = 0; j < keep; ++j) probs[j] /= sum;
  size_t cutoff = keep;
  if (has_top_p) {
    float c = 0.0f;
    for (size_t j = 0; j < keep; ++j) {
      c += probs[j];
      if (c >= top_p) {
        cutoff = j + 1;
        break;
      }
    }
  }
  float total = 0.0f;
  for (size_t j = 0; j < cutoff; ++j) total += probs[j];
  const float r = u * total;
  float acc = 0.0f;
  uint32_t out = idx[cutoff - 1].idx;
  for (size_t j = 0; j < cutoff; ++j) {
    acc += probs[j];
    if (acc >= r) {
      out = idx[j].idx;
      break;
    }
  }
  free(idx);
  free(probs);
  return out;
}

/* ---------------------------------------------------- eval.rs:17-22 -- */

/* -log softmax(logits)[target]: the max in f32 (f32::max fold), exp of
 * each (l - max) taken in f64 and summed in f64, the result cast to f32. */
float tor_token_nll(const float *logits, size_t n, uint32_t target) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, logits[i]);
  double sumexp = 0.0;
  for (size_t i = 0; i < n; ++i) sumexp += exp((double)(logits[i] - mx));
  const double log_prob = (double)(logits[target] - mx) - log(sumexp);
  return (float)(-log_prob);
}

/* ------------------------------------------- GGUF, reader.rs:193-351 -- */

enum { GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7, GT_STR = 8, GT_ARR = 9 };

typedef struct {
  char *key;
  uint32_t tag;     /* scalar tag, or GT_ARR */
  uint32_t inner;   /* array element tag */
  uint64_t count;   /* array length */
  uint32_t u32;
  float f32;
  int b;
  char *str;
} tor_kv;

typedef struct {
  char *name;
  uint32_t n_dims;
  uint64_t dims[4];
  uint32_t type;
  uint64_t offset;
} tor_tinfo;

struct tor_gguf {
  const uint8_t *bytes;
  size_t len;
  tor_kv *kv;
  size_t n_kv;
  tor_tinfo *t;
  size_t n_t;
  size_t data_start;
};

typedef struct {
  const uint8_t *b;
  size_t len, pos;
  int bad;
} cur_t;

static const uint8_t *take(cur_t *c, size_t n) {
  if (c->bad || n > c->len - c->pos) {
    c->bad = 1;
    return NULL;
  }
  const uint8_t *p = c->b + c->pos;
  c->pos += n;
  return p;
}
static uint32_t cu32(cur_t *c) {
  const uint8_t *p = take(c, 4);
  uint32_t v = 0;
  if (p) memcpy(&v, p, 4);
  return v;
}
static uint64_t cu64(cur_t *c) {
  const uint8_t *p = take(c, 8);
  uint64_t v = 0;
  if (p) memcpy(&v, p, 8);
  return v;
}
static char *cstr(cur_t *c) {
  uint64_t n = cu64(c);
  if (c->bad || n > c->len - c->pos) {
    c->bad = 1;
    return NULL;
  }
  const uint8_t *p = take(c, (size_t)n);
  char *s = (char *)malloc((size_t)n + 1);
  memcpy(s, p, (size_t)n);
  s[n] = 0;
  return s;
}

void tor_gguf_free(tor_gguf *g) {
  if (!g) return;
  for (size_t i = 0; i < g->n_kv; ++i) {
    free(g->kv[i].key);
    free(g->kv[i].str);
  }
  for (size_t i = 0; i < g->n_t; ++i) free(g->t[i].name);
  free(g->kv);
  free(g->t);
  free(g);
}

tor_gguf *tor_gguf_parse(const uint8_t *bytes, size_t len, char *err,
                         size_t errlen) {
  cur_t c = {bytes, len, 0, 0};
  const uint8_t *magic = take(&c, 4);
  if (!magic || memcmp(magic, "GGUF", 4) != 0) {
    seterr(err, errlen, "not a GGUF file (bad magic)");
    return NULL;
  }
  uint32_t version = cu32(&c);
  if (c.bad) goto trunc0;
  if (version != 3) {
    seterr(err, errlen, "unsupported GGUF version %u (expected 3)", version);
    return NULL;
  }
  uint64_t n_t = cu64(&c), n_kv = cu64(&c);
  if (c.bad) goto trunc0;
  if (n_kv > len || n_t > len) goto trunc0;
  tor_gguf *g = (tor_gguf *)calloc(1, sizeof(tor_gguf));
  g->bytes = bytes;
  g->len = len;
  g->kv = (tor_kv *)calloc(n_kv ? n_kv : 1, sizeof(tor_kv));
  g->t = (tor_tinfo *)calloc(n_t ? n_t : 1, sizeof(tor_tinfo));
  for (uint64_t i = 0; i < n_kv; ++i) {
    tor_kv *kv = &g->kv[g->n_kv++];
    kv->key = cstr(&c);
    kv->tag = cu32(&c);
    if (c.bad) goto trunc;
    switch (kv->tag) { /* reader.rs:135-171 */
      case GT_U32: kv->u32 = cu32(&c); break;
      case GT_F32: {
        uint32_t v = cu32(&c);
        memcpy(&kv->f32, &v, 4);
        break;
      }
      case GT_BOOL: {
        const uint8_t *p = take(&c, 1);
        kv->b = p ? p[0] != 0 : 0;
        break;
      }
      case GT_STR: kv->str = cstr(&c); break;
      case GT_ARR: {
        kv->inner = cu32(&c);
        kv->count = cu64(&c);
        if (c.bad) goto trunc;
        if (kv->inner == GT_STR) {
          for (uint64_t k = 0; k < kv->count && !c.bad; ++k) free(cstr(&c));
        } else if (kv->inner == GT_I32 || kv->inner == GT_F32) {
          if (kv->count > (len - c.pos) / 4) goto trunc;
          take(&c, (size_t)kv->count * 4);
        } else {
          seterr(err, errlen, "reading metadata key \"%s\": unsupported array element type tag %u",
                 kv->key, kv->inner);
          tor_gguf_free(g);
          return NULL;
        }
        break;
      }
      default:
        seterr(err, errlen, "reading metadata key \"%s\": unsupported metadata value type tag %u",
               kv->key, kv->tag);
        tor_gguf_free(g);
        return NULL;
    }
    if (c.bad) goto trunc;
  }
  for (uint64_t i = 0; i < n_t; ++i) { /* reader.rs:218-231 */
    tor_tinfo *t = &g->t[g->n_t++];
    t->name = cstr(&c);
    t->n_dims = cu32(&c);
    if (c.bad) goto trunc;
    if (t->n_dims > 4) {
      seterr(err, errlen, "tensor \"%s\" has %u dims (max 4)", t->name, t->n_dims);
      tor_gguf_free(g);
      return NULL;
    }
    for (uint32_t d = 0; d < t->n_dims; ++d) t->dims[d] = cu64(&c);
    t->type = cu32(&c);
    if (c.bad) goto trunc;
    if (!tor_type_supported(t->type)) {
      seterr(err, errlen, "tensor \"%s\" has unsupported ggml type %u", t->name, t->type);
      tor_gguf_free(g);
      return NULL;
    }
    t->offset = cu64(&c);
    if (c.bad) goto trunc;
  }
  g->data_start = (c.pos + 31) / 32 * 32; /* reader.rs:234-237 */
  if (g->data_start > len) {
    seterr(err, errlen, "data section start %zu past end of file %zu", g->data_start, len);
    tor_gguf_free(g);
    return NULL;
  }
  return g;
trunc:
  tor_gguf_free(g);
trunc0:
  seterr(err, errlen, "unexpected end of file");
  return NULL;
}

static const tor_kv *find_kv(const tor_gguf *g, const char *key) {
  /* Later duplicates win, as HashMap::insert does. */
  for (size_t i = g->n_kv; i-- > 0;)
    if (strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
  return NULL;
}
int tor_gguf_get_u32(const tor_gguf *g, const char *key, uint32_t *out) {
  const tor_kv *kv = find_kv(g, key);
  if (!kv || kv->tag != GT_U32) return 0;
  *out = kv->u32;
  return 1;
}
int tor_gguf_get_f32(const tor_gguf *g, const char *key, float *out) {
  const tor_kv *kv = find_kv(g, key);
  if (!kv || kv->tag != GT_F32) return 0;
  *out = kv->f32;
  return 1;
}
const char *tor_gguf_get_str(const tor_gguf *g, const char *key) {
  const tor_kv *kv = find_kv(g, key);
  return kv && kv->tag == GT_STR ? kv->str : NULL;
}
long tor_gguf_arr_str_len(const tor_gguf *g, const char *key) {
  const tor_kv *kv = find_kv(g, key);
  return kv && kv->tag == GT_ARR && kv->inner == GT_STR ? (long)kv->count : -1;
}
size_t tor_gguf_tensor_count(const tor_gguf *g) { return g->n_t; }
int tor_gguf_tensor_info(const tor_gguf *g, size_t i, const char **name,
                         uint32_t *n_dims, uint64_t *dims, uint32_t *type,
                         uint64_t *offset) {
  if (i >= g->n_t) return -1;
  const tor_tinfo *t = &g->t[i];
  *name = t->name;
  *n_dims = t->n_dims;
  for (int d = 0; d < 4; ++d) dims[d] = d < (int)t->n_dims ? t->dims[d] : 0;
  *type = t->type;
  *offset = t->offset;
  return 0;
}

static const tor_tinfo *find_t(const tor_gguf *g, const char *name) {
  for (size_t i = g->n_t; i-- > 0;)
    if (strcmp(g->t[i].name, name) == 0) return &g->t[i];
  return NULL;
}

/* reader.rs:328-351 */
int tor_gguf_tensor_raw(const tor_gguf *g, const char *name,
                        const uint8_t **bytes, size_t *len, int *type,
                        char *err, size_t errlen) {
  const tor_tinfo *t = find_t(g, name);
  if (!t) {
    seterr(err, errlen, "no tensor named \"%s\"", name);
    return -1;
  }
  uint64_t elems = 1;
  for (uint32_t d = 0; d < t->n_dims; ++d) {
    if (t->dims[d] && elems > UINT64_MAX / t->dims[d]) {
      seterr(err, errlen, "tensor byte length overflow");
      return -1;
    }
    elems *= t->dims[d];
  }
  size_t blk = tor_block_elems((int)t->type);
  if (elems % blk) {
    seterr(err, errlen, "tensor \"%s\" has %llu elems, not a multiple of block %zu", name,
           (unsigned long long)elems, blk);
    return -1;
  }
  uint64_t blen = elems / blk * tor_block_bytes((int)t->type);
  uint64_t start = (uint64_t)g->data_start + t->offset;
  if (start < t->offset || start + blen < start || start + blen > g->len) {
    seterr(err, errlen, "tensor \"%s\" data range past end of file", name);
    return -1;
  }
  *bytes = g->bytes + start;
  *len = (size_t)blen;
  *type = (int)t->type;
  return 0;
}

/* ------------------------------------------------------------- model -- */

typedef struct {
  const uint8_t *bytes;
  int type;
  size_t rows, cols;
} qtensor;

typedef struct {
  const float *attn_norm, *ffn_norm;
  qtensor q, k, v, o, gate, up, down;
} layer_w;

struct tor_model {
  tor_gguf *g;
  tor_config cfg;
  qtensor token_embd, output;
  const float *output_norm;
  layer_w *layers;
  float **kc, **vc; /* per layer, [len][kv_dim] */
  size_t kv_len, kv_cap;
  int nthreads;
};

static int bind_q(tor_model *m, const char *name, size_t rows, size_t cols,
                  qtensor *out, char *err, size_t errlen) {
  const uint8_t *b;
  size_t len;
  int type;
  if (tor_gguf_tensor_raw(m->g, name, &b, &len, &type, err, errlen)) return -1;
  size_t be = tor_block_elems(type);
  if (cols % be || len != rows * (cols / be) * tor_block_bytes(type)) {
    seterr(err, errlen, "tensor \"%s\": %zu bytes do not hold [%zu, %zu] of type %d", name, len,
           rows, cols, type);
    return -1;
  }
  out->bytes = b;
  out->type = type;
  out->rows = rows;
  out->cols = cols;
  return 0;
}

/* reader.rs:302-324 (tensor_f32): must be F32; length checked against n. */
static int bind_f32(tor_model *m, const char *name, size_t n, const float **out,
                    char *err, size_t errlen) {
  const uint8_t *b;
  size_t len;
  int type;
  if (tor_gguf_tensor_raw(m->g, name, &b, &len, &type, err, errlen)) return -1;
  if (type != TOR_F32) {
    seterr(err, errlen, "tensor \"%s\" is type %d, not F32", name, type);
    return -1;
  }
  if (len != n * 4) {
    seterr(err, errlen, "tensor \"%s\" has %zu elems, expected %zu", name, len / 4, n);
    return -1;
  }
  *out = (const float *)b;
  return 0;
}

static void kv_alloc(tor_model *m, size_t cap) {
  size_t kvd = (size_t)m->cfg.n_head_kv * (m->cfg.n_embd / m->cfg.n_head);
  for (uint32_t l = 0; l < m->cfg.n_layer; ++l) {
    m->kc[l] = (float *)realloc(m->kc[l], (cap ? cap : 1) * kvd * 4);
    m->vc[l] = (float *)realloc(m->vc[l], (cap ? cap : 1) * kvd * 4);
  }
  m->kv_cap = cap;
}

void tor_model_free(tor_model *m) {
  if (!m) return;
  if (m->kc)
    for (uint32_t l = 0; l < m->cfg.n_layer; ++l) {
      free(m->kc[l]);
      free(m->vc[l]);
    }
  free(m->kc);
  free(m->vc);
  free(m->layers);
  tor_gguf_free(m->g);
  free(m);
}

/* llama.rs:43-62 + config.rs:40-67 + weights.rs:92-114 */
tor_model *tor_model_load(const uint8_t *bytes, size_t len, int nthreads,
                          char *err, size_t errlen) {
  tor_gguf *g = tor_gguf_parse(bytes, len, err, errlen);
  if (!g) return NULL;
  tor_model *m = (tor_model *)calloc(1, sizeof(tor_model));
  m->g = g;
  m->nthreads = nthreads > 0 ? nthreads : 1;
  const char *arch = tor_gguf_get_str(g, "general.architecture");
  if (!arch || strcmp(arch, "llama") != 0) {
    seterr(err, errlen, "unsupported architecture \"%s\" (expected \"llama\")", arch ? arch : "");
    goto fail;
  }
  tor_config *c = &m->cfg;
  struct {
    const char *k;
    uint32_t *dst;
  } req[] = {{"llama.block_count", &c->n_layer},
             {"llama.attention.head_count", &c->n_head},
             {"llama.attention.head_count_kv", &c->n_head_kv},
             {"llama.embedding_length", &c->n_embd},
             {"llama.feed_forward_length", &c->n_ff},
             {"llama.context_length", &c->context_length},
             {"llama.rope.dimension_count", &c->rope_dim}};
  long vocab = tor_gguf_arr_str_len(g, "tokenizer.ggml.tokens");
  if (vocab < 0) {
    seterr(err, errlen, "missing tokenizer.ggml.tokens (needed for vocab size)");
    goto fail;
  }
  c->vocab_size = (uint32_t)vocab;
  for (size_t i = 0; i < sizeof(req) / sizeof(req[0]); ++i)
    if (!tor_gguf_get_u32(g, req[i].k, req[i].dst)) {
      seterr(err, errlen, "missing metadata key %s", req[i].k);
      goto fail;
    }
  if (!tor_gguf_get_f32(g, "llama.attention.layer_norm_rms_epsilon", &c->rms_eps)) c->rms_eps = 1e-5f;
  if (!tor_gguf_get_f32(g, "llama.rope.freq_base", &c->rope_freq_base)) c->rope_freq_base = 10000.0f;
  if (c->n_head_kv == 0 || c->n_head == 0 || c->n_head % c->n_head_kv != 0) {
    seterr(err, errlen, "head_count %u must be a positive multiple of head_count_kv %u", c->n_head,
           c->n_head_kv);
    goto fail;
  }
  size_t cc = c->n_embd, ff = c->n_ff, v = c->vocab_size;
  size_t kvd = (size_t)c->n_head_kv * (c->n_embd / c->n_head);
  m->layers = (layer_w *)calloc(c->n_layer ? c->n_layer : 1, sizeof(layer_w));
  char nm[128];
  for (uint32_t l = 0; l < c->n_layer; ++l) {
    layer_w *lw = &m->layers[l];
#define NM(s) (snprintf(nm, sizeof nm, "blk.%u." s, l), nm)
    if (bind_f32(m, NM("attn_norm.weight"), cc, &lw->attn_norm, err, errlen) ||
        bind_q(m, NM("attn_q.weight"), cc, cc, &lw->q, err, errlen) ||
        bind_q(m, NM("attn_k.weight"), kvd, cc, &lw->k, err, errlen) ||
        bind_q(m, NM("attn_v.weight"), kvd, cc, &lw->v, err, errlen) ||
        bind_q(m, NM("attn_output.weight"), cc, cc, &lw->o, err, errlen) ||
        bind_f32(m, NM("ffn_norm.weight"), cc, &lw->ffn_norm, err, errlen) ||
        bind_q(m, NM("ffn_gate.weight"), ff, cc, &lw->gate, err, errlen) ||
        bind_q(m, NM("ffn_up.weight"), ff, cc, &lw->up, err, errlen) ||
        bind_q(m, NM("ffn_down.weight"), cc, ff, &lw->down, err, errlen))
      goto fail;
#undef NM
  }
  if (bind_q(m, "token_embd.weight", v, cc, &m->token_embd, err, errlen) ||
      bind_f32(m, "output_norm.weight", cc, &m->output_norm, err, errlen) ||
      bind_q(m, "output.weight", v, cc, &m->output, err, errlen))
    goto fail;
  m->kc = (float **)calloc(c->n_layer ? c->n_layer : 1, sizeof(float *));
  m->vc = (float **)calloc(c->n_layer ? c->n_layer : 1, sizeof(float *));
  kv_alloc(m, c->context_length);
  return m;
fail:
  tor_model_free(m);
  return NULL;
}

void tor_model_config(const tor_model *m, tor_config *out) { *out = m->cfg; }
void tor_model_set_threads(tor_model *m, int n) { m->nthreads = n > 0 ? n : 1; }

/* llama.rs:69-81: cap the context, rebuild a fresh empty cache. */
void tor_model_cap_context(tor_model *m, size_t max_ctx) {
  size_t c = m->cfg.context_length;
  size_t cap = max_ctx > 0 ? max_ctx : 1;
  m->cfg.context_length = (uint32_t)(c < cap ? c : cap);
  m->kv_len = 0;
  kv_alloc(m, m->cfg.context_length);
}

void tor_model_reset(tor_model *m) { m->kv_len = 0; } /* llama.rs:236-238 */
size_t tor_model_kv_len(const tor_model *m) { return m->kv_len; }

int tor_model_set_kv(tor_model *m, const float *k, const float *v, size_t len) {
  size_t kvd = (size_t)m->cfg.n_head_kv * (m->cfg.n_embd / m->cfg.n_head);
  if (len > m->kv_cap) kv_alloc(m, len);
  for (uint32_t l = 0; l < m->cfg.n_layer; ++l) {
    memcpy(m->kc[l], k + (size_t)l * len * kvd, len * kvd * 4);
    memcpy(m->vc[l], v + (size_t)l * len * kvd, len * kvd * 4);
  }
  m->kv_len = len;
  return 0;
}

int tor_model_get_kv(const tor_model *m, float *k, float *v, size_t len) {
  size_t kvd = (size_t)m->cfg.n_head_kv * (m->cfg.n_embd / m->cfg.n_head);
  if (len > m->kv_len) return -1;
  for (uint32_t l = 0; l < m->cfg.n_layer; ++l) {
    memcpy(k + (size_t)l * len * kvd, m->kc[l], len * kvd * 4);
    memcpy(v + (size_t)l * len * kvd, m->vc[l], len * kvd * 4);
  }
  return 0;
}

static void qmatvec(const tor_model *m, const qtensor *t, const float *x, float *out) {
  tor_matvec_quant(t->bytes, t->type, x, out, t->rows, t->cols, m->nthreads);
}

/* weights.rs:58-62 */
static void dequant_row(const qtensor *t, size_t r, float *out) {
  size_t be = tor_block_elems(t->type), bb = tor_block_bytes(t->type);
  size_t row_bytes = t->cols / be * bb;
  tor_dequantize(t->type, t->bytes + r * row_bytes, out, t->cols);
}

/* llama.rs:96-183 */
int tor_model_forward_hidden(tor_model *m, uint32_t token, size_t pos, float *hidden) {
  (void)pos; /* seq comes from the cache length, as KvCache::len */
  const tor_config *cfg = &m->cfg;
  if (token >= cfg->vocab_size) return -1;
  size_t c = cfg->n_embd, nh = cfg->n_head, nkv = cfg->n_head_kv;
  size_t hd = c / nh, kv_dim = nkv * hd, group = nh / nkv, f = cfg->n_ff;
  float eps = cfg->rms_eps;
  float scale = 1.0f / sqrtf((float)hd);
  if (m->kv_len + 1 > m->kv_cap) kv_alloc(m, m->kv_cap * 2 + 1);

  float *x = (float *)calloc(c, 4), *normed = (float *)calloc(c, 4);
  float *q = (float *)calloc(c, 4), *k = (float *)calloc(kv_dim, 4), *v = (float *)calloc(kv_dim, 4);
  float *atty = (float *)calloc(c, 4), *attproj = (float *)calloc(c, 4);
  float *gate = (float *)calloc(f, 4), *up = (float *)calloc(f, 4), *glu = (float *)calloc(f, 4);
  float *down = (float *)calloc(c, 4);
  float *scores = (float *)calloc(m->kv_len + 1, 4);

  dequant_row(&m->token_embd, token, x); /* llama.rs:112-113 */
  size_t seq = m->kv_len + 1;
  for (uint32_t l = 0; l < cfg->n_layer; ++l) {
    const layer_w *lw = &m->layers[l];
    tor_rmsnorm(x, lw->attn_norm, eps, normed, c);
    qmatvec(m, &lw->q, normed, q);
    qmatvec(m, &lw->k, normed, k);
    qmatvec(m, &lw->v, normed, v);
    tor_rope(q, pos, nh, hd, cfg->rope_freq_base);
    tor_rope(k, pos, nkv, hd, cfg->rope_freq_base);
    memcpy(m->kc[l] + m->kv_len * kv_dim, k, kv_dim * 4); /* kv_cache.rs:21-26 */
    memcpy(m->vc[l] + m->kv_len * kv_dim, v, kv_dim * 4);
    const float *keys = m->kc[l], *vals = m->vc[l];
    memset(atty, 0, c * 4);
    for (size_t h = 0; h < nh; ++h) { /* llama.rs:139-155 */
      size_t kvh = h / group;
      const float *qh = q + h * hd;
      for (size_t t = 0; t < seq; ++t) {
        const float *kh = keys + t * kv_dim + kvh * hd;
        float dot = 0.0f;
        for (size_t i = 0; i < hd; ++i) dot += qh[i] * kh[i];
        scores[t] = dot * scale;
      }
      tor_softmax(scores, seq);
      float *oh = atty + h * hd;
      for (size_t t = 0; t < seq; ++t) {
        const float *vh = vals + t * kv_dim + kvh * hd;
        float a = scores[t];
        for (size_t i = 0; i < hd; ++i) oh[i] += a * vh[i];
      }
    }
    qmatvec(m, &lw->o, atty, attproj);
    for (size_t i = 0; i < c; ++i) x[i] += attproj[i];
    tor_rmsnorm(x, lw->ffn_norm, eps, normed, c);
    qmatvec(m, &lw->gate, normed, gate);
    qmatvec(m, &lw->up, normed, up);
    tor_swiglu(gate, up, glu, f);
    qmatvec(m, &lw->down, glu, down);
    for (size_t i = 0; i < c; ++i) x[i] += down[i];
  }
  m->kv_len = seq;
  tor_rmsnorm(x, m->output_norm, eps, hidden, c);
  free(x); free(normed); free(q); free(k); free(v); free(atty); free(attproj);
  free(gate); free(up); free(glu); free(down); free(scores);
  return 0;
}

/* llama.rs:85-91 */
int tor_model_forward(tor_model *m, uint32_t token, size_t pos, float *logits) {
  float *xf = (float *)malloc(m->cfg.n_embd * 4);
  int rc = tor_model_forward_hidden(m, token, pos, xf);
  if (rc == 0) qmatvec(m, &m->output, xf, logits);
  free(xf);
  return rc;
}
