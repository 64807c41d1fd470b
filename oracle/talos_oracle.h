/*
 * talos_oracle.h -- CPU oracle for the Talos batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU forward pass (Tsuskov/talos, Rust).  It is the checker for the HIP
 * backend and the CPU baseline timed beside it.  Only tests/, the smoke check
 * and the CPU-baseline leg of bench.py may load it; the product library never
 * links or calls it.
 *
 * Every function cites the reference file:line it restates.  Arithmetic is
 * fp32 with no contraction (built with -ffp-contract=off), transcendental
 * calls go to glibc powf/sinf/cosf/expf/sqrtf as Rust's f32 methods do on
 * Linux.
 *
 * Pinning (tests/test_oracle_kat.py, tests/test_oracle_model.py): every
 * function is checked against the reference's own unit-test values, closed
 * forms, layout probes or brute force, and the composed forward against the
 * GQA == replicated-MHA invariant and an independent float64 forward.
 * Parity unpinned: bit-for-bit equality with the Rust CPU path.  tor_dot
 * takes matmul::dot's wide::f32x8 mul_add as unfused and its reduce_add as a
 * left-to-right sum of the 8 lanes; the `wide` crate is not available to
 * confirm either, so results agree with the reference to fp32 reordering
 * error, not to the bit.
 */
#ifndef TALOS_ORACLE_H
#define TALOS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type tags, src/gguf/dtype.rs:33-41. */
enum { TOR_F32 = 0, TOR_Q4_0 = 2, TOR_Q8_0 = 8, TOR_Q6_K = 14 };

/* ---- f16 (the `half` crate: f32 -> f16 is round-to-nearest-even) ---- */
float tor_f16_to_f32(uint16_t h);
uint16_t tor_f32_to_f16(float f);

/* ---- block formats, src/gguf/dtype.rs ---- */
int tor_type_supported(uint32_t tag);
size_t tor_block_elems(int type);
size_t tor_block_bytes(int type);
/* Dequantize n elements (n a multiple of the block size). */
void tor_dequantize(int type, const uint8_t *raw, float *out, size_t n);

/* ---- quantizers ----
 * Q8_0 / Q4_0 follow the reference's test quantizers
 * (src/math/metal/mod.rs:551-574, src/gguf/dtype.rs:132-167).
 * Q6_K: the reference has no quantizer; this one is the build's own
 * (per-16 signed-max sub-scales, int8 sub-scale codes, round to nearest). */
void tor_quantize_q8_0(const float *x, uint8_t *out, size_t n);
void tor_quantize_q4_0(const float *x, uint8_t *out, size_t n);
void tor_quantize_q6_k(const float *x, uint8_t *out, size_t n);

/* ---- math, src/math/{matmul,quant,ops}.rs ---- */
float tor_dot(const float *a, const float *b, size_t n);
void tor_matvec_f32(const float *w, const float *x, float *out, size_t rows,
                    size_t cols, int nthreads);
void tor_matvec_quant(const uint8_t *bytes, int type, const float *x,
                      float *out, size_t rows, size_t cols, int nthreads);
void tor_rmsnorm(const float *x, const float *w, float eps, float *out,
                 size_t n);
void tor_softmax(float *x, size_t n);
float tor_silu(float x);
void tor_swiglu(const float *gate, const float *up, float *out, size_t n);
void tor_rope(float *v, size_t pos, size_t n_head, size_t head_dim,
              float freq_base);
uint32_t tor_argmax(const float *logits, size_t n);
uint32_t tor_sample(const float *logits, size_t n, float temperature, size_t top_k, int has_top_p, float top_p,
                    float u);
float tor_token_nll(const float *logits, size_t n, uint32_t target);

/* ---- GGUF v3 parse, src/gguf/reader.rs:193-351 ---- */
typedef struct tor_gguf tor_gguf;
tor_gguf *tor_gguf_parse(const uint8_t *bytes, size_t len, char *err,
                         size_t errlen);
void tor_gguf_free(tor_gguf *g);
/* Returns 1 and fills *out when the key exists with the asked type. */
int tor_gguf_get_u32(const tor_gguf *g, const char *key, uint32_t *out);
int tor_gguf_get_f32(const tor_gguf *g, const char *key, float *out);
/* String value; returns NULL if missing or not a string. */
const char *tor_gguf_get_str(const tor_gguf *g, const char *key);
/* Length of an array-of-strings value, or -1. */
long tor_gguf_arr_str_len(const tor_gguf *g, const char *key);
size_t tor_gguf_tensor_count(const tor_gguf *g);
/* Tensor info by index: name, dims (ne order), type, offset. */
int tor_gguf_tensor_info(const tor_gguf *g, size_t i, const char **name,
                         uint32_t *n_dims, uint64_t *dims /*[4]*/,
                         uint32_t *type, uint64_t *offset);
/* Raw bytes of a tensor (tensor_raw); returns 0 on success. */
int tor_gguf_tensor_raw(const tor_gguf *g, const char *name,
                        const uint8_t **bytes, size_t *len, int *type,
                        char *err, size_t errlen);

/* ---- the model, src/model/{config,weights,llama}.rs + src/kv_cache.rs ---- */
typedef struct {
  uint32_t n_layer, n_head, n_head_kv, n_embd, n_ff;
  uint32_t context_length, vocab_size, rope_dim;
  float rms_eps, rope_freq_base;
} tor_config;

typedef struct tor_model tor_model;
/* The bytes must outlive the model (weights are views into them). */
tor_model *tor_model_load(const uint8_t *bytes, size_t len, int nthreads,
                          char *err, size_t errlen);
void tor_model_free(tor_model *m);
void tor_model_config(const tor_model *m, tor_config *out);
void tor_model_cap_context(tor_model *m, size_t max_ctx);
void tor_model_set_threads(tor_model *m, int nthreads);
/* Model::forward / forward_hidden: appends this step's K/V to the cache. */
int tor_model_forward(tor_model *m, uint32_t token, size_t pos, float *logits);
int tor_model_forward_hidden(tor_model *m, uint32_t token, size_t pos,
                             float *hidden);
void tor_model_reset(tor_model *m);
/* Cached positions (KvCache::len). */
size_t tor_model_kv_len(const tor_model *m);
/* Replace the cache with `len` positions of K and V for every layer,
 * laid out [layer][pos][kv_dim] -- used to start the oracle from a long
 * prefix the GPU filled. */
int tor_model_set_kv(tor_model *m, const float *k, const float *v,
                     size_t len);
/* Copy the first `len` cached positions out, in the same layout. */
int tor_model_get_kv(const tor_model *m, float *k, float *v, size_t len);

#ifdef __cplusplus
}
#endif
#endif
