/*
 * talos_host.h -- C ABI of the host-side Model that drives the HIP backend.
 *
 * The reference's caller of the GPU boundary is the Rust `Model`
 * (Tsuskov/talos src/model/llama.rs): it owns the GGUF mmap, binds weight
 * views (src/model/weights.rs), dequantizes the embedding row on the CPU and
 * calls the backend.  With no Rust toolchain in this build that caller is
 * C++ (talos_amd/csrc/host); these entry points expose it to Python tests,
 * the benchmark and any other FFI.  Status codes and the last-error string
 * follow include/talos_hip.h.
 */
#ifndef TALOS_HOST_H
#define TALOS_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "talos_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct talos_model talos_model;

/* Model::load (src/model/llama.rs:33-35): mmap and parse a GGUF file. */
int talos_model_load(const char* path, int32_t device, talos_model** out);
/* Model::load_bytes (llama.rs:39-41): the library copies the bytes. */
int talos_model_load_bytes(const void* bytes, size_t len, int32_t device, talos_model** out);
void talos_model_free(talos_model* m);
/* Last error on this model; with NULL, the last failed load. */
const char* talos_model_last_error(const talos_model* m);

/* Hyper-parameters (src/model/config.rs:14-25); `device` is the ordinal. */
int talos_model_config(const talos_model* m, talos_hip_cfg* out);
/* The GGUF bytes the model reads (valid while the model lives). */
int talos_model_gguf_bytes(const talos_model* m, const uint8_t** bytes, size_t* len);

int talos_model_cap_context(talos_model* m, size_t max_ctx);                      /* llama.rs:69-81 */
int talos_model_forward_gpu(talos_model* m, uint32_t token, size_t pos, float* logits); /* :188-195 */
int talos_model_forward_hidden_gpu(talos_model* m, uint32_t token, size_t pos, float* hidden); /* :199-206 */
int talos_model_reset(talos_model* m);                                            /* :236-238 */
/* Host dequant_row of token_embd (src/model/weights.rs:58-62). */
int talos_model_dequant_row(const talos_model* m, uint32_t token, float* out);

/* Device-side embedding lookup and greedy decode (talos_hip_forward_token /
 * talos_hip_decode_greedy through this model's backend). */
int talos_model_forward_token(talos_model* m, uint32_t token, size_t pos, float* logits, uint32_t* argmax);
int talos_model_decode_greedy(talos_model* m, uint32_t token, size_t pos, uint32_t n_steps, uint32_t* tokens);
/* The prompt loop of src/main.rs:88-94 (Model::step per prompt token) run
 * through talos_hip_prefill; logits (optional) and argmax of the last token. */
int talos_model_prefill(talos_model* m, const uint32_t* tokens, uint32_t n, size_t pos, float* logits,
                        uint32_t* argmax);
/* The backend context (created and filled with the resident weights on
 * first use). */
talos_hip_ctx* talos_model_backend(talos_model* m);

/* ---- seeded synthetic models (tests and benchmarks) ---- */
typedef struct talos_synth_spec {
  uint32_t n_layer, n_head, n_head_kv, n_embd, n_ff, vocab_size, context_length;
  float rope_freq_base, rms_eps;
  uint32_t layer_type;  /* ggml tag of q/k/v/o/gate/up/down */
  uint32_t output_type; /* ggml tag of output.weight */
  uint32_t embd_type;   /* ggml tag of token_embd.weight */
  uint64_t seed;
  float stdev;          /* N(0, stdev) weights */
} talos_synth_spec;

/* Generate a model and load it without an intermediate copy. */
int talos_synth_model_load(const talos_synth_spec* s, int32_t nthreads, int32_t device, talos_model** out);
/* Generate a model as GGUF bytes into a malloc'ed buffer (free with
 * talos_synth_free); or write it to `path`. */
int talos_synth_model_bytes(const talos_synth_spec* s, int32_t nthreads, uint8_t** out, size_t* len);
int talos_synth_model_write(const talos_synth_spec* s, int32_t nthreads, const char* path);
void talos_synth_free(uint8_t* p);
/* The generator's normal stream for one tensor: n values from index i0. */
int talos_synth_normal(uint64_t seed, const char* name, uint64_t i0, size_t n, float stdev, float* out);
/* Quantize n floats (a multiple of the block) into ggml type `type`. */
int talos_quantize(uint32_t type, const float* x, size_t n, uint8_t* out);
/* Message of the last failed synth/quantize call on this thread. */
const char* talos_synth_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
