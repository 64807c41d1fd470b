/*
 * talos_hip.h -- C ABI of the MI355X (gfx950) decode backend for Talos.
 *
 * This is the drop-in replacement for the reference's GPU backend boundary,
 * Tsuskov/talos `src/math/metal/mod.rs` (and the call sites in
 * `src/model/llama.rs:188-206`).  Plain C types only: a Rust `src/math/hip`
 * crate (or any other FFI) binds these directly.
 *
 * Conventions
 *  - Every function returns a talos_status (0 = ok).  On failure the context
 *    keeps a message readable with talos_hip_last_error().  Where the
 *    reference panics (`expect`, metal/mod.rs:46,51,78,82) this library
 *    returns an error instead; the caller may abort to keep that behaviour.
 *  - A context is single-thread affine and owns one HIP stream on one device
 *    (the reference keeps one thread-local Metal context, metal/mod.rs:25-29).
 *  - Host buffers passed in are only read during the call; the caller keeps
 *    ownership.  Outputs are written into caller buffers.
 *  - Weights are resident in HBM, keyed by tensor name; a second upload under
 *    the same name with the same byte length is a no-op, a different length
 *    replaces the tensor (metal/mod.rs:63-72).
 *  - The per-layer K/V cache is device memory sized to context_length at the
 *    first forward; rows are written at `pos` so a new sequence can start at
 *    pos 0 without clearing (metal/mod.rs:391-396,443-454).
 */
#ifndef TALOS_HIP_H
#define TALOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum talos_status {
  TALOS_OK = 0,
  TALOS_ERR_ARG = 1,            /* null pointer, bad size, bad config */
  TALOS_ERR_HIP = 2,            /* a HIP runtime call failed */
  TALOS_ERR_DTYPE = 3,          /* unsupported ggml type tag */
  TALOS_ERR_SHAPE = 4,          /* byte length / rows / cols disagree */
  TALOS_ERR_MISSING_WEIGHT = 5, /* a tensor the forward needs is not uploaded */
  TALOS_ERR_POS = 6,            /* pos >= context_length */
  TALOS_ERR_TOKEN = 7           /* token id >= vocab_size */
} talos_status;

/* GGUF tensor type tags (src/gguf/dtype.rs:33-41). */
enum {
  TALOS_GGML_F32 = 0,
  TALOS_GGML_Q4_0 = 2,
  TALOS_GGML_Q8_0 = 8,
  TALOS_GGML_Q6_K = 14
};

/* Model hyper-parameters: src/model/config.rs:14-25 (rope_dim is unused by
 * the forward, config.rs:64, so it is not carried). */
typedef struct talos_hip_cfg {
  uint32_t n_layer;
  uint32_t n_head;
  uint32_t n_head_kv;
  uint32_t n_embd;
  uint32_t n_ff;
  uint32_t vocab_size;
  uint32_t context_length;
  float rms_eps;
  float rope_freq_base;
  int32_t device; /* HIP device ordinal */
} talos_hip_cfg;

typedef struct talos_hip_ctx talos_hip_ctx;

/* Create a context: device, stream, RoPE table.  Replaces the lazily built
 * thread-local MetalCtx (metal/mod.rs:31-59) plus GpuKv::new (:278-280). */
int talos_hip_create(const talos_hip_cfg* cfg, talos_hip_ctx** out);

/* Free every device buffer, graph and the stream.  NULL is a no-op. */
void talos_hip_destroy(talos_hip_ctx* ctx);

/* Message for the last failing call on this context ("" if none).  With a
 * NULL context, the message of the last failed talos_hip_create. */
const char* talos_hip_last_error(const talos_hip_ctx* ctx);

/* Make `bytes` (GGUF block layout, `len` bytes, type tag `ggml_type`, a
 * row-major [rows, cols] matrix or a 1-D norm with rows = 1) resident under
 * `name`.  Replaces MetalCtx::resident_weight (metal/mod.rs:63-72), which the
 * reference feeds from QTensor::gpu_parts (src/model/weights.rs:64-69).
 * Tensor names follow src/model/weights.rs:95-111. */
int talos_hip_upload_weight(talos_hip_ctx* ctx, const char* name, const void* bytes, size_t len,
                            uint32_t ggml_type, size_t rows, size_t cols);

/* One decode step: x_embed is the token's embedding row (n_embd floats, the
 * caller's dequant_row as in src/model/llama.rs:192-193); writes vocab_size
 * logits.  Replaces math::metal::forward (metal/mod.rs:351-353).  Appends the
 * step's K/V at `pos`; attends over positions 0..=pos.
 * Errors with TALOS_ERR_POS if pos >= context_length. */
int talos_hip_forward(talos_hip_ctx* ctx, const float* x_embed, uint32_t pos, float* logits);

/* Same step, returning the final-norm hidden state (n_embd floats) instead of
 * logits.  Replaces math::metal::forward_hidden (metal/mod.rs:358-366). */
int talos_hip_forward_hidden(talos_hip_ctx* ctx, const float* x_embed, uint32_t pos, float* hidden);

/* Embedding lookup on the device (token_embd.weight must be resident): the
 * token id goes in, logits (nullable) and the greedy argmax (nullable; ties
 * to the last index, src/sample.rs:7-14) come out.  No reference
 * counterpart: it removes the host dequant_row and shrinks the read-back. */
int talos_hip_forward_token(talos_hip_ctx* ctx, uint32_t token, uint32_t pos, float* logits,
                            uint32_t* argmax);

/* Greedy decode entirely on the device: starting from `token` at `pos`, run
 * n_steps forwards, each feeding the argmax of the previous one, and write
 * the n_steps argmax tokens to tokens_out.  This is the loop of
 * benches/tokps.rs:33-39 / src/main.rs:100-112 with temperature 0 and no EOS
 * stop; the host only launches graph replays.  pos + n_steps must be
 * <= context_length. */
int talos_hip_decode_greedy(talos_hip_ctx* ctx, uint32_t token, uint32_t pos, uint32_t n_steps,
                            uint32_t* tokens_out);

/* Prompt processing on the device: run tokens[0..n) at positions
 * pos..pos+n-1 (the prefill loop of src/main.rs:88-94, Model::step per
 * prompt token) and leave the cache and the device state as that loop does.
 * Models with head_dim a multiple of 16 up to 256 (n_head * head_dim ==
 * n_embd, groups up to 8), whatever their layer matrices' formats,
 * take the prompt in chunks of up to 1024 tokens through each layer at once
 * on the matrix cores: the same products and f32 sums in another order, so
 * within f32 rounding of the token loop rather than bit-identical.  Other
 * models, or any model with TALOS_HIP_BATCH=0 in the environment when the
 * context is created, run one forward per token with each next token taken
 * from a device copy of `tokens` (bit-identical to a host loop of
 * talos_hip_forward_token).  Returns the last step's logits (nullable) and
 * argmax (nullable), which is the first greedy token.  pos + n must be
 * <= context_length and every token < vocab_size.  The first batched call
 * also makes the prefill GEMMs' tiled copy of the Q4_0 / Q8_0 layer
 * matrices (one more device copy of them, kept until a weight is uploaded
 * or the context destroyed; none with TALOS_HIP_PF_TILED=0 in the
 * environment when the context is created). */
int talos_hip_prefill(talos_hip_ctx* ctx, const uint32_t* tokens, uint32_t n, uint32_t pos, float* logits,
                      uint32_t* argmax);

/* Draw one token from the logits of the context's latest forward step
 * (src/sample.rs:19-76): temperature <= 0 is the greedy argmax (ties to the
 * last index); otherwise the logits sorted descending by total_cmp (equal
 * logits by descending index -- the reference's unstable sort leaves their
 * order open), cut to the top_k largest (0: no cut, the reference's None),
 * softmax at `temperature` over the kept set, cut to the shortest prefix
 * whose cumulative probability reaches top_p (a value above 1, or NaN: no
 * cut), and the first token whose cumulative probability reaches u times
 * the kept mass.  u in [0, 1) is the caller's uniform draw, the reference's
 * rng.gen::<f32>() (its StdRng stream is not reproduced here).  The draw
 * runs on the device; only the token is read back. */
int talos_hip_sample(talos_hip_ctx* ctx, float temperature, uint32_t top_k, float top_p, float u, uint32_t* token);

/* The same draw from n device logits into a device uint32, enqueued on the
 * context's stream and not waited for (the sampler's workspace is allocated
 * by the library on first use and grown with n).  No reference
 * counterpart: sampling inside a device-resident serving loop. */
int talos_hip_sample_dev(talos_hip_ctx* ctx, const float* d_logits, uint32_t n, float temperature, uint32_t top_k,
                         float top_p, float u, uint32_t* d_token);

/* talos_hip_sample_dev without any allocation: the draw's workspace is a
 * fixed scratch array in device memory that every GPU the library runs on
 * holds for the life of the process (2.5 MB), so n is at most 131072
 * (TALOS_ERR_SHAPE beyond).  It calls no hipMalloc/hipFree.  Calls that
 * overlap on one GPU share that scratch and race; order them on one stream.
 * No reference counterpart: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid it). */
int talos_hip_sample_noalloc(talos_hip_ctx* ctx, const float* d_logits, uint32_t n, float temperature,
                             uint32_t top_k, float top_p, float u, uint32_t* d_token);

/* Sampled decode entirely on the device: starting from `token` at `pos`,
 * run n_steps forwards, each followed by a draw (as talos_hip_sample, with
 * draw u[s] for step s) that becomes the next input; writes the n_steps
 * drawn tokens.  The loop of src/main.rs:100-112 with temperature > 0 and
 * no EOS stop.  pos + n_steps <= context_length. */
int talos_hip_decode_sample(talos_hip_ctx* ctx, uint32_t token, uint32_t pos, uint32_t n_steps, float temperature,
                            uint32_t top_k, float top_p, const float* u, uint32_t* tokens_out);

/* Teacher-forced perplexity of tokens[0..n) (src/eval.rs:35-52): chunks of
 * context_length tokens, each from position 0; within a chunk every
 * position's forward scores the next token's -log softmax (src/eval.rs:
 * 17-22, on the device, exponential sum in f64); ppl = exp(mean NLL).  The
 * per-position NLLs go to nll (nullable; one per scored position, at most
 * n - 1).  Replaces eval::perplexity's CPU Model::forward (eval.rs:46). */
int talos_hip_perplexity(talos_hip_ctx* ctx, const uint32_t* tokens, uint32_t n, float* ppl, float* nll);

/* Reset the cache for a new sequence.  Rows are position-indexed, so this
 * only records that no position is valid (the reference's GpuKv needs no
 * clear either, metal/mod.rs:443-454). */
int talos_hip_kv_reset(talos_hip_ctx* ctx);

/* Copy `n_pos` positions of the K and V caches of every layer to host
 * buffers laid out [layer][pos][kv_dim] (for tests and state handoff). */
int talos_hip_kv_read(talos_hip_ctx* ctx, uint32_t n_pos, float* k_out, float* v_out);

/* The inverse: load `n_pos` positions of K and V for every layer from host
 * buffers laid out [layer][pos][kv_dim] (state handoff, e.g. restoring a
 * saved long prefix).  No reference counterpart. */
int talos_hip_kv_write(talos_hip_ctx* ctx, uint32_t n_pos, const float* k, const float* v);

/* Standalone resident matvec, out[rows] = W x: uploads `bytes` under `name`
 * on first use (or on a length change) and runs the fused dequant-matvec.
 * Replaces matvec_f32_resident / matvec_quant_resident (metal/mod.rs:226-253).
 * Synchronous; x and out are host buffers. */
int talos_hip_matvec(talos_hip_ctx* ctx, const char* name, const void* bytes, size_t len,
                     uint32_t ggml_type, size_t rows, size_t cols, const float* x, float* out);

/* Device-pointer variant for timing: `name` must already be resident; d_x
 * (cols floats) and d_out (rows floats) are device pointers.  Enqueued on
 * the context's stream and not waited for. */
int talos_hip_matvec_dev(talos_hip_ctx* ctx, const char* name, const float* d_x, float* d_out);

/* Time `reps` standalone matvecs (as talos_hip_matvec_dev) rotating over the
 * resident weights `names` (one shape; give more bytes than the 256 MB MALL
 * so every launch streams from HBM), with HIP events on the context's
 * stream.  Writes the mean launch duration (us) and the algorithmic bytes of
 * one launch (the weight bytes plus x and y).  No reference counterpart: the
 * matvec microbenchmark (metal/mod.rs:195-253 is the API it times). */
int talos_hip_bench_matvec(talos_hip_ctx* ctx, const char* const* names, uint32_t n_names, uint32_t reps,
                           float* avg_us, double* bytes);

/* Time one decode kernel kind ("qkv", "oproj", "gateup", "down", "output")
 * with HIP events on the context's stream: `reps` back-to-back launches on
 * the resident weights, rotating through the layers so the weights stream
 * from HBM.  Writes the mean launch duration (us) and the algorithmic bytes
 * one launch moves (weights + activations).  No reference counterpart: the
 * roofline measurement.  The qkv kind rewrites K/V row 0. */
int talos_hip_bench_kernel(talos_hip_ctx* ctx, const char* kind, uint32_t reps, float* avg_us,
                           double* bytes);

/* Time `reps` device-token steps (as talos_hip_forward_token, without the
 * read-back) of `token` at `pos` with HIP events on the context's stream;
 * returns the mean step time and the step's algorithmic bytes: all weights
 * once (one embedding row), K/V rows 0..pos read, the K/V row at pos
 * written, the logits.  Rewrites the K/V row at pos.  No reference
 * counterpart: the roofline measurement of the decode step. */
int talos_hip_bench_token(talos_hip_ctx* ctx, uint32_t token, uint32_t pos, uint32_t reps, float* avg_us,
                          double* bytes);

/* Time `reps` launches of a plain device copy of nbytes (a multiple of 16):
 * the HBM reference point, and the known-size kernel that scales the
 * FETCH_SIZE / WRITE_SIZE counters.  No reference counterpart. */
int talos_hip_bench_copy(talos_hip_ctx* ctx, size_t nbytes, uint32_t reps, float* avg_us);

/* Profiling aid for the persistent decode kernel: run one device-token step
 * (as talos_hip_forward_token) and record, per workgroup, a wall-clock mark
 * at each phase boundary (16 per layer: ten phase ends, a spare, five inside
 * the first attention item; then the head).  Writes nblocks *
 * slots marks (cap must allow them) and the tick length in ns.  No reference
 * counterpart. */
int talos_hip_phase_timeline(talos_hip_ctx* ctx, uint32_t token, uint32_t pos, uint64_t* marks, size_t cap,
                             uint32_t* nblocks, uint32_t* slots, double* tick_ns);

/* Poll limit of the persistent kernel's bounded waits (grid barriers and
 * producer waits; default 2^20 polls, 0 restores the default).  A wait that
 * reaches it stops waiting, later barriers of the launch are skipped, every
 * workgroup runs to the end and the step returns TALOS_ERR_HIP (the results
 * of that step are invalid; the next step starts clean).  A tuning and test
 * knob: a tiny limit forces that error path from the host.  No reference
 * counterpart (the Metal backend has no cross-workgroup waits). */
int talos_hip_set_spin_limit(talos_hip_ctx* ctx, uint32_t polls);

/* Implementations of the token step (talos_hip_path). */
enum {
  TALOS_PATH_NONE = 0,
  TALOS_PATH_PERSISTENT = 1,    /* one persistent-kernel launch per token */
  TALOS_PATH_GRAPH = 2,         /* ~5 fused kernels per layer replayed as one hipGraph */
  TALOS_PATH_GRAPH_GENERIC = 3  /* the graph with generic-shape kernels for some steps (any head_dim,
                                   group, mixed formats) */
};

/* Which implementation runs this context's token step for the resident
 * weights (every tensor the forward needs must be uploaded; the choice is
 * made as at the first forward).  No reference counterpart: the Metal
 * backend has one path (metal/mod.rs:368-520); this one picks per model. */
int talos_hip_path(talos_hip_ctx* ctx, int* path);

/* The context's HIP stream (hipStream_t), for callers that time or order
 * work around talos_hip_matvec_dev. */
void* talos_hip_stream(talos_hip_ctx* ctx);

/* Wait for all work enqueued on the context's stream. */
int talos_hip_sync(talos_hip_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif
