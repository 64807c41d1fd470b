// model.cpp -- host Model driving the HIP backend (see model.h).
#include "model.h"

#include <cstring>

namespace talos {

namespace {
void check(talos_hip_ctx* ctx, int rc) {
  if (rc != TALOS_OK) throw BackendError(rc, talos_hip_last_error(ctx));
}
}  // namespace

Config Config::from_gguf(const GgufFile& g) {
  const std::string* arch = g.get_str("general.architecture");
  if (!arch || *arch != "llama")
    throw Error("general.architecture is \"" + (arch ? *arch : std::string()) + "\"; only \"llama\" models load");
  Config c;
  auto u = [&](const char* k) {
    uint32_t v;
    if (!g.get_u32(k, &v)) throw Error(std::string("model metadata lacks ") + k);
    return v;
  };
  const auto* toks = g.get_arr_str("tokenizer.ggml.tokens");
  if (!toks) throw Error("model metadata lacks tokenizer.ggml.tokens, which sets the vocabulary size");
  c.vocab_size = (uint32_t)toks->size();
  c.n_layer = u("llama.block_count");
  c.n_head = u("llama.attention.head_count");
  c.n_head_kv = u("llama.attention.head_count_kv");
  c.n_embd = u("llama.embedding_length");
  c.n_ff = u("llama.feed_forward_length");
  c.context_length = u("llama.context_length");
  if (!g.get_f32("llama.attention.layer_norm_rms_epsilon", &c.rms_eps)) c.rms_eps = 1e-5f;
  c.rope_dim = u("llama.rope.dimension_count");
  if (!g.get_f32("llama.rope.freq_base", &c.rope_freq_base)) c.rope_freq_base = 10000.f;
  return c;
}

QTensor QTensor::bind(const GgufFile& g, const std::string& name, size_t rows, size_t cols) {
  QTensor t;
  t.bytes = g.tensor_raw(name, &t.len, &t.dtype);
  t.rows = rows;
  t.cols = cols;
  t.name = name;
  const size_t be = block_elems(t.dtype);
  if (cols % be || t.len != rows * (cols / be) * block_bytes(t.dtype))
    throw Error("tensor \"" + name + "\": " + std::to_string(t.len) + " bytes do not hold [" + std::to_string(rows) +
                ", " + std::to_string(cols) + "]");
  return t;
}

void QTensor::dequant_row(size_t r, float* out) const {
  const size_t row_bytes = cols / block_elems(dtype) * block_bytes(dtype);
  dequantize(dtype, bytes + r * row_bytes, out, cols);
}

Weights Weights::from_gguf(const GgufFile& g, const Config& cfg) {
  const size_t c = cfg.n_embd, ff = cfg.n_ff, v = cfg.vocab_size, kv = cfg.kv_dim();
  Weights w;
  for (uint32_t l = 0; l < cfg.n_layer; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    LayerWeights lw;
    lw.attn_norm = QTensor::bind(g, p + "attn_norm.weight", 1, c);
    lw.attn_q = QTensor::bind(g, p + "attn_q.weight", c, c);
    lw.attn_k = QTensor::bind(g, p + "attn_k.weight", kv, c);
    lw.attn_v = QTensor::bind(g, p + "attn_v.weight", kv, c);
    lw.attn_output = QTensor::bind(g, p + "attn_output.weight", c, c);
    lw.ffn_norm = QTensor::bind(g, p + "ffn_norm.weight", 1, c);
    lw.ffn_gate = QTensor::bind(g, p + "ffn_gate.weight", ff, c);
    lw.ffn_up = QTensor::bind(g, p + "ffn_up.weight", ff, c);
    lw.ffn_down = QTensor::bind(g, p + "ffn_down.weight", c, ff);
    for (const QTensor* n : {&lw.attn_norm, &lw.ffn_norm})
      if (n->dtype != GgmlType::F32) throw Error("norm \"" + n->name + "\" must be stored as F32");
    w.layers.push_back(std::move(lw));
  }
  w.token_embd = QTensor::bind(g, "token_embd.weight", v, c);
  w.output_norm = QTensor::bind(g, "output_norm.weight", 1, c);
  if (w.output_norm.dtype != GgmlType::F32) throw Error("norm \"output_norm.weight\" must be stored as F32");
  w.output = QTensor::bind(g, "output.weight", v, c);
  return w;
}

Model::Model(GgufFile g, int device) : gguf_(std::move(g)), device_(device) {}

Model::~Model() { talos_hip_destroy(ctx_); }

std::unique_ptr<Model> Model::load(const std::string& path, int device) {
  return from_gguf(GgufFile::open(path), device);
}

std::unique_ptr<Model> Model::from_gguf(GgufFile g, int device) {
  Config cfg = Config::from_gguf(g);
  if (cfg.n_head_kv == 0 || cfg.n_head % cfg.n_head_kv != 0)
    throw Error("attention head_count " + std::to_string(cfg.n_head) + " is not divisible by a nonzero head_count_kv (" +
                std::to_string(cfg.n_head_kv) + ")");
  std::unique_ptr<Model> m(new Model(std::move(g), device));
  m->cfg = cfg;
  m->w_ = Weights::from_gguf(m->gguf_, m->cfg);
  return m;
}

void Model::ensure_backend() {
  if (ctx_) return;
  talos_hip_cfg c{};
  c.n_layer = cfg.n_layer;
  c.n_head = cfg.n_head;
  c.n_head_kv = cfg.n_head_kv;
  c.n_embd = cfg.n_embd;
  c.n_ff = cfg.n_ff;
  c.vocab_size = cfg.vocab_size;
  c.context_length = cfg.context_length;
  c.rms_eps = cfg.rms_eps;
  c.rope_freq_base = cfg.rope_freq_base;
  c.device = device_;
  if (talos_hip_create(&c, &ctx_) != TALOS_OK) throw Error(talos_hip_last_error(nullptr));
  uploaded_ = false;
}

// Every tensor becomes resident under its GGUF name, as
// MetalCtx::resident_weight does on first use (src/math/metal/mod.rs:63-72).
void Model::upload_all() {
  if (uploaded_) return;
  auto up = [&](const QTensor& t) {
    check(ctx_, talos_hip_upload_weight(ctx_, t.name.c_str(), t.bytes, t.len, (uint32_t)t.dtype, t.rows, t.cols));
  };
  for (const auto& lw : w_.layers)
    for (const QTensor* t : {&lw.attn_norm, &lw.attn_q, &lw.attn_k, &lw.attn_v, &lw.attn_output, &lw.ffn_norm,
                             &lw.ffn_gate, &lw.ffn_up, &lw.ffn_down})
      up(*t);
  up(w_.token_embd);
  up(w_.output_norm);
  up(w_.output);
  uploaded_ = true;
}

talos_hip_ctx* Model::backend() {
  ensure_backend();
  upload_all();
  return ctx_;
}

void Model::cap_context(size_t max_ctx) {
  const size_t cap = max_ctx > 0 ? max_ctx : 1;
  cfg.context_length = (uint32_t)std::min<size_t>(cfg.context_length, cap);
  talos_hip_destroy(ctx_);  // a fresh device KV sized to the new context
  ctx_ = nullptr;
  uploaded_ = false;
}

std::vector<float> Model::forward_gpu(uint32_t token, size_t pos) {
  if (token >= cfg.vocab_size)
    throw BackendError(TALOS_ERR_TOKEN, ("token " + std::to_string(token) + " out of range").c_str());
  talos_hip_ctx* c = backend();
  std::vector<float> x(cfg.n_embd), logits(cfg.vocab_size);
  w_.token_embd.dequant_row(token, x.data());  // llama.rs:192-193
  check(c, talos_hip_forward(c, x.data(), (uint32_t)pos, logits.data()));
  return logits;
}

std::vector<float> Model::forward_hidden_gpu(uint32_t token, size_t pos) {
  if (token >= cfg.vocab_size)
    throw BackendError(TALOS_ERR_TOKEN, ("token " + std::to_string(token) + " out of range").c_str());
  talos_hip_ctx* c = backend();
  std::vector<float> x(cfg.n_embd), hidden(cfg.n_embd);
  w_.token_embd.dequant_row(token, x.data());
  check(c, talos_hip_forward_hidden(c, x.data(), (uint32_t)pos, hidden.data()));
  return hidden;
}

void Model::reset() {
  if (ctx_) check(ctx_, talos_hip_kv_reset(ctx_));
}

uint32_t Model::forward_token(uint32_t token, size_t pos, std::vector<float>* logits) {
  talos_hip_ctx* c = backend();
  uint32_t am = 0;
  if (logits) logits->resize(cfg.vocab_size);
  check(c, talos_hip_forward_token(c, token, (uint32_t)pos, logits ? logits->data() : nullptr, &am));
  return am;
}

std::vector<uint32_t> Model::decode_greedy(uint32_t token, size_t pos, uint32_t n_steps) {
  talos_hip_ctx* c = backend();
  std::vector<uint32_t> out(n_steps);
  check(c, talos_hip_decode_greedy(c, token, (uint32_t)pos, n_steps, out.data()));
  return out;
}

uint32_t Model::prefill(const uint32_t* tokens, uint32_t n, size_t pos, std::vector<float>* logits) {
  talos_hip_ctx* c = backend();
  uint32_t am = 0;
  if (logits) logits->resize(cfg.vocab_size);
  check(c, talos_hip_prefill(c, tokens, n, (uint32_t)pos, logits ? logits->data() : nullptr, &am));
  return am;
}

}  // namespace talos
