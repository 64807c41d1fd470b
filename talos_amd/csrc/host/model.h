// model.h -- host side of the decode path: Config, weight handles and the
// Model whose forward_gpu drives the HIP backend.
//
// Mirrors Tsuskov/talos src/model/config.rs (Config::from_gguf),
// src/model/weights.rs (QTensor, Weights::from_gguf, tensor names) and the GPU
// half of src/model/llama.rs (forward_gpu, forward_hidden_gpu, step,
// step_hidden, reset, cap_context).  The CPU forward of llama.rs is not part
// of the product: it is the oracle the tests compare against.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../../include/talos_hip.h"
#include "gguf.h"

namespace talos {

struct Config {  // src/model/config.rs:14-25
  uint32_t n_layer = 0, n_head = 0, n_head_kv = 0, n_embd = 0, n_ff = 0;
  uint32_t context_length = 0, vocab_size = 0, rope_dim = 0;
  float rms_eps = 1e-5f, rope_freq_base = 10000.f;
  uint32_t head_dim() const { return n_embd / n_head; }             // config.rs:28-30
  uint32_t kv_dim() const { return n_head_kv * head_dim(); }        // config.rs:34-36
  static Config from_gguf(const GgufFile& g);                       // config.rs:40-67
};

// A [rows, cols] weight in its stored dtype (src/model/weights.rs:20-69).
struct QTensor {
  const uint8_t* bytes = nullptr;
  size_t len = 0;
  GgmlType dtype = GgmlType::F32;
  size_t rows = 0, cols = 0;
  std::string name;
  static QTensor bind(const GgufFile& g, const std::string& name, size_t rows, size_t cols);
  void dequant_row(size_t r, float* out) const;  // weights.rs:58-62
};

struct LayerWeights {  // weights.rs:72-82
  QTensor attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down;
};

struct Weights {  // weights.rs:84-114
  QTensor token_embd, output_norm, output;
  std::vector<LayerWeights> layers;
  static Weights from_gguf(const GgufFile& g, const Config& cfg);
};

class Model {
 public:
  // src/model/llama.rs:33-62 (n_head % n_head_kv checked as :45-51).
  static std::unique_ptr<Model> load(const std::string& path, int device);
  static std::unique_ptr<Model> from_gguf(GgufFile g, int device);
  ~Model();

  Config cfg;
  const GgufFile& gguf() const { return gguf_; }

  void cap_context(size_t max_ctx);                                 // llama.rs:69-81
  std::vector<float> forward_gpu(uint32_t token, size_t pos);        // llama.rs:188-195
  std::vector<float> forward_hidden_gpu(uint32_t token, size_t pos); // llama.rs:199-206
  std::vector<float> step(uint32_t token, size_t pos) { return forward_gpu(token, pos); }          // :211-220
  std::vector<float> step_hidden(uint32_t token, size_t pos) { return forward_hidden_gpu(token, pos); }
  void reset();                                                     // llama.rs:236-238

  // Device-side embedding lookup + argmax (no reference counterpart).
  uint32_t forward_token(uint32_t token, size_t pos, std::vector<float>* logits);
  std::vector<uint32_t> decode_greedy(uint32_t token, size_t pos, uint32_t n_steps);
  // The prompt loop of main.rs:88-94 (step per prompt token) with the
  // tokens fed on the device; returns the last step's argmax.
  uint32_t prefill(const uint32_t* tokens, uint32_t n, size_t pos, std::vector<float>* logits);

  talos_hip_ctx* backend();

 private:
  Model(GgufFile g, int device);
  void ensure_backend();
  void upload_all();
  GgufFile gguf_;
  Weights w_;
  int device_ = 0;
  talos_hip_ctx* ctx_ = nullptr;
  bool uploaded_ = false;
};

}  // namespace talos
