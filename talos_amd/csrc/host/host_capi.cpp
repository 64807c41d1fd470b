// host_capi.cpp -- C ABI over the host Model (include/talos_host.h).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <fstream>
#include <string>

#include "../../../include/talos_host.h"
#include "model.h"
#include "synth.h"

struct talos_model {
  std::unique_ptr<talos::Model> m;
  std::string err;
};

namespace {
std::string g_load_error;
thread_local std::string g_synth_error;

template <class F>
int guard(talos_model* m, F f) {
  if (!m) return TALOS_ERR_ARG;
  m->err.clear();
  try {
    f();
    return TALOS_OK;
  } catch (const talos::BackendError& e) {
    m->err = e.what();
    return e.status;
  } catch (const std::exception& e) {
    m->err = e.what();
    return TALOS_ERR_ARG;
  }
}

bool to_type(uint32_t tag, talos::GgmlType* t) { return talos::ggml_type_from_u32(tag, t); }

int spec_of(const talos_synth_spec* s, talos::SynthSpec* out) {
  if (!s) return TALOS_ERR_ARG;
  talos::SynthSpec p;
  p.n_layer = s->n_layer;
  p.n_head = s->n_head;
  p.n_head_kv = s->n_head_kv;
  p.n_embd = s->n_embd;
  p.n_ff = s->n_ff;
  p.vocab = s->vocab_size;
  p.ctx = s->context_length;
  p.rope_freq_base = s->rope_freq_base;
  p.rms_eps = s->rms_eps;
  if (!to_type(s->layer_type, &p.layer_type) || !to_type(s->output_type, &p.output_type) ||
      !to_type(s->embd_type, &p.embd_type)) {
    g_synth_error = "unsupported ggml type in synth spec";
    return TALOS_ERR_DTYPE;
  }
  p.seed = s->seed;
  p.stdev = s->stdev;
  *out = p;
  return TALOS_OK;
}
}  // namespace

extern "C" {

int talos_model_load(const char* path, int32_t device, talos_model** out) {
  g_load_error.clear();
  if (!path || !out) return TALOS_ERR_ARG;
  try {
    auto* h = new talos_model;
    h->m = talos::Model::load(path, device);
    *out = h;
    return TALOS_OK;
  } catch (const std::exception& e) {
    g_load_error = e.what();
    return TALOS_ERR_ARG;
  }
}

int talos_model_load_bytes(const void* bytes, size_t len, int32_t device, talos_model** out) {
  g_load_error.clear();
  if (!bytes || !out) return TALOS_ERR_ARG;
  try {
    const uint8_t* b = static_cast<const uint8_t*>(bytes);
    auto* h = new talos_model;
    h->m = talos::Model::from_gguf(talos::GgufFile::from_bytes(std::vector<uint8_t>(b, b + len)), device);
    *out = h;
    return TALOS_OK;
  } catch (const std::exception& e) {
    g_load_error = e.what();
    return TALOS_ERR_ARG;
  }
}

void talos_model_free(talos_model* m) { delete m; }

const char* talos_model_last_error(const talos_model* m) { return m ? m->err.c_str() : g_load_error.c_str(); }

int talos_model_config(const talos_model* m, talos_hip_cfg* out) {
  if (!m || !out) return TALOS_ERR_ARG;
  const auto& c = m->m->cfg;
  out->n_layer = c.n_layer;
  out->n_head = c.n_head;
  out->n_head_kv = c.n_head_kv;
  out->n_embd = c.n_embd;
  out->n_ff = c.n_ff;
  out->vocab_size = c.vocab_size;
  out->context_length = c.context_length;
  out->rms_eps = c.rms_eps;
  out->rope_freq_base = c.rope_freq_base;
  out->device = 0;
  return TALOS_OK;
}

int talos_model_gguf_bytes(const talos_model* m, const uint8_t** bytes, size_t* len) {
  if (!m || !bytes || !len) return TALOS_ERR_ARG;
  *bytes = m->m->gguf().data();
  *len = m->m->gguf().size();
  return TALOS_OK;
}

int talos_model_cap_context(talos_model* m, size_t max_ctx) {
  return guard(m, [&] { m->m->cap_context(max_ctx); });
}

int talos_model_forward_gpu(talos_model* m, uint32_t token, size_t pos, float* logits) {
  if (!logits) return TALOS_ERR_ARG;
  return guard(m, [&] {
    auto v = m->m->forward_gpu(token, pos);
    memcpy(logits, v.data(), v.size() * 4);
  });
}

int talos_model_forward_hidden_gpu(talos_model* m, uint32_t token, size_t pos, float* hidden) {
  if (!hidden) return TALOS_ERR_ARG;
  return guard(m, [&] {
    auto v = m->m->forward_hidden_gpu(token, pos);
    memcpy(hidden, v.data(), v.size() * 4);
  });
}

int talos_model_reset(talos_model* m) {
  return guard(m, [&] { m->m->reset(); });
}

int talos_model_dequant_row(const talos_model* m, uint32_t token, float* out) {
  if (!m || !out) return TALOS_ERR_ARG;
  if (token >= m->m->cfg.vocab_size) return TALOS_ERR_TOKEN;
  talos::QTensor t = talos::QTensor::bind(m->m->gguf(), "token_embd.weight", m->m->cfg.vocab_size, m->m->cfg.n_embd);
  t.dequant_row(token, out);
  return TALOS_OK;
}

int talos_model_forward_token(talos_model* m, uint32_t token, size_t pos, float* logits, uint32_t* argmax) {
  return guard(m, [&] {
    std::vector<float> l;
    const uint32_t a = m->m->forward_token(token, pos, logits ? &l : nullptr);
    if (logits) memcpy(logits, l.data(), l.size() * 4);
    if (argmax) *argmax = a;
  });
}

int talos_model_prefill(talos_model* m, const uint32_t* tokens, uint32_t n, size_t pos, float* logits,
                        uint32_t* argmax) {
  if (!tokens && n) return TALOS_ERR_ARG;
  return guard(m, [&] {
    std::vector<float> l;
    const uint32_t a = m->m->prefill(tokens, n, pos, logits ? &l : nullptr);
    if (logits && n) memcpy(logits, l.data(), l.size() * 4);
    if (argmax) *argmax = a;
  });
}

int talos_model_decode_greedy(talos_model* m, uint32_t token, size_t pos, uint32_t n_steps, uint32_t* tokens) {
  if (!tokens && n_steps) return TALOS_ERR_ARG;
  return guard(m, [&] {
    auto v = m->m->decode_greedy(token, pos, n_steps);
    memcpy(tokens, v.data(), v.size() * 4);
  });
}

talos_hip_ctx* talos_model_backend(talos_model* m) {
  if (!m) return nullptr;
  talos_hip_ctx* c = nullptr;
  if (guard(m, [&] { c = m->m->backend(); }) != TALOS_OK) return nullptr;
  return c;
}

int talos_synth_model_load(const talos_synth_spec* s, int32_t nthreads, int32_t device, talos_model** out) {
  talos::SynthSpec p;
  int rc = spec_of(s, &p);
  if (rc) return rc;
  if (!out) return TALOS_ERR_ARG;
  try {
    auto* h = new talos_model;
    h->m = talos::Model::from_gguf(talos::GgufFile::from_bytes(talos::synth_model(p, nthreads)), device);
    *out = h;
    return TALOS_OK;
  } catch (const std::exception& e) {
    g_synth_error = e.what();
    g_load_error = e.what();
    return TALOS_ERR_ARG;
  }
}

int talos_synth_model_bytes(const talos_synth_spec* s, int32_t nthreads, uint8_t** out, size_t* len) {
  talos::SynthSpec p;
  int rc = spec_of(s, &p);
  if (rc) return rc;
  if (!out || !len) return TALOS_ERR_ARG;
  try {
    auto v = talos::synth_model(p, nthreads);
    *out = static_cast<uint8_t*>(malloc(v.size() ? v.size() : 1));
    if (!*out) return TALOS_ERR_ARG;
    memcpy(*out, v.data(), v.size());
    *len = v.size();
    return TALOS_OK;
  } catch (const std::exception& e) {
    g_synth_error = e.what();
    return TALOS_ERR_ARG;
  }
}

int talos_synth_model_write(const talos_synth_spec* s, int32_t nthreads, const char* path) {
  talos::SynthSpec p;
  int rc = spec_of(s, &p);
  if (rc) return rc;
  if (!path) return TALOS_ERR_ARG;
  try {
    auto v = talos::synth_model(p, nthreads);
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)v.size());
    if (!f) throw talos::Error(std::string("writing ") + path);
    return TALOS_OK;
  } catch (const std::exception& e) {
    g_synth_error = e.what();
    return TALOS_ERR_ARG;
  }
}

void talos_synth_free(uint8_t* p) { free(p); }

int talos_synth_normal(uint64_t seed, const char* name, uint64_t i0, size_t n, float stdev, float* out) {
  if (!name || (!out && n)) return TALOS_ERR_ARG;
  talos::synth_normal(seed, name, i0, n, stdev, out);
  return TALOS_OK;
}

int talos_quantize(uint32_t type, const float* x, size_t n, uint8_t* out) {
  talos::GgmlType t;
  if (!to_type(type, &t)) {
    g_synth_error = "unsupported ggml type " + std::to_string(type);
    return TALOS_ERR_DTYPE;
  }
  if ((!x || !out) && n) return TALOS_ERR_ARG;
  if (n % talos::block_elems(t)) {
    g_synth_error = "n is not a multiple of the block size";
    return TALOS_ERR_SHAPE;
  }
  talos::quantize(t, x, n, out);
  return TALOS_OK;
}

const char* talos_synth_last_error(void) { return g_synth_error.c_str(); }

}  // extern "C"
