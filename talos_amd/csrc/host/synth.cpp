// synth.cpp -- seeded synthetic GGUF models (see synth.h).
#include "synth.h"

#include <cmath>
#include <cstring>
#include <thread>

namespace talos {

namespace {

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 0xCBF29CE484222325ULL;
  for (unsigned char ch : s) {
    h ^= ch;
    h *= 0x100000001B3ULL;
  }
  return h;
}

// Uniform in (0, 1], 53 bits.
double unit(uint64_t key, uint64_t k) {
  return (double)((mix64(key + k * 0x9E3779B97F4A7C15ULL) >> 11) + 1) * (1.0 / 9007199254740992.0);
}

uint16_t f32_to_f16(float f) {  // round to nearest even, as half::f16::from_f32
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0));
  const int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m24 = man | 0x800000u;
    const int shift = 14 - e;
    uint32_t hm = m24 >> shift;
    const uint32_t rem = m24 & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

float f16_to_f32(uint16_t h) {
  float out;
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      const float v = (float)man * 5.9604644775390625e-8f;
      return sign ? -v : v;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  memcpy(&out, &bits, 4);
  return out;
}

void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xFF);
  p[1] = (uint8_t)(v >> 8);
}

// Q8_0 as the reference's test quantizer (src/math/metal/mod.rs:553-561).
void quant_q8_0(const float* v, uint8_t* o) {
  float amax = 0.f;
  for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(v[j]));
  const float d = amax / 127.0f;
  put16(o, f32_to_f16(d));
  for (int j = 0; j < 32; ++j) {
    float q = 0.f;
    if (d != 0.f) q = std::fmin(std::fmax(std::round(v[j] / d), -128.f), 127.f);
    o[2 + j] = (uint8_t)(int8_t)q;
  }
}

// Q4_0 as the reference's test quantizer (src/math/metal/mod.rs:564-574).
void quant_q4_0(const float* v, uint8_t* o) {
  float max = 0.f;
  for (int j = 0; j < 32; ++j)
    if (std::fabs(v[j]) > std::fabs(max)) max = v[j];
  const float d = max / -8.0f;
  const float id = d != 0.f ? 1.0f / d : 0.f;
  put16(o, f32_to_f16(d));
  for (int j = 0; j < 16; ++j) {
    int a = (int)std::trunc(v[j] * id + 8.5f), b = (int)std::trunc(v[j + 16] * id + 8.5f);
    a = a < 0 ? 0 : (a > 15 ? 15 : a);
    b = b < 0 ? 0 : (b > 15 ? 15 : b);
    o[2 + j] = (uint8_t)(a | (b << 4));
  }
}

// Q6_K, this project's quantizer: per-16 signed-max sub-scales s_j =
// max/-32, super scale d = max_j s_j / -128 (f16), codes round(s_j/d) as
// int8, elements round(v/(d*code)) in [-32, 31] stored +32 in the
// ql/qh layout that src/gguf/dtype.rs:103-116 decodes.
void quant_q6_k(const float* v, uint8_t* b) {
  float s[16];
  for (int j = 0; j < 16; ++j) {
    float m = 0.f;
    for (int e = 0; e < 16; ++e)
      if (std::fabs(v[j * 16 + e]) > std::fabs(m)) m = v[j * 16 + e];
    s[j] = m / -32.0f;
  }
  float smax = 0.f;
  for (int j = 0; j < 16; ++j)
    if (std::fabs(s[j]) > std::fabs(smax)) smax = s[j];
  const float d = smax / -128.0f;
  const uint16_t dh = f32_to_f16(d);
  const float d16 = f16_to_f32(dh);
  int8_t sc[16];
  for (int j = 0; j < 16; ++j) {
    float cde = d16 != 0.f ? std::round(s[j] / d16) : 0.f;
    cde = std::fmin(std::fmax(cde, -128.f), 127.f);
    sc[j] = (int8_t)cde;
  }
  uint8_t q[256];
  for (int e = 0; e < 256; ++e) {
    const float es = d16 * (float)sc[e / 16];
    float qq = es != 0.f ? std::round(v[e] / es) : 0.f;
    qq = std::fmin(std::fmax(qq, -32.f), 31.f);
    q[e] = (uint8_t)((int)qq + 32);
  }
  memset(b, 0, 210);
  for (int h = 0; h < 2; ++h) {
    uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
    const uint8_t* qq = q + h * 128;
    for (int l = 0; l < 32; ++l) {
      ql[l] = (uint8_t)((qq[l] & 0xF) | ((qq[l + 64] & 0xF) << 4));
      ql[l + 32] = (uint8_t)((qq[l + 32] & 0xF) | ((qq[l + 96] & 0xF) << 4));
      qh[l] = (uint8_t)((qq[l] >> 4) | ((qq[l + 32] >> 4) << 2) | ((qq[l + 64] >> 4) << 4) | ((qq[l + 96] >> 4) << 6));
    }
  }
  for (int j = 0; j < 16; ++j) b[192 + j] = (uint8_t)sc[j];
  put16(b + 208, dh);
}

template <class F>
void parallel_rows(size_t rows, int nthreads, F f) {
  if (nthreads <= 1 || rows < 64) {
    f(0, rows);
    return;
  }
  std::vector<std::thread> th;
  const size_t per = (rows + nthreads - 1) / nthreads;
  for (int t = 0; t < nthreads; ++t) {
    const size_t r0 = t * per, r1 = std::min(rows, r0 + per);
    if (r0 >= r1) break;
    th.emplace_back([=] { f(r0, r1); });
  }
  for (auto& x : th) x.join();
}

}  // namespace

void synth_normal(uint64_t seed, const std::string& name, uint64_t i0, size_t n, float stdev, float* out) {
  const uint64_t key = mix64(seed ^ fnv1a(name));
  for (size_t k = 0; k < n; ++k) {
    const uint64_t i = i0 + k;
    const uint64_t pair = i >> 1;
    const double u1 = unit(key, 2 * pair), u2 = unit(key, 2 * pair + 1);
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586476925286766559 * u2;
    const double z = (i & 1) ? r * std::sin(th) : r * std::cos(th);
    out[k] = (float)(stdev * z);
  }
}

void quantize(GgmlType type, const float* x, size_t n, uint8_t* out) {
  const size_t be = block_elems(type), bb = block_bytes(type);
  if (type == GgmlType::F32) {
    memcpy(out, x, n * 4);
    return;
  }
  for (size_t b = 0; b < n / be; ++b) {
    if (type == GgmlType::Q8_0) quant_q8_0(x + b * be, out + b * bb);
    else if (type == GgmlType::Q4_0) quant_q4_0(x + b * be, out + b * bb);
    else quant_q6_k(x + b * be, out + b * bb);
  }
}

std::vector<uint8_t> synth_model(const SynthSpec& s, int nthreads) {
  if (!s.n_layer || !s.n_head || !s.n_head_kv || !s.n_embd || !s.n_ff || !s.vocab || !s.ctx)
    throw Error("synthetic model spec has a zero dimension");
  if (s.n_head % s.n_head_kv || s.n_embd % s.n_head) throw Error("inconsistent head counts");
  const uint32_t c = s.n_embd, hd = c / s.n_head, kv = s.n_head_kv * hd, ff = s.n_ff, V = s.vocab;
  GgufWriter w;
  w.str("general.architecture", "llama");
  w.u32("llama.context_length", s.ctx);
  w.u32("llama.embedding_length", c);
  w.u32("llama.block_count", s.n_layer);
  w.u32("llama.feed_forward_length", ff);
  w.u32("llama.attention.head_count", s.n_head);
  w.u32("llama.attention.head_count_kv", s.n_head_kv);
  w.f32("llama.attention.layer_norm_rms_epsilon", s.rms_eps);
  w.u32("llama.rope.dimension_count", hd);
  w.f32("llama.rope.freq_base", s.rope_freq_base);
  std::vector<std::string> toks(V);
  for (uint32_t i = 0; i < V; ++i) toks[i] = i == 0 ? "<unk>" : "t" + std::to_string(i);
  w.arr_str("tokenizer.ggml.tokens", toks);
  w.arr_str("tokenizer.ggml.merges", {});
  w.u32("tokenizer.ggml.unknown_token_id", 0);
  w.u32("tokenizer.ggml.bos_token_id", 1);
  w.u32("tokenizer.ggml.eos_token_id", 2);

  struct Spec {
    std::string name;
    size_t rows, cols;
    GgmlType type;
    bool norm;
  };
  std::vector<Spec> ts;
  ts.push_back({"token_embd.weight", V, c, s.embd_type, false});
  ts.push_back({"output_norm.weight", 1, c, GgmlType::F32, true});
  ts.push_back({"output.weight", V, c, s.output_type, false});
  for (uint32_t l = 0; l < s.n_layer; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    ts.push_back({p + "attn_norm.weight", 1, c, GgmlType::F32, true});
    ts.push_back({p + "attn_q.weight", c, c, s.layer_type, false});
    ts.push_back({p + "attn_k.weight", kv, c, s.layer_type, false});
    ts.push_back({p + "attn_v.weight", kv, c, s.layer_type, false});
    ts.push_back({p + "attn_output.weight", c, c, s.layer_type, false});
    ts.push_back({p + "ffn_norm.weight", 1, c, GgmlType::F32, true});
    ts.push_back({p + "ffn_gate.weight", ff, c, s.layer_type, false});
    ts.push_back({p + "ffn_up.weight", ff, c, s.layer_type, false});
    ts.push_back({p + "ffn_down.weight", c, ff, s.layer_type, false});
  }
  for (const auto& t : ts) {
    if (t.cols % block_elems(t.type))
      throw Error("tensor " + t.name + ": cols " + std::to_string(t.cols) + " not a multiple of its block");
    const size_t nbytes = t.rows * (t.cols / block_elems(t.type)) * block_bytes(t.type);
    std::vector<uint64_t> dims = t.norm ? std::vector<uint64_t>{t.cols} : std::vector<uint64_t>{t.cols, t.rows};
    w.tensor_sized(t.name, dims, t.type, nbytes);
  }
  return w.finish_fill([&](size_t i, uint8_t* dst) {
    const Spec& t = ts[i];
    if (t.norm) {
      for (size_t e = 0; e < t.cols; ++e) {
        const float one = 1.0f;
        memcpy(dst + e * 4, &one, 4);
      }
      return;
    }
    const size_t row_bytes = t.cols / block_elems(t.type) * block_bytes(t.type);
    parallel_rows(t.rows, nthreads, [&](size_t r0, size_t r1) {
      std::vector<float> buf(t.cols);
      for (size_t r = r0; r < r1; ++r) {
        synth_normal(s.seed, t.name, (uint64_t)r * t.cols, t.cols, s.stdev, buf.data());
        quantize(t.type, buf.data(), t.cols, dst + r * row_bytes);
      }
    });
  });
}

}  // namespace talos
