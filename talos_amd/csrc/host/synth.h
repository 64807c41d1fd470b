// synth.h -- seeded synthetic Llama GGUF models for tests and benchmarks.
//
// Plays the role of the reference's absent model exporter (the bench and
// parity models come from Hephaistos, benches/tokps.rs:8-9): matrices are
// N(0, std) from a counter-based generator keyed by (seed, tensor name,
// element index), quantized with the same quantizers the reference's tests
// use (src/math/metal/mod.rs:551-574; Q6_K is this project's own), norms are
// 1.0, and the tokenizer keys Model::load requires are present
// (tests/forward_gpu.rs:323-337).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "gguf.h"

namespace talos {

struct SynthSpec {
  uint32_t n_layer = 0, n_head = 0, n_head_kv = 0, n_embd = 0, n_ff = 0, vocab = 0, ctx = 0;
  float rope_freq_base = 10000.f, rms_eps = 1e-5f;
  GgmlType layer_type = GgmlType::F32;   // q/k/v/o/gate/up/down
  GgmlType output_type = GgmlType::F32;  // output.weight
  GgmlType embd_type = GgmlType::F32;    // token_embd.weight
  uint64_t seed = 42;
  float stdev = 0.02f;
};

// Element i of tensor `name`: stdev * z_i, z ~ N(0,1) by Box-Muller over a
// splitmix64 stream keyed by (seed, name).  Writes n values starting at i0.
void synth_normal(uint64_t seed, const std::string& name, uint64_t i0, size_t n, float stdev, float* out);

// Quantize n floats (n a multiple of the block) into `type`'s block layout.
void quantize(GgmlType type, const float* x, size_t n, uint8_t* out);

// The whole model as GGUF v3 bytes.  Deterministic for any thread count.
std::vector<uint8_t> synth_model(const SynthSpec& s, int nthreads);

}  // namespace talos
