// talos_hip.hip -- MI355X decode backend behind the C ABI in include/talos_hip.h.
//
// Host orchestration for the reference's GPU forward (Tsuskov/talos
// src/math/metal/mod.rs:368-520), re-designed for gfx950:
//  * weights are repacked once at upload (layout.h) and stay resident in HBM,
//    keyed by tensor name;
//  * the K/V cache, residual stream and activations stay on the device;
//  * a token step is one launch of the persistent kernel (mega.h: every
//    layer, the output projection and the argmax, phases separated by grid
//    barriers) reading position/token from device memory;
//  * models without a persistent-kernel instantiation (mixed layer formats,
//    shapes it does not take) run ~5 kernels per layer (kernels.h) captured
//    once into a hipGraph.  Either way only the logits (or nothing, in the
//    device token loop) are read back.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/talos_hip.h"
#include "mega.h"
#include "mega_inst.h"
#include "sample.h"
#include "prefill.h"
#include "rows_iq.h"

// Scratch of the allocation-free sampling entry point
// (talos_hip_sample_noalloc): keys twice and the probabilities for up to
// TALOS_SAMPLE_NOALLOC_MAX logits.  Each GPU holds its own copy for the life
// of the process; host code reaches it only through the device address
// hipGetSymbolAddress returns on that GPU.
#define TALOS_SAMPLE_NOALLOC_MAX (1u << 17)
static __device__ __align__(256) uint8_t scratch[(size_t)TALOS_SAMPLE_NOALLOC_MAX * 20];

namespace {

std::string g_create_error;

std::mutex g_scratch_mu;
std::vector<uint8_t*> g_scratch_ptr;  // per device ordinal, null until set up

// With `dev` current: record this GPU's address of `scratch` (once).
hipError_t scratch_setup(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (g_scratch_ptr[dev]) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e == hipSuccess) g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  return e;
}

uint8_t* scratch_ptr(int dev) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return dev < (int)g_scratch_ptr.size() ? g_scratch_ptr[dev] : nullptr;
}

struct DevWeight {
  uint32_t type = 0;
  size_t rows = 0, cols = 0, len = 0;
  void* mem = nullptr;
  DevMat mat{};
  const float* f32 = nullptr;  // F32 tensors: the plain row-major data
  void* tiled = nullptr;       // the prefill GEMMs' tiled copy, in the context's pool (pf_tile_weights), or null
};

// G_TOKEN: embedding on the device + argmax; G_GREEDY: + greedy advance;
// G_FEED: + advance to the next fed prompt token (advance_state).
enum GraphKind { G_LOGITS = 0, G_HIDDEN = 1, G_TOKEN = 2, G_GREEDY = 3, G_FEED = 4, G_COUNT = 5 };
static inline bool device_token(int kind) { return kind == G_TOKEN || kind == G_GREEDY || kind == G_FEED; }
static inline int advance_mode(int kind) { return kind == G_GREEDY ? 2 : (kind == G_FEED ? 3 : 0); }

}  // namespace

struct talos_hip_ctx {
  talos_hip_cfg cfg{};
  uint32_t hd = 0, kv_dim = 0, group = 0, nsplit = 1, max_chunk = 1;
  hipStream_t stream = nullptr;
  std::string err;
  std::unordered_map<std::string, DevWeight> weights;
  size_t max_lds = 0;

  // device buffers
  bool acts_ready = false;
  std::vector<float*> kc, vc;
  int32_t* io = nullptr;  // [state: 16 int32][x: n_embd floats]
  float* x = nullptr;     // = io + 16
  float* q = nullptr;
  float* atty = nullptr;
  float* h = nullptr;
  float* logits = nullptr;
  float* hidden = nullptr;
  float* part = nullptr;
  uint32_t* count = nullptr;
  int32_t* tokens = nullptr;
  float* rope = nullptr;
  // generic-shape graph path: raw projections and the attention scores
  float* qraw = nullptr;   // [n_embd]
  float* kraw = nullptr;   // [kv_dim]
  float* vraw = nullptr;   // [kv_dim]
  float* graw = nullptr;   // [n_ff]
  float* uraw = nullptr;   // [n_ff]
  float* scores = nullptr; // [n_head][context_length]
  int path = TALOS_PATH_NONE;  // decided with the persistent-kernel set-up
  // sampling workspace (k_sample): keys twice and the probabilities for up
  // to samp_cap logits, the drawn token, the per-step draws and NLLs
  uint64_t* samp_ka = nullptr;
  uint64_t* samp_kb = nullptr;
  float* samp_pb = nullptr;
  uint32_t samp_cap = 0;
  uint32_t* samp_out = nullptr;
  float* samp_u = nullptr;
  uint32_t samp_u_cap = 0;
  float* nll = nullptr;
  uint32_t nll_cap = 0;
  // batched prompt processing (prefill.h): chunk buffers of pf_cap rows
  uint32_t pf_cap = 0;
  float *pf_x = nullptr, *pf_xn = nullptr, *pf_qr = nullptr, *pf_q = nullptr, *pf_att = nullptr;
  float *pf_kr = nullptr, *pf_vr = nullptr, *pf_g = nullptr, *pf_u = nullptr, *pf_h = nullptr;
  // split-f16 shadow of one layer's K/V rows for k_pf_attn16 (k_pf_kv16):
  // per KV head K [kv_cap][hd] and V^T in 64-position tiles, hi and lo;
  // kv_cap = the context length rounded up to 64
  uint16_t *pf_kh = nullptr, *pf_kl = nullptr, *pf_vh = nullptr, *pf_vl = nullptr;
  // the split-f16 GEMMs' inputs pf_xn, pf_att, pf_h as interleaved halves
  uint16_t *pf_xn16 = nullptr, *pf_att16 = nullptr, *pf_h16 = nullptr;
  uint32_t pf_kv_cap = 0;
  int32_t* pf_tok = nullptr;
  bool allow_batch = true;  // TALOS_HIP_BATCH=0: prompts one step per token
  bool pf_f16 = true;       // TALOS_HIP_PF16=0: Q4_0/Q8_0 prefill GEMMs on f32 MFMA instead of split f16
  bool pf_attn16 = true;    // TALOS_HIP_PFA16=0: prefill attention on f32 MFMA instead of split f16
  bool pf_tiled = true;     // TALOS_HIP_PF_TILED=0: the split-f16 GEMMs read the weights without tiled copies
  void* pf_tile_pool = nullptr;  // every tiled copy (one allocation), or null
  float* mv_x = nullptr;  // standalone matvec staging
  float* mv_out = nullptr;
  size_t mv_x_cap = 0, mv_out_cap = 0;

  // pinned host staging
  int32_t* h_io = nullptr;
  float* h_out = nullptr;
  int32_t* h_tokens = nullptr;

  hipGraphExec_t graph[G_COUNT] = {};
  // TALOS_HIP_GRAPHS=0 enqueues the kernels directly instead of replaying a
  // captured graph (same kernels; used under tracers that mishandle graphs).
  bool use_graphs = true;

  // Persistent one-kernel-per-token path (mega.h); TALOS_HIP_MEGA=0 turns it
  // off.  mega_fn is the instantiation for this model's formats, or null.
  bool allow_mega = true;
  bool mega_ready = false;
  const void* mega_fn = nullptr;
  uint32_t mega_blocks = 0;
  size_t mega_lds = 0;
  MegaLayer* d_layers = nullptr;
  uint32_t* d_sync = nullptr;
  float* mact = nullptr;   // per-layer activation slots
  float* mpart = nullptr;  // per-layer attention slice partials
  bool mega_prefetch = true;  // TALOS_HIP_PREFETCH=0 turns cross-barrier weight prefetch off
  bool one_hop = true;        // TALOS_HIP_BAR1=0: grid barriers through block 0's release word
  // The persistent kernel goes out as an ordinary launch: its grid is one
  // workgroup per CU and the set-up's occupancy check admits it only when at
  // least one fits per CU, so on an otherwise idle device every workgroup is resident
  // at once; a workgroup held back by other work on the device makes the
  // bounded barrier spins time out and the step report an error, never hang.
  // TALOS_HIP_COOP=1 uses hipLaunchCooperativeKernel instead (the runtime
  // then checks co-residency), which adds ~25 us per step on the MI355X.
  bool mega_coop = false;
  // TALOS_HIP_MFMA=1 runs the Q4_0 layer matvecs of the persistent kernel on
  // the matrix cores (mfma.h; parity-tested, not yet faster than the vector
  // path, so off by default).
  bool allow_mfma = false;
  bool mega_mfma = false;  // the chosen instantiation runs them on the matrix cores
  // TALOS_HIP_DOT4=0 keeps x in f32 for the Q4_0 / Q8_0 layer matvecs of the
  // persistent kernel instead of int8 planes with v_dot4 (the default).
  bool allow_dot4 = true;
  // TALOS_HIP_ATTN_DIRECT: longest sequence whose attention runs one item
  // per q head with no slice merge (0: always slices).
  int attn_direct = 256;
  // TALOS_HIP_DSPLIT=0 keeps the down-projection rows whole, =1 splits their
  // columns over the waves of a workgroup only (default: over workgroups).
  int allow_dsplit = 2;
  // TALOS_HIP_ATTN_WAIT=0 keeps a grid barrier in front of the attention.
  bool allow_attn_wait = true;
  int mega_mode = 0;  // MEGA_MM_* of the chosen instantiation
  uint32_t spin_limit = TALOS_SPIN_LIMIT;  // talos_hip_set_spin_limit
  MegaParams mp{};
};

namespace {

int fail(talos_hip_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  else g_create_error = buf;
  return code;
}

#define HIPCHK(c, call)                                                                         \
  do {                                                                                          \
    hipError_t e_ = (call);                                                                     \
    if (e_ != hipSuccess)                                                                       \
      return fail((c), TALOS_ERR_HIP, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),    \
                  __FILE__, __LINE__);                                                          \
  } while (0)

size_t block_elems(uint32_t t) { return t == TALOS_GGML_F32 ? 1 : t == TALOS_GGML_Q6_K ? 256 : 32; }
size_t block_bytes(uint32_t t) {
  return t == TALOS_GGML_F32 ? 4 : t == TALOS_GGML_Q8_0 ? 34 : t == TALOS_GGML_Q4_0 ? 18 : 210;
}
bool type_ok(uint32_t t) {
  return t == TALOS_GGML_F32 || t == TALOS_GGML_Q8_0 || t == TALOS_GGML_Q4_0 || t == TALOS_GGML_Q6_K;
}
size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

void destroy_graphs(talos_hip_ctx* c) {
  for (auto& g : c->graph)
    if (g) {
      (void)hipGraphExecDestroy(g);
      g = nullptr;
    }
}

// Repack GGUF blocks into the device layout of layout.h; returns the host
// image and the plane offsets.
struct Packed {
  std::vector<uint8_t> img;
  size_t q_off = 0, sc_off = 0, d_off = 0;
  uint32_t nchunk = 0;
};

void repack(const uint8_t* src, uint32_t type, size_t rows, size_t cols, Packed& P) {
  if (type == TALOS_GGML_F32) {  // rows zero-padded to a multiple of 16 floats
    const size_t ld = (cols + 15) & ~size_t(15);
    P.img.assign(rows * ld * 4, 0);
    for (size_t r = 0; r < rows; ++r) memcpy(P.img.data() + r * ld * 4, src + r * cols * 4, cols * 4);
    P.nchunk = (uint32_t)(ld / 4);
    return;
  }
  if (type == TALOS_GGML_Q8_0 || type == TALOS_GGML_Q4_0) {
    const size_t nb = cols / 32, bb = block_bytes(type), qb = type == TALOS_GGML_Q8_0 ? 32 : 16;
    P.nchunk = (uint32_t)nb;
    P.q_off = 0;
    P.d_off = align256(rows * nb * qb);
    P.img.assign(P.d_off + align256(rows * nb * 2), 0);
    uint8_t* q = P.img.data();
    uint16_t* d = reinterpret_cast<uint16_t*>(P.img.data() + P.d_off);
    for (size_t b = 0; b < rows * nb; ++b) {
      const uint8_t* s = src + b * bb;
      d[b] = (uint16_t)(s[0] | (s[1] << 8));
      if (type == TALOS_GGML_Q8_0) {
        for (int j = 0; j < 32; ++j) q[b * 32 + j] = s[2 + j] ^ 0x80;
      } else {
        memcpy(q + b * 16, s + 2, 16);
      }
    }
    return;
  }
  // Q6_K: super-block = ql[128] qh[64] sc[16] d(f16) (src/gguf/dtype.rs:94-102)
  const size_t nsb = cols / 256, nc = nsb * 4;
  P.nchunk = (uint32_t)nc;
  P.q_off = 0;
  P.sc_off = align256(rows * nc * 48);
  P.d_off = P.sc_off + align256(rows * nc * 4);
  P.img.assign(P.d_off + align256(rows * nsb * 2), 0);
  uint8_t* q = P.img.data();
  uint32_t* scw = reinterpret_cast<uint32_t*>(P.img.data() + P.sc_off);
  uint16_t* d = reinterpret_cast<uint16_t*>(P.img.data() + P.d_off);
  for (size_t r = 0; r < rows; ++r) {
    uint8_t* qrow = q + r * nc * 48;
    for (size_t sb = 0; sb < nsb; ++sb) {
      const uint8_t* s = src + (r * nsb + sb) * 210;
      const uint8_t *ql = s, *qh = s + 128, *sc = s + 192;
      d[r * nsb + sb] = (uint16_t)(s[208] | (s[209] << 8));
      for (int n = 0; n < 2; ++n)
        for (int g = 0; g < 2; ++g) {
          const size_t c = sb * 4 + n * 2 + g;
          memcpy(qrow + 0 * nc * 16 + c * 16, ql + n * 64 + g * 16, 16);
          memcpy(qrow + 1 * nc * 16 + c * 16, ql + n * 64 + 32 + g * 16, 16);
          memcpy(qrow + 2 * nc * 16 + c * 16, qh + n * 32 + g * 16, 16);
          const int is = n * 8 + g;
          scw[r * nc + c] = (uint32_t)sc[is] | ((uint32_t)sc[is + 2] << 8) | ((uint32_t)sc[is + 4] << 16) |
                            ((uint32_t)sc[is + 6] << 24);
        }
    }
  }
}

const DevWeight* find_w(talos_hip_ctx* c, const std::string& name) {
  auto it = c->weights.find(name);
  return it == c->weights.end() ? nullptr : &it->second;
}

int need_matrix(talos_hip_ctx* c, const std::string& name, size_t rows, size_t cols, const DevWeight** out) {
  const DevWeight* w = find_w(c, name);
  if (!w) return fail(c, TALOS_ERR_MISSING_WEIGHT, "weight \"%s\" is not resident", name.c_str());
  if (w->rows != rows || w->cols != cols)
    return fail(c, TALOS_ERR_SHAPE, "weight \"%s\" is [%zu, %zu], the model needs [%zu, %zu]", name.c_str(),
                w->rows, w->cols, rows, cols);
  *out = w;
  return TALOS_OK;
}

int need_norm(talos_hip_ctx* c, const std::string& name, size_t n, const float** out) {
  const DevWeight* w = find_w(c, name);
  if (!w) return fail(c, TALOS_ERR_MISSING_WEIGHT, "weight \"%s\" is not resident", name.c_str());
  if (w->type != TALOS_GGML_F32 || w->rows * w->cols != n)
    return fail(c, TALOS_ERR_SHAPE, "norm \"%s\" must be F32 with %zu elements", name.c_str(), n);
  *out = w->f32;
  return TALOS_OK;
}

int layout_need(uint32_t fmt) { return 1 << fmt_xlayout(fmt); }

// Staging rounds of the int8-plane x for a matvec over rows n long in
// format fmt, or 0 for f32 x (other formats, n beyond the planes,
// TALOS_HIP_DOT4=0).
int iq_rounds(const talos_hip_ctx* c, uint32_t fmt, size_t n) {
  return c->allow_dot4 && (fmt == TALOS_FMT_Q4_0 || fmt == TALOS_FMT_Q8_0) ? rows_iq_rounds(n) : 0;
}

// Instantiate KERN<format, rows-per-unit, U> for the runtime (fmt, U) pair.
#define TALOS_MV_U(KERN, F, U, ...)                                      \
  do {                                                                   \
    if ((U) >= 4) hipLaunchKernelGGL((KERN<F, mv_rows(F), 4>), __VA_ARGS__); \
    else if ((U) == 2) hipLaunchKernelGGL((KERN<F, mv_rows(F), 2>), __VA_ARGS__); \
    else hipLaunchKernelGGL((KERN<F, mv_rows(F), 1>), __VA_ARGS__);      \
  } while (0)
#define TALOS_MV_LAUNCH(KERN, fmt, U, ...)                                    \
  do {                                                                        \
    switch (fmt) {                                                            \
      case TALOS_FMT_F32: TALOS_MV_U(KERN, TALOS_FMT_F32, U, __VA_ARGS__); break;   \
      case TALOS_FMT_Q4_0: TALOS_MV_U(KERN, TALOS_FMT_Q4_0, U, __VA_ARGS__); break; \
      case TALOS_FMT_Q8_0: TALOS_MV_U(KERN, TALOS_FMT_Q8_0, U, __VA_ARGS__); break; \
      default: TALOS_MV_U(KERN, TALOS_FMT_Q6_K, U, __VA_ARGS__); break;       \
    }                                                                         \
  } while (0)

// KERN<F, mv_rows(F), U, XPlanes<NR>>: the int8-plane x staging for a
// Q4_0 / Q8_0 matrix whose rows are n long, NR = rows_iq_rounds(n).
#define TALOS_MV_IQ_NR(KERN, F, U_, nr, ...)                                                \
  do {                                                                                      \
    if ((nr) == 2) hipLaunchKernelGGL((KERN<F, mv_rows(F), U_, XPlanes<2>>), __VA_ARGS__); \
    else hipLaunchKernelGGL((KERN<F, mv_rows(F), U_, XPlanes<8>>), __VA_ARGS__);           \
  } while (0)
#define TALOS_MV_IQ_U(KERN, F, U, nr, ...)                             \
  do {                                                                 \
    if ((U) >= 4) TALOS_MV_IQ_NR(KERN, F, 4, nr, __VA_ARGS__);        \
    else if ((U) == 2) TALOS_MV_IQ_NR(KERN, F, 2, nr, __VA_ARGS__);   \
    else TALOS_MV_IQ_NR(KERN, F, 1, nr, __VA_ARGS__);                 \
  } while (0)
#define TALOS_MV_LAUNCH_IQ(KERN, fmt, U, nr, ...)                                             \
  do {                                                                                        \
    if ((fmt) == TALOS_FMT_Q4_0) TALOS_MV_IQ_U(KERN, TALOS_FMT_Q4_0, U, nr, __VA_ARGS__);     \
    else TALOS_MV_IQ_U(KERN, TALOS_FMT_Q8_0, U, nr, __VA_ARGS__);                             \
  } while (0)

// Let kernel k take up to `bytes` of LDS in all (dynamic plus its own static
// arrays).  A refused request leaves the kernel at the default limit, and
// the runtime's last-error state is cleared so that it does not surface in
// a later hipGetLastError.
void set_max_lds(const void* k, int bytes) {
  hipFuncAttributes a{};
  int dyn = bytes;
  if (hipFuncGetAttributes(&a, k) == hipSuccess) dyn -= (int)a.sharedSizeBytes;
  if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess) (void)hipGetLastError();
}

template <uint32_t F>
void set_lds_attr_fmt(int bytes) {
  for (const void* k : {(const void*)k_qkv<F, mv_rows(F), 1>, (const void*)k_qkv<F, mv_rows(F), 2>,
                        (const void*)k_qkv<F, mv_rows(F), 4>, (const void*)k_rows<F, mv_rows(F), 1>,
                        (const void*)k_rows<F, mv_rows(F), 2>, (const void*)k_rows<F, mv_rows(F), 4>,
                        (const void*)k_gateup<F, mv_rows(F), 1>, (const void*)k_gateup<F, mv_rows(F), 2>,
                        (const void*)k_gateup<F, mv_rows(F), 4>})
    set_max_lds(k, bytes);
}

void plan(uint32_t units, uint32_t& upw, uint32_t& blocks) {
  const uint32_t max_waves = 1024 * 4;
  upw = (units + max_waves - 1) / max_waves;
  if (upw == 0) upw = 1;
  const uint32_t waves = (units + upw - 1) / upw;
  blocks = (waves + 3) / 4;
  if (blocks == 0) blocks = 1;
}

int alloc_acts(talos_hip_ctx* c) {
  if (c->acts_ready) return TALOS_OK;
  const auto& cf = c->cfg;
  const size_t kvb = (size_t)cf.context_length * c->kv_dim * 4;
  c->kc.assign(cf.n_layer, nullptr);
  c->vc.assign(cf.n_layer, nullptr);
  for (uint32_t l = 0; l < cf.n_layer; ++l) {
    HIPCHK(c, hipMalloc(&c->kc[l], kvb));
    HIPCHK(c, hipMalloc(&c->vc[l], kvb));
    HIPCHK(c, hipMemsetAsync(c->kc[l], 0, kvb, c->stream));
    HIPCHK(c, hipMemsetAsync(c->vc[l], 0, kvb, c->stream));
  }
  HIPCHK(c, hipMalloc(&c->io, 64 + (size_t)cf.n_embd * 4));
  HIPCHK(c, hipMemsetAsync(c->io, 0, 64 + (size_t)cf.n_embd * 4, c->stream));
  c->x = reinterpret_cast<float*>(c->io + 16);
  HIPCHK(c, hipMalloc(&c->q, (size_t)cf.n_embd * 4));
  HIPCHK(c, hipMalloc(&c->atty, (size_t)cf.n_embd * 4));
  // past the heads (n_embd > n_head * head_dim) the attention output stays 0
  HIPCHK(c, hipMemsetAsync(c->atty, 0, (size_t)cf.n_embd * 4, c->stream));
  HIPCHK(c, hipMalloc(&c->qraw, (size_t)cf.n_embd * 4));
  HIPCHK(c, hipMalloc(&c->kraw, (size_t)c->kv_dim * 4));
  HIPCHK(c, hipMalloc(&c->vraw, (size_t)c->kv_dim * 4));
  HIPCHK(c, hipMalloc(&c->graw, (size_t)cf.n_ff * 4));
  HIPCHK(c, hipMalloc(&c->uraw, (size_t)cf.n_ff * 4));
  HIPCHK(c, hipMalloc(&c->scores, (size_t)cf.n_head * cf.context_length * 4));
  HIPCHK(c, hipMalloc(&c->h, (size_t)cf.n_ff * 4));
  HIPCHK(c, hipMalloc(&c->logits, (size_t)cf.vocab_size * 4));
  HIPCHK(c, hipMalloc(&c->hidden, (size_t)cf.n_embd * 4));
  const size_t part_n = (size_t)cf.n_head_kv * c->nsplit * c->group * (c->hd + 2);
  HIPCHK(c, hipMalloc(&c->part, part_n * 4));
  HIPCHK(c, hipMalloc(&c->count, (size_t)cf.n_head_kv * 4));
  HIPCHK(c, hipMemsetAsync(c->count, 0, (size_t)cf.n_head_kv * 4, c->stream));
  HIPCHK(c, hipMalloc(&c->tokens, (size_t)cf.context_length * 4));
  HIPCHK(c, hipHostMalloc(&c->h_io, 64 + (size_t)cf.n_embd * 4, hipHostMallocDefault));
  HIPCHK(c, hipHostMalloc(&c->h_out, (size_t)std::max(cf.vocab_size, cf.n_embd) * 4, hipHostMallocDefault));
  HIPCHK(c, hipHostMalloc(&c->h_tokens, (size_t)cf.context_length * 4, hipHostMallocDefault));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->acts_ready = true;
  return TALOS_OK;
}

// ---- per-kernel enqueue (shared by graph capture and kernel timing)

struct LayerW {
  const DevWeight *q, *k, *v, *o, *g, *u, *d;
  const float *an, *fn;
};

int layer_weights(talos_hip_ctx* c, uint32_t l, LayerW* w) {
  const auto& cf = c->cfg;
  const uint32_t n = cf.n_embd, kvd = c->kv_dim;
  char nm[128];
  int rc;
#define NM(s) (snprintf(nm, sizeof nm, "blk.%u." s, l), std::string(nm))
  if ((rc = need_norm(c, NM("attn_norm.weight"), n, &w->an)) || (rc = need_matrix(c, NM("attn_q.weight"), n, n, &w->q)) ||
      (rc = need_matrix(c, NM("attn_k.weight"), kvd, n, &w->k)) ||
      (rc = need_matrix(c, NM("attn_v.weight"), kvd, n, &w->v)) ||
      (rc = need_matrix(c, NM("attn_output.weight"), n, n, &w->o)) ||
      (rc = need_norm(c, NM("ffn_norm.weight"), n, &w->fn)) ||
      (rc = need_matrix(c, NM("ffn_gate.weight"), cf.n_ff, n, &w->g)) ||
      (rc = need_matrix(c, NM("ffn_up.weight"), cf.n_ff, n, &w->u)) ||
      (rc = need_matrix(c, NM("ffn_down.weight"), n, cf.n_ff, &w->d)))
    return rc;
#undef NM
  return TALOS_OK;
}

void enq_qkv(talos_hip_ctx* c, uint32_t l, const LayerW& w) {
  const uint32_t n = c->cfg.n_embd, kvd = c->kv_dim;
  QKVParams P{};
  P.m[0] = w.q->mat;
  P.m[1] = w.k->mat;
  P.m[2] = w.v->mat;
  const int R = mv_rows(w.q->mat.fmt);
  P.units[0] = n / R;
  P.units[1] = kvd / R;
  P.units[2] = kvd / R;
  P.x = c->x;
  P.norm_w = w.an;
  P.eps = c->cfg.rms_eps;
  P.n = n;
  P.q_out = c->q;
  P.kc = c->kc[l];
  P.vc = c->vc[l];
  P.kv_dim = kvd;
  P.hd = c->hd;
  P.rope = c->rope;
  P.state = c->io;
  P.need = layout_need(w.q->mat.fmt) | layout_need(w.k->mat.fmt) | layout_need(w.v->mat.fmt);
  uint32_t blocks;
  plan(P.units[0] + P.units[1] + P.units[2], P.upw, blocks);
  if (const int nr = iq_rounds(c, w.q->mat.fmt, n))
    TALOS_MV_LAUNCH_IQ(k_qkv, w.q->mat.fmt, mv_u(w.q->mat.nchunk), nr, dim3(blocks), dim3(256), rows_iq_lds_bytes(n),
                       c->stream, P);
  else
    TALOS_MV_LAUNCH(k_qkv, w.q->mat.fmt, mv_u(w.q->mat.nchunk), dim3(blocks), dim3(256), stage_lds_bytes(n, P.need),
                    c->stream, P);
}

// The layer forms the graph path can fuse: q/k/v in one kernel with RoPE in
// its epilogue (one format, whole heads, even head_dim, rows in whole
// units), gate/up in one kernel (one format); attention in one kernel per
// KV-head slice (head_dim a multiple of 16 in [32, 128], group <= 8).
bool fused_qkv(const talos_hip_ctx* c, const LayerW& w) {
  const uint32_t R = (uint32_t)mv_rows(w.q->mat.fmt), n = c->cfg.n_embd;
  return w.k->type == w.q->type && w.v->type == w.q->type && c->hd % 2 == 0 && n == c->cfg.n_head * c->hd &&
         n % R == 0 && c->kv_dim % R == 0;
}
bool fused_gateup(const LayerW& w) { return w.u->type == w.g->type; }
bool fast_attn(const talos_hip_ctx* c) {
  return c->hd % 16 == 0 && c->hd >= 32 && c->hd <= 128 && c->group <= TALOS_MAX_GROUP &&
         attn_lds_bytes(c->hd, c->group, c->nsplit, c->max_chunk) <= c->max_lds;
}

// out[rows] = W rmsnorm(x) (norm_w non-null) or W x, no residual.
void enq_rows(talos_hip_ctx* c, const DevWeight* w, const float* x, uint32_t n, const float* norm_w, float* out) {
  RowParams R{};
  R.m = w->mat;
  R.x = x;
  R.n = n;
  R.norm_w = norm_w;
  R.eps = c->cfg.rms_eps;
  R.out = out;
  R.accumulate = 0;
  R.units = (uint32_t)((w->rows + mv_rows(w->mat.fmt) - 1) / mv_rows(w->mat.fmt));
  R.need = layout_need(w->mat.fmt);
  uint32_t blocks;
  plan(R.units, R.upw, blocks);
  if (const int nr = iq_rounds(c, w->mat.fmt, n))
    TALOS_MV_LAUNCH_IQ(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), nr, dim3(blocks), dim3(256), rows_iq_lds_bytes(n),
                       c->stream, R);
  else
    TALOS_MV_LAUNCH(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), dim3(blocks), dim3(256), stage_lds_bytes(n, R.need),
                    c->stream, R);
}

// q/k/v of different formats or shapes the fused epilogue does not take:
// three raw projections, then RoPE and the cache append.
void enq_qkv_split(talos_hip_ctx* c, uint32_t l, const LayerW& w) {
  const uint32_t n = c->cfg.n_embd;
  enq_rows(c, w.q, c->x, n, w.an, c->qraw);
  enq_rows(c, w.k, c->x, n, w.an, c->kraw);
  enq_rows(c, w.v, c->x, n, w.an, c->vraw);
  const uint32_t m = std::max(n, c->kv_dim);
  hipLaunchKernelGGL(k_rope_qkv, dim3((m + 255) / 256), dim3(256), 0, c->stream, c->qraw, c->kraw, c->vraw, c->q,
                     c->kc[l], c->vc[l], c->rope, (const int32_t*)c->io, n, c->cfg.n_head, c->hd, c->kv_dim);
}

void enq_gateup_split(talos_hip_ctx* c, const LayerW& w) {
  const uint32_t n = c->cfg.n_embd, ff = c->cfg.n_ff;
  enq_rows(c, w.g, c->x, n, w.fn, c->graw);
  enq_rows(c, w.u, c->x, n, w.fn, c->uraw);
  hipLaunchKernelGGL(k_swiglu, dim3((ff + 255) / 256), dim3(256), 0, c->stream, c->graw, c->uraw, c->h, ff);
}

// Attention of any head_dim and group: scores, softmax, weighted V rows.
void enq_attn_generic(talos_hip_ctx* c, uint32_t l) {
  const auto& cf = c->cfg;
  const int32_t* st = (const int32_t*)c->io;
  hipLaunchKernelGGL(k_attn_scores, dim3(cf.n_head, (cf.context_length + 255) / 256), dim3(256), c->hd * 4, c->stream,
                     c->q, c->kc[l], c->scores, st, c->hd, c->kv_dim, c->group, cf.context_length,
                     1.0f / sqrtf((float)c->hd));
  hipLaunchKernelGGL(k_attn_softmax, dim3(cf.n_head), dim3(256), 0, c->stream, c->scores, st, cf.context_length);
  hipLaunchKernelGGL(k_attn_out, dim3(cf.n_head, (c->hd + 63) / 64), dim3(256), 0, c->stream, c->scores, c->vc[l],
                     c->atty, st, c->hd, c->kv_dim, c->group, cf.context_length);
}

void enq_attn(talos_hip_ctx* c, uint32_t l) {
  AttnParams A{};
  A.q = c->q;
  A.kc = c->kc[l];
  A.vc = c->vc[l];
  A.out = c->atty;
  A.part = c->part;
  A.count = c->count;
  A.state = c->io;
  A.hd = c->hd;
  A.kv_dim = c->kv_dim;
  A.group = c->group;
  A.nsplit = c->nsplit;
  A.max_chunk = c->max_chunk;
  A.scale = 1.0f / sqrtf((float)c->hd);
  const dim3 grid(c->cfg.n_head_kv, c->nsplit);
  const size_t lds = attn_lds_bytes(c->hd, c->group, c->nsplit, c->max_chunk);
  switch (c->hd / 16) {
    case 2: hipLaunchKernelGGL(k_attn<2>, grid, dim3(256), lds, c->stream, A); break;
    case 3: hipLaunchKernelGGL(k_attn<3>, grid, dim3(256), lds, c->stream, A); break;
    case 4: hipLaunchKernelGGL(k_attn<4>, grid, dim3(256), lds, c->stream, A); break;
    case 5: hipLaunchKernelGGL(k_attn<5>, grid, dim3(256), lds, c->stream, A); break;
    case 6: hipLaunchKernelGGL(k_attn<6>, grid, dim3(256), lds, c->stream, A); break;
    case 7: hipLaunchKernelGGL(k_attn<7>, grid, dim3(256), lds, c->stream, A); break;
    default: hipLaunchKernelGGL(k_attn<8>, grid, dim3(256), lds, c->stream, A); break;
  }
}

void enq_resid(talos_hip_ctx* c, const DevWeight* w, const float* x, uint32_t n, float* out) {
  RowParams R{};
  R.m = w->mat;
  R.x = x;
  R.n = n;
  R.out = out;
  R.accumulate = 1;
  R.units = (uint32_t)((w->rows + mv_rows(w->mat.fmt) - 1) / mv_rows(w->mat.fmt));
  R.need = layout_need(w->mat.fmt);
  uint32_t blocks;
  plan(R.units, R.upw, blocks);
  if (const int nr = iq_rounds(c, w->mat.fmt, n))
    TALOS_MV_LAUNCH_IQ(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), nr, dim3(blocks), dim3(256), rows_iq_lds_bytes(n),
                       c->stream, R);
  else
    TALOS_MV_LAUNCH(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), dim3(blocks), dim3(256), stage_lds_bytes(n, R.need),
                    c->stream, R);
}

void enq_gateup(talos_hip_ctx* c, const LayerW& w) {
  GateUpParams G{};
  G.g = w.g->mat;
  G.u = w.u->mat;
  G.x = c->x;
  G.norm_w = w.fn;
  G.eps = c->cfg.rms_eps;
  G.n = c->cfg.n_embd;
  G.h = c->h;
  const uint32_t pr = mv_rows(w.g->mat.fmt) / 2;
  G.units = (c->cfg.n_ff + pr - 1) / pr;
  G.need = layout_need(w.g->mat.fmt) | layout_need(w.u->mat.fmt);
  uint32_t blocks;
  plan(G.units, G.upw, blocks);
  if (const int nr = iq_rounds(c, w.g->mat.fmt, G.n))
    TALOS_MV_LAUNCH_IQ(k_gateup, w.g->mat.fmt, mv_u(w.g->mat.nchunk), nr, dim3(blocks), dim3(256),
                       rows_iq_lds_bytes(G.n), c->stream, G);
  else
    TALOS_MV_LAUNCH(k_gateup, w.g->mat.fmt, mv_u(w.g->mat.nchunk), dim3(blocks), dim3(256),
                    stage_lds_bytes(G.n, G.need), c->stream, G);
}

void enq_output(talos_hip_ctx* c, const DevWeight* wout, const float* onorm) {
  RowParams R{};
  R.m = wout->mat;
  R.x = c->x;
  R.norm_w = onorm;
  R.eps = c->cfg.rms_eps;
  R.n = c->cfg.n_embd;
  R.out = c->logits;
  R.accumulate = 0;
  R.units = (c->cfg.vocab_size + mv_rows(wout->mat.fmt) - 1) / mv_rows(wout->mat.fmt);
  R.need = layout_need(wout->mat.fmt);
  uint32_t blocks;
  plan(R.units, R.upw, blocks);
  if (const int nr = iq_rounds(c, wout->mat.fmt, R.n))
    TALOS_MV_LAUNCH_IQ(k_rows, wout->mat.fmt, mv_u(wout->mat.nchunk), nr, dim3(blocks), dim3(256),
                       rows_iq_lds_bytes(R.n), c->stream, R);
  else
    TALOS_MV_LAUNCH(k_rows, wout->mat.fmt, mv_u(wout->mat.nchunk), dim3(blocks), dim3(256),
                    stage_lds_bytes(R.n, R.need), c->stream, R);
}

// Enqueue one token step on the stream.
int enqueue_token(talos_hip_ctx* c, GraphKind kind) {
  const auto& cf = c->cfg;
  const uint32_t n = cf.n_embd;
  int rc;
  if (device_token(kind)) {
    const DevWeight* emb;
    if ((rc = need_matrix(c, "token_embd.weight", cf.vocab_size, n, &emb))) return rc;
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, c->stream, emb->mat, (const int32_t*)c->io, c->x);
  }
  for (uint32_t l = 0; l < cf.n_layer; ++l) {
    LayerW w;
    if ((rc = layer_weights(c, l, &w))) return rc;
    if (fused_qkv(c, w)) enq_qkv(c, l, w);
    else enq_qkv_split(c, l, w);
    if (fast_attn(c)) enq_attn(c, l);
    else enq_attn_generic(c, l);
    enq_resid(c, w.o, c->atty, n, c->x);
    if (fused_gateup(w)) enq_gateup(c, w);
    else enq_gateup_split(c, w);
    enq_resid(c, w.d, c->h, cf.n_ff, c->x);
  }
  const float* onorm;
  if ((rc = need_norm(c, "output_norm.weight", n, &onorm))) return rc;
  if (kind == G_HIDDEN) {
    hipLaunchKernelGGL(k_norm, dim3(1), dim3(256), 0, c->stream, c->x, onorm, cf.rms_eps, n, c->hidden);
    return TALOS_OK;
  }
  const DevWeight* wout;
  if ((rc = need_matrix(c, "output.weight", cf.vocab_size, n, &wout))) return rc;
  enq_output(c, wout, onorm);
  if (device_token(kind))
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, c->stream, c->logits, cf.vocab_size, c->io, c->tokens,
                       advance_mode(kind));
  return TALOS_OK;
}

int mega_setup(talos_hip_ctx* c);

// The graph path's form for the resident weights: every layer fused and the
// one-kernel attention, or some generic-shape kernels.
int graph_path_kind(talos_hip_ctx* c, int* kind) {
  *kind = fast_attn(c) ? TALOS_PATH_GRAPH : TALOS_PATH_GRAPH_GENERIC;
  for (uint32_t l = 0; l < c->cfg.n_layer; ++l) {
    LayerW w;
    int rc = layer_weights(c, l, &w);
    if (rc) return rc;
    if (!fused_qkv(c, w) || !fused_gateup(w)) *kind = TALOS_PATH_GRAPH_GENERIC;
  }
  return TALOS_OK;
}

// Buffers and the persistent-kernel set-up for the resident weights; fixes
// which path the token step takes.
int prepare(talos_hip_ctx* c) {
  int rc;
  if ((rc = alloc_acts(c))) return rc;
  if ((rc = mega_setup(c))) return rc;
  if (c->mega_fn) c->path = TALOS_PATH_PERSISTENT;
  else if ((rc = graph_path_kind(c, &c->path))) return rc;
  return TALOS_OK;
}

int get_graph(talos_hip_ctx* c, GraphKind kind, hipGraphExec_t* out) {
  int rc;
  if ((rc = prepare(c))) return rc;
  if (c->mega_fn) {
    *out = nullptr;
    return TALOS_OK;
  }
  if (!c->use_graphs) {
    *out = nullptr;
    return TALOS_OK;
  }
  if (c->graph[kind]) {
    *out = c->graph[kind];
    return TALOS_OK;
  }
  hipGraph_t g = nullptr;
  HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  rc = enqueue_token(c, kind);
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return fail(c, TALOS_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(&c->graph[kind], g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail(c, TALOS_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  *out = c->graph[kind];
  return TALOS_OK;
}

int set_state(talos_hip_ctx* c, uint32_t token, uint32_t pos);

// After a step has synchronized with h_io holding the device state block:
// a timed-out grid barrier in the persistent kernel leaves ST_ERR set.
int check_device_err(talos_hip_ctx* c) {
  if (c->h_io[ST_ERR] != 0)
    return fail(c, TALOS_ERR_HIP, "persistent decode kernel: a grid barrier timed out (results invalid)");
  return TALOS_OK;
}

// ---- persistent path

// The instantiations this library carries (mega_inst_*.hip): the 7B-shape
// Q4_0 model on the matrix cores (n = 4096, ff = 14336 -> 4 and 14 tiles per
// wave), and the vector-ALU streaming path with int8-plane x (Q4_0 / Q8_0)
// or f32 x for the tested shapes of each format.
const void* mega_kernel_for(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  static const MegaInstFn fns[] = MEGA_INST_FNS;
  for (MegaInstFn f : fns)
    if (const void* k = f(lf, of, un, uf, uo, dpl, mm)) return k;
  return nullptr;
}

// Prepare the persistent kernel for the resident weights; returns OK with
// c->mega_fn == nullptr when this model has no instantiation.
int mega_setup(talos_hip_ctx* c) {
  if (c->mega_ready) return TALOS_OK;
  c->mega_fn = nullptr;
  if (!c->allow_mega) {
    c->mega_ready = true;
    return TALOS_OK;
  }
  int rc;
  const auto& cf = c->cfg;
  std::vector<MegaLayer> L(cf.n_layer);
  uint32_t lf = 0;
  for (uint32_t l = 0; l < cf.n_layer; ++l) {
    LayerW w;
    if ((rc = layer_weights(c, l, &w))) return rc;
    const DevWeight* ms[] = {w.q, w.k, w.v, w.o, w.g, w.u, w.d};
    if (l == 0) lf = w.q->mat.fmt;
    for (const DevWeight* m : ms)
      if (m->mat.fmt != lf) {
        c->mega_ready = true;  // mixed formats: graph path
        return TALOS_OK;
      }
    L[l] = MegaLayer{w.q->mat, w.k->mat, w.v->mat, w.o->mat, w.g->mat, w.u->mat, w.d->mat,
                     w.an, w.fn, c->kc[l], c->vc[l]};
  }
  const DevWeight *wout, *emb;
  const float* onorm;
  if ((rc = need_matrix(c, "output.weight", cf.vocab_size, cf.n_embd, &wout)) ||
      (rc = need_norm(c, "output_norm.weight", cf.n_embd, &onorm)) ||
      (rc = need_matrix(c, "token_embd.weight", cf.vocab_size, cf.n_embd, &emb)))
    return rc;
  LayerW w0;
  if ((rc = layer_weights(c, 0, &w0))) return rc;
  int dev0 = cf.device;
  hipDeviceProp_t prop0;
  HIPCHK(c, hipGetDeviceProperties(&prop0, dev0));
  const uint32_t nblk = (uint32_t)prop0.multiProcessorCount;
  auto gpb = [&](uint32_t groups) { return (groups + nblk - 1) / nblk; };
  // Matrix-core layer phases: Q4_0 layers, rows of whole 1024-element tiles
  // per wave, at most MEGA_GPB 16-row groups per block in every phase.
  const bool mf = c->allow_mfma && lf == TALOS_FMT_Q4_0 && cf.n_embd % 1024 == 0 && cf.n_ff % 1024 == 0 &&
                  c->kv_dim % 16 == 0 && gpb((cf.n_embd + 2 * c->kv_dim) / 16) <= MEGA_GPB &&
                  gpb(cf.n_ff / 8) <= MEGA_GPB && gpb(cf.n_embd / 16) <= MEGA_GPB;
  const void* fn = nullptr;
  c->mega_mode = MEGA_MM_F32;
  if (mf) {
    fn = mega_kernel_for(lf, wout->mat.fmt, (int)(cf.n_embd / 1024), (int)(cf.n_ff / 1024), mv_u(wout->mat.nchunk),
                         (int)(c->hd / 16), MEGA_MM_MFMA);
    if (fn) c->mega_mode = MEGA_MM_MFMA;
  }
  c->mega_mfma = fn != nullptr;
  // down rows (two per unit) take up to 4 chunk-steps per item for Q4_0 with
  // int8-plane x, 2 otherwise (Q8_0 has twice the bytes per chunk; f32 x
  // twice the registers): about 9 KB in flight per wave
  const int un = mv_u(w0.q->mat.nchunk), uo = mv_u(wout->mat.nchunk);
  const int ud = mv_u(w0.d->mat.nchunk);
  // (int8-plane x also keeps each lane's x of an n-wide row in registers,
  // so such a row must fit one item: n / 32 <= un * 64)
  if (!fn && c->allow_dot4 && (lf == TALOS_FMT_Q4_0 || lf == TALOS_FMT_Q8_0) &&
      cf.n_embd / 32 <= (uint32_t)un * 64) {
    fn = mega_kernel_for(lf, wout->mat.fmt, un, std::min(ud, lf == TALOS_FMT_Q4_0 ? 4 : 2), uo, (int)(c->hd / 16),
                         MEGA_MM_DOT4);
    if (fn) c->mega_mode = MEGA_MM_DOT4;
  }
  if (!fn) fn = mega_kernel_for(lf, wout->mat.fmt, un, std::min(ud, 2), uo, (int)(c->hd / 16), MEGA_MM_F32);
  if (!fn) {
    c->mega_ready = true;
    return TALOS_OK;
  }
  int dev = cf.device;
  hipDeviceProp_t prop;
  HIPCHK(c, hipGetDeviceProperties(&prop, dev));
  // Shapes the persistent kernel handles: batched staging of up to
  // MEGA_STAGE_MAX floats, head_dim a multiple of 16, at most MEGA_ATTN_HG
  // q heads per KV head.
  if (cf.n_embd % 16 || cf.n_ff % 16 || std::max(cf.n_embd, cf.n_ff) > MEGA_STAGE_MAX || c->hd % 16 ||
      c->group > MEGA_ATTN_HG || cf.n_embd != cf.n_head * c->hd) {
    c->mega_ready = true;
    return TALOS_OK;
  }
  // LDS: x staging for the widest input, or the attention scratch.
  const size_t st = stage_lds_bytes((int)std::max(cf.n_embd, cf.n_ff), 3);
  const uint32_t msplit = mega_attn_max_splits(cf.n_head_kv, (uint32_t)prop.multiProcessorCount);
  const size_t at = mega_attn_lds_floats(c->hd, c->group) * 4;
  c->mega_lds = std::max(st, at);
  if (c->mega_mode != MEGA_MM_F32)
    c->mega_lds = std::max(c->mega_lds, xq_lds_bytes((int)std::max(cf.n_embd, cf.n_ff), MEGA_GPB, MEGA_NW));
  if (c->mega_lds > c->max_lds) {
    c->mega_ready = true;
    return TALOS_OK;
  }
  HIPCHK(c, hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)c->mega_lds));
  int per_cu = 0;
  HIPCHK(c, hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, MEGA_NT, c->mega_lds));
  if (per_cu < 1) {
    c->mega_ready = true;
    return TALOS_OK;
  }
  c->mega_blocks = (uint32_t)prop.multiProcessorCount;
  if (!c->d_layers) HIPCHK(c, hipMalloc(&c->d_layers, sizeof(MegaLayer) * cf.n_layer));
  HIPCHK(c, hipMemcpy(c->d_layers, L.data(), sizeof(MegaLayer) * cf.n_layer, hipMemcpyHostToDevice));
  const uint32_t lstride = mega_lstride(cf.n_embd, cf.n_ff);
  const size_t pstride = (size_t)cf.n_head_kv * msplit * c->group * (c->hd + 2);
  if (!c->mact) HIPCHK(c, hipMalloc(&c->mact, mega_act_floats(cf.n_layer, cf.n_embd, cf.n_ff) * 4));
  if (!c->mpart) HIPCHK(c, hipMalloc(&c->mpart, (size_t)cf.n_layer * pstride * 4));
  if (!c->d_sync) {
    const size_t words = mega_sync_words(c->mega_blocks);
    HIPCHK(c, hipMalloc(&c->d_sync, words * 4));
    HIPCHK(c, hipMemset(c->d_sync, 0, words * 4));
  }
  MegaParams& P = c->mp;
  P = MegaParams{};
  P.layers = c->d_layers;
  P.n_layer = cf.n_layer;
  P.out_w = wout->mat;
  P.out_norm = onorm;
  P.embd = emb->mat;
  P.n = cf.n_embd;
  P.ff = cf.n_ff;
  P.kv_dim = c->kv_dim;
  P.hd = c->hd;
  P.group = c->group;
  P.n_kv = cf.n_head_kv;
  P.vocab = cf.vocab_size;
  P.eps = cf.rms_eps;
  P.scale = 1.0f / sqrtf((float)c->hd);
  P.rope = c->rope;
  P.x = c->x;
  P.act = c->mact;
  P.np = mega_np(cf.n_embd);
  P.lstride = lstride;
  P.logits = c->logits;
  P.hidden = c->hidden;
  P.part = c->mpart;
  P.pstride = pstride;
  P.prefetch = c->mega_prefetch ? 1 : 0;
  P.one_hop = c->one_hop && c->mega_blocks <= 8192 ? 1 : 0;
  P.count = c->count;
  P.state = c->io;
  P.tokens = c->tokens;
  P.sync = c->d_sync;
  P.nsplit = msplit;
  P.max_chunk = MEGA_ATTN_STEP;
  P.attn_direct = c->attn_direct;
  P.attn_wait = c->allow_attn_wait ? 1 : 0;
  {
    // split down-projection: whole quarters of the row chunks that fit one
    // item, and an even number of rows per team of MEGA_DSPLIT waves
    const uint32_t teams = c->mega_blocks * (MEGA_NW / MEGA_DSPLIT), dch = cf.n_ff / 32;
    const uint32_t rpt = cf.n_embd / teams;
    const bool quarters = c->mega_mode == MEGA_MM_DOT4 && c->allow_dsplit > 0 && dch % MEGA_DSPLIT == 0 &&
                          dch / MEGA_DSPLIT <= (uint32_t)mv_u(cf.n_embd / 32) * 64;
    P.dsplit = quarters && rpt * teams == cf.n_embd && rpt % 2 == 0 && rpt <= MEGA_DSPLIT_ROWS &&
               rpt * (MEGA_NW / MEGA_DSPLIT) <= MEGA_NT;
    // the quarters on different workgroups: whole groups of four blocks, an
    // even number of rows per wave
    const uint32_t groups = c->mega_blocks / MEGA_DSPLIT;
    if (quarters && c->allow_dsplit == 2 && c->mega_blocks % MEGA_DSPLIT == 0 && cf.n_embd % groups == 0 &&
        (cf.n_embd / groups) % (2 * MEGA_NW) == 0)
      P.dsplit = 2;
  }
  c->mega_fn = fn;
  c->mega_ready = true;
  return TALOS_OK;
}

int mega_launch(talos_hip_ctx* c, GraphKind kind, uint64_t* timeline = nullptr) {
  MegaParams P = c->mp;
  P.timeline = timeline;
  P.spin_limit = c->spin_limit;
  P.embed = device_token(kind);
  P.hidden_only = kind == G_HIDDEN;
  P.argmax = device_token(kind) ? (kind == G_TOKEN ? 1 : advance_mode(kind)) : 0;
  void* args[] = {&P};
  if (c->mega_coop)
    HIPCHK(c, hipLaunchCooperativeKernel(c->mega_fn, dim3(c->mega_blocks), dim3(MEGA_NT), args,
                                         (unsigned)c->mega_lds, c->stream));
  else
    HIPCHK(c, hipLaunchKernel(c->mega_fn, dim3(c->mega_blocks), dim3(MEGA_NT), args, (unsigned)c->mega_lds,
                              c->stream));
  return TALOS_OK;
}

// One token step: replay the captured graph, or enqueue the kernels.
int run_step(talos_hip_ctx* c, GraphKind kind, hipGraphExec_t g) {
  if (c->mega_fn) return mega_launch(c, kind);
  if (g) {
    HIPCHK(c, hipGraphLaunch(g, c->stream));
    return TALOS_OK;
  }
  int rc = enqueue_token(c, kind);
  if (rc) return rc;
  HIPCHK(c, hipGetLastError());
  return TALOS_OK;
}

// Grow the sampling workspace to n logits.
int samp_reserve(talos_hip_ctx* c, uint32_t n) {
  if (!c->samp_out) HIPCHK(c, hipMalloc(&c->samp_out, 64));
  if (c->samp_cap >= n) return TALOS_OK;
  (void)hipStreamSynchronize(c->stream);
  for (void* p : {(void*)c->samp_ka, (void*)c->samp_kb, (void*)c->samp_pb})
    if (p) (void)hipFree(p);
  c->samp_ka = c->samp_kb = nullptr;
  c->samp_pb = nullptr;
  c->samp_cap = 0;
  HIPCHK(c, hipMalloc(&c->samp_ka, (size_t)n * 8));
  HIPCHK(c, hipMalloc(&c->samp_kb, (size_t)n * 8));
  HIPCHK(c, hipMalloc(&c->samp_pb, (size_t)n * 4));
  c->samp_cap = n;
  return TALOS_OK;
}

int samp_check(talos_hip_ctx* c, float temperature, float top_p, float u) {
  if (std::isnan(temperature)) return fail(c, TALOS_ERR_ARG, "temperature is NaN");
  if (!(u >= 0.f && u < 1.f)) return fail(c, TALOS_ERR_ARG, "u %g outside [0, 1)", (double)u);
  (void)top_p;
  return TALOS_OK;
}

void enq_sample(talos_hip_ctx* c, const float* logits, uint32_t n, float temperature, uint32_t top_k, float top_p,
                float u, const float* u_dev, uint64_t* ka, uint64_t* kb, float* pb, uint32_t* out, int32_t* state,
                int32_t* tokens) {
  SampleArgs A{};
  A.logits = logits;
  A.n = n;
  A.temperature = temperature;
  A.top_k = top_k;
  A.top_p = top_p;
  A.u = u;
  A.u_dev = u_dev;
  A.ka = ka;
  A.kb = kb;
  A.pb = pb;
  A.out = out;
  A.state = state;
  A.tokens = tokens;
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(SAMPLE_NT), 0, c->stream, A);
}

// ---- batched prompt processing (prefill.h)

#define PF_CHUNK 1024

// The batched path takes layer matrices of every format (F32, Q4_0, Q8_0,
// Q6_K) and attention heads of a multiple of 16 up to 256 that tile n_embd
// exactly, with groups of at most 8.
int pf_supported(talos_hip_ctx* c, bool* ok) {
  *ok = false;
  if (!c->allow_batch || c->hd % 16 || c->hd > 256 || c->group > 8 || c->cfg.n_embd != c->cfg.n_head * c->hd ||
      c->cfg.n_ff % 4)
    return TALOS_OK;
  for (uint32_t l = 0; l < c->cfg.n_layer; ++l) {
    LayerW w;
    int rc = layer_weights(c, l, &w);
    if (rc) return rc;
  }
  const size_t lds = (size_t)PF_ATT_KT * (2 * c->hd + 20) * 4;
  *ok = lds <= c->max_lds;
  return TALOS_OK;
}

// The prefill attention runs on f16 matrix cores with split operands when
// head_dim is a multiple of 32 and its tiles fit the LDS.
bool pf_attn16_on(const talos_hip_ctx* c) {
  return c->pf_f16 && c->pf_attn16 && c->hd % 32 == 0 && pf_attn16_lds_bytes(c->hd) <= c->max_lds;
}

int pf_reserve(talos_hip_ctx* c, uint32_t T) {
  if (pf_attn16_on(c) && !c->pf_kh) {
    const uint32_t cap = (c->cfg.context_length + 63) / 64 * 64;
    const size_t bytes = (size_t)cap * c->kv_dim * 2;
    for (uint16_t** p : {&c->pf_kh, &c->pf_kl, &c->pf_vh, &c->pf_vl}) HIPCHK(c, hipMalloc(p, bytes));
    c->pf_kv_cap = cap;
  }
  if (c->pf_cap >= T) return TALOS_OK;
  (void)hipStreamSynchronize(c->stream);
  for (float** p : {&c->pf_x, &c->pf_xn, &c->pf_qr, &c->pf_q, &c->pf_att, &c->pf_kr, &c->pf_vr, &c->pf_g, &c->pf_u,
                    &c->pf_h}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  for (uint16_t** p : {&c->pf_xn16, &c->pf_att16, &c->pf_h16}) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
  }
  if (c->pf_tok) (void)hipFree(c->pf_tok);
  c->pf_tok = nullptr;
  c->pf_cap = 0;
  const size_t n = c->cfg.n_embd, kv = c->kv_dim, ff = c->cfg.n_ff;
  for (float** p : {&c->pf_x, &c->pf_xn, &c->pf_qr, &c->pf_q, &c->pf_att}) HIPCHK(c, hipMalloc(p, (size_t)T * n * 4));
  for (float** p : {&c->pf_kr, &c->pf_vr}) HIPCHK(c, hipMalloc(p, (size_t)T * kv * 4));
  for (float** p : {&c->pf_g, &c->pf_u, &c->pf_h}) HIPCHK(c, hipMalloc(p, (size_t)T * ff * 4));
  if (c->pf_f16) {
    for (uint16_t** p : {&c->pf_xn16, &c->pf_att16}) HIPCHK(c, hipMalloc(p, (size_t)T * n * 4));
    if (ff % 8 == 0) HIPCHK(c, hipMalloc(&c->pf_h16, (size_t)T * ff * 4));
  }
  HIPCHK(c, hipMalloc(&c->pf_tok, (size_t)T * 4));
  c->pf_cap = T;
  return TALOS_OK;
}

// The tiled copies the split-f16 GEMMs read (k_pf_tile): made for every
// Q4_0 / Q8_0 layer matrix with rows % 16 == 0 and cols % 64 == 0 at the
// first batched prefill, in one allocation -- one more device copy of those
// matrices, kept until a weight is uploaded (pf_tile_drop) or the context is
// destroyed.  When the pool does not fit the device the GEMMs read the
// matrices themselves.
static bool pf_tileable(const DevWeight* w) {
  return (w->type == TALOS_GGML_Q4_0 || w->type == TALOS_GGML_Q8_0) && w->rows % 16 == 0 && w->cols % 64 == 0;
}
int pf_tile_weights(talos_hip_ctx* c) {
  if (!c->pf_f16 || !c->pf_tiled || c->pf_tile_pool) return TALOS_OK;
  std::vector<DevWeight*> ms;
  size_t total = 0;
  for (uint32_t l = 0; l < c->cfg.n_layer; ++l) {
    LayerW w;
    int rc = layer_weights(c, l, &w);
    if (rc) return rc;
    for (const DevWeight* cw : {w.q, w.k, w.v, w.o, w.g, w.u, w.d}) {
      if (!pf_tileable(cw)) continue;
      ms.push_back(const_cast<DevWeight*>(cw));  // the weights live in c->weights, which is not const
      total += (pf_tile_bytes(cw->type, cw->rows, cw->cols) + 255) / 256 * 256;
    }
  }
  if (ms.empty()) return TALOS_OK;
  if (hipMalloc(&c->pf_tile_pool, total) != hipSuccess) {
    (void)hipGetLastError();
    c->pf_tile_pool = nullptr;
    return TALOS_OK;
  }
  uint8_t* p = static_cast<uint8_t*>(c->pf_tile_pool);
  for (DevWeight* m : ms) {
    m->tiled = p;
    const size_t qb = m->type == TALOS_GGML_Q8_0 ? 64 : 32, pieces = m->rows * (m->cols / 64);
    uint32_t* td = reinterpret_cast<uint32_t*>(p + pieces * qb);
    const dim3 grid((unsigned)((pieces + 255) / 256));
    if (m->type == TALOS_GGML_Q8_0)
      hipLaunchKernelGGL(k_pf_tile<TALOS_FMT_Q8_0>, grid, dim3(256), 0, c->stream, m->mat, p, td);
    else
      hipLaunchKernelGGL(k_pf_tile<TALOS_FMT_Q4_0>, grid, dim3(256), 0, c->stream, m->mat, p, td);
    HIPCHK(c, hipGetLastError());
    p += (pf_tile_bytes(m->type, m->rows, m->cols) + 255) / 256 * 256;
  }
  return TALOS_OK;
}
// Every tiled copy goes (an upload may change any matrix); the next batched
// prefill makes them again.
void pf_tile_drop(talos_hip_ctx* c) {
  if (!c->pf_tile_pool) return;
  (void)hipStreamSynchronize(c->stream);
  (void)hipFree(c->pf_tile_pool);
  c->pf_tile_pool = nullptr;
  for (auto& kv : c->weights) kv.second.tiled = nullptr;
}
void pf_seg_tiled(PfSeg& S, const DevWeight* w) {
  if (!w->tiled) {
    S.tq = nullptr;
    S.td = nullptr;
    return;
  }
  S.tq = static_cast<const uint8_t*>(w->tiled);
  S.td = reinterpret_cast<const uint32_t*>(S.tq + w->rows * (w->cols / 64) * (w->type == TALOS_GGML_Q8_0 ? 64 : 32));
}

// Y_i[T][ldy_i] (+)= X[T][K] W_i^T for matrices sharing X; consecutive ones
// of one format go out as one launch (up to three).
struct GemmOut {
  const DevWeight* w;
  float* y;
  uint32_t ldy;
};
struct GemmIn {
  const float* x;       // [T][K]
  const uint16_t* x16;  // x as the split-f16 GEMM's interleaved halves (or null: only the f32 GEMM)
};
void enq_gemm(talos_hip_ctx* c, std::initializer_list<GemmOut> outs, GemmIn X, uint32_t T, int acc) {
  const GemmOut* o = outs.begin();
  const size_t n = outs.size();
  for (size_t i = 0; i < n;) {
    PfGemm G{};
    G.X = X.x;
    G.X16 = X.x16;
    G.T = T;
    G.K = (uint32_t)o[i].w->cols;
    G.accumulate = acc;
    const uint32_t type = o[i].w->type;
    uint32_t tiles = 0;
    while (i < n && G.nseg < 3 && o[i].w->type == type) {
      PfSeg& S = G.S[G.nseg++];
      S.W = o[i].w->mat;
      pf_seg_tiled(S, o[i].w);
      S.Y = o[i].y;
      S.ldy = o[i].ldy;
      S.tiles = (uint32_t)((o[i].w->rows + PF_ROWS - 1) / PF_ROWS);
      tiles += S.tiles;
      ++i;
    }
    // token tiles on x: a row tile's token tiles go out together and land
    // on the XCDs round-robin by token tile, so each XCD's L2 serves a few
    // token tiles of X and a row tile's weights are fetched about once per
    // XCD (+0.6 % at a 16k prompt against row tiles on x)
    const dim3 grid((T + PF_TOK - 1) / PF_TOK, tiles);
    bool tiled = true;  // every segment has its tiled copy
    for (uint32_t s = 0; s < G.nseg; ++s) tiled = tiled && G.S[s].tq;
    switch (type) {
      case TALOS_GGML_Q4_0:
        if (G.X16 && tiled)
          hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q4_0, false, true>), grid, dim3(PF_NT), 0, c->stream, G);
        else if (G.X16)
          hipLaunchKernelGGL(k_pf_gemm16<TALOS_FMT_Q4_0>, grid, dim3(PF_NT), 0, c->stream, G);
        else
          hipLaunchKernelGGL(k_pf_gemm<TALOS_FMT_Q4_0>, grid, dim3(PF_NT), 0, c->stream, G);
        break;
      case TALOS_GGML_Q8_0:
        if (G.X16 && tiled)
          hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q8_0, false, true>), grid, dim3(PF_NT), 0, c->stream, G);
        else if (G.X16)
          hipLaunchKernelGGL(k_pf_gemm16<TALOS_FMT_Q8_0>, grid, dim3(PF_NT), 0, c->stream, G);
        else
          hipLaunchKernelGGL(k_pf_gemm<TALOS_FMT_Q8_0>, grid, dim3(PF_NT), 0, c->stream, G);
        break;
      case TALOS_GGML_Q6_K: hipLaunchKernelGGL(k_pf_gemm<TALOS_FMT_Q6_K>, grid, dim3(PF_NT), 0, c->stream, G); break;
      default: hipLaunchKernelGGL(k_pf_gemm<TALOS_FMT_F32>, grid, dim3(PF_NT), 0, c->stream, G); break;
    }
  }
}

// H = silu(X W_gate^T) * (X W_up^T) in one launch when both matrices are
// Q4_0 or both Q8_0 and X comes split: the split-f16 GEMM with the SwiGLU in
// its epilogue (k_pf_gemm16<FMT, true>).  Returns false when it does not apply.
bool enq_gateup_swiglu(talos_hip_ctx* c, const DevWeight* wg, const DevWeight* wu, GemmIn X, uint32_t T) {
  if (!X.x16 || !c->pf_h16 || wg->type != wu->type || wg->rows != wu->rows || wg->cols != wu->cols ||
      (wg->type != TALOS_GGML_Q4_0 && wg->type != TALOS_GGML_Q8_0))
    return false;
  PfGemm G{};
  G.X = X.x;
  G.X16 = X.x16;
  G.T = T;
  G.K = (uint32_t)wg->cols;
  G.nseg = 2;
  G.S[0].W = wg->mat;
  G.S[1].W = wu->mat;
  pf_seg_tiled(G.S[0], wg);
  pf_seg_tiled(G.S[1], wu);
  G.H = c->pf_h;
  G.H16 = c->pf_h16;
  G.ldh = (uint32_t)wg->rows;
  const dim3 grid((T + PF_TOK - 1) / PF_TOK, (uint32_t)((wg->rows + PF_ROWS / 2 - 1) / (PF_ROWS / 2)));
  const bool tiled = G.S[0].tq && G.S[1].tq;
  if (wg->type == TALOS_GGML_Q4_0) {
    if (tiled)
      hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q4_0, true, true>), grid, dim3(PF_NT), 0, c->stream, G);
    else
      hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q4_0, true>), grid, dim3(PF_NT), 0, c->stream, G);
  } else {
    if (tiled)
      hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q8_0, true, true>), grid, dim3(PF_NT), 0, c->stream, G);
    else
      hipLaunchKernelGGL((k_pf_gemm16<TALOS_FMT_Q8_0, true>), grid, dim3(PF_NT), 0, c->stream, G);
  }
  return true;
}

void enq_pf_attn(talos_hip_ctx* c, uint32_t l, uint32_t T, uint32_t p0) {
  PfAttn A{};
  A.Q = c->pf_q;
  A.kc = c->kc[l];
  A.vc = c->vc[l];
  A.out = c->pf_att;
  A.out16 = c->pf_att16;
  A.T = T;
  A.p0 = p0;
  A.n = c->cfg.n_embd;
  A.kv_dim = c->kv_dim;
  A.hd = c->hd;
  A.group = c->group;
  A.scale = 1.0f / sqrtf((float)c->hd);
  const bool wide = c->group > 4 || c->hd > 128;  // 8 waves, else 4
  const dim3 grid(c->cfg.n_head_kv, (T + PF_ATT_Q - 1) / PF_ATT_Q), block(wide ? 512 : 256);
  if (pf_attn16_on(c)) {
    // the layer's rows [0, p0 + T) split into the shadow (rows up to the
    // next multiple of 64 zero), then the attention over it
    PfKv16 P{};
    P.kc = c->kc[l];
    P.vc = c->vc[l];
    P.kh = c->pf_kh;
    P.kl = c->pf_kl;
    P.vh = c->pf_vh;
    P.vl = c->pf_vl;
    P.R = p0 + T;
    P.kv_dim = c->kv_dim;
    P.hd = c->hd;
    P.cap = c->pf_kv_cap;
    hipLaunchKernelGGL(k_pf_kv16, dim3((c->kv_dim + 63) / 64, (P.R + 63) / 64), dim3(256), 0, c->stream, P);
    PfAttn16 B{};
    B.Q = c->pf_q;
    B.kh = c->pf_kh;
    B.kl = c->pf_kl;
    B.vh = c->pf_vh;
    B.vl = c->pf_vl;
    B.out = c->pf_att;
    B.out16 = c->pf_att16;
    B.T = T;
    B.p0 = p0;
    B.n = c->cfg.n_embd;
    B.group = c->group;
    B.cap = c->pf_kv_cap;
    B.scale = A.scale;
    const size_t lds16 = pf_attn16_lds_bytes(c->hd);
    // 8 waves: groups of up to 4 q heads take two 16-query groups per block
    // (the K/V tile staged once for twice the matrix work), larger groups one
    const bool two = c->group <= 4;
    const uint32_t qb = PF_ATT_Q * (two ? 2 : 1);
    const dim3 grid16(c->cfg.n_head_kv, (T + qb - 1) / qb), block16(512);
    switch (c->hd / 32) {
#define PF_ATT16_CASE(N)                                                                                  \
  case N:                                                                                                 \
    if (two) hipLaunchKernelGGL((k_pf_attn16<32 * N, 512, 2>), grid16, block16, lds16, c->stream, B);    \
    else hipLaunchKernelGGL((k_pf_attn16<32 * N, 512, 1>), grid16, block16, lds16, c->stream, B);        \
    break;
      PF_ATT16_CASE(1) PF_ATT16_CASE(2) PF_ATT16_CASE(3) PF_ATT16_CASE(4) PF_ATT16_CASE(5) PF_ATT16_CASE(6)
      PF_ATT16_CASE(7) PF_ATT16_CASE(8)
#undef PF_ATT16_CASE
      default: break;
    }
    return;
  }
  const size_t lds = (size_t)PF_ATT_KT * (2 * c->hd + 20) * 4;
  switch (c->hd / 16) {
#define PF_ATT_CASE(N)                                                                       \
  case N:                                                                                    \
    if (wide) hipLaunchKernelGGL((k_pf_attn<16 * N, 512>), grid, block, lds, c->stream, A); \
    else hipLaunchKernelGGL((k_pf_attn<16 * N, 256>), grid, block, lds, c->stream, A);      \
    break;
    PF_ATT_CASE(1) PF_ATT_CASE(2) PF_ATT_CASE(3) PF_ATT_CASE(4) PF_ATT_CASE(5) PF_ATT_CASE(6) PF_ATT_CASE(7)
    PF_ATT_CASE(8) PF_ATT_CASE(9) PF_ATT_CASE(10) PF_ATT_CASE(11) PF_ATT_CASE(12) PF_ATT_CASE(13) PF_ATT_CASE(14)
    PF_ATT_CASE(15) PF_ATT_CASE(16)
#undef PF_ATT_CASE
    default: break;
  }
}

void set_pf_attn_lds(int bytes) {
#define PF_ATT_SET(N)                                        \
  set_max_lds((const void*)k_pf_attn<16 * N, 256>, bytes); \
  set_max_lds((const void*)k_pf_attn<16 * N, 512>, bytes);
#define PF_ATT16_SET(N)                                           \
  set_max_lds((const void*)k_pf_attn16<32 * N, 512, 2>, bytes); \
  set_max_lds((const void*)k_pf_attn16<32 * N, 512, 1>, bytes);
  PF_ATT16_SET(1) PF_ATT16_SET(2) PF_ATT16_SET(3) PF_ATT16_SET(4) PF_ATT16_SET(5) PF_ATT16_SET(6)
  PF_ATT16_SET(7) PF_ATT16_SET(8)
#undef PF_ATT16_SET
  PF_ATT_SET(1) PF_ATT_SET(2) PF_ATT_SET(3) PF_ATT_SET(4) PF_ATT_SET(5) PF_ATT_SET(6) PF_ATT_SET(7) PF_ATT_SET(8)
  PF_ATT_SET(9) PF_ATT_SET(10) PF_ATT_SET(11) PF_ATT_SET(12) PF_ATT_SET(13) PF_ATT_SET(14) PF_ATT_SET(15)
  PF_ATT_SET(16)
#undef PF_ATT_SET
}

// One chunk of T prompt tokens at positions p0 .. p0 + T - 1 through every
// layer; leaves the chunk's rows in pf_x.
int pf_chunk(talos_hip_ctx* c, const uint32_t* tokens, uint32_t T, uint32_t p0) {
  const auto& cf = c->cfg;
  const uint32_t n = cf.n_embd, kv = c->kv_dim, ff = cf.n_ff;
  int rc;
  const DevWeight* emb;
  if ((rc = need_matrix(c, "token_embd.weight", cf.vocab_size, n, &emb))) return rc;
  for (uint32_t i = 0; i < T; ++i) c->h_tokens[i] = (int32_t)tokens[i];
  HIPCHK(c, hipMemcpyAsync(c->pf_tok, c->h_tokens, (size_t)T * 4, hipMemcpyHostToDevice, c->stream));
  hipLaunchKernelGGL(k_pf_embed, dim3(T), dim3(256), 0, c->stream, emb->mat, c->pf_tok, n, c->pf_x);
  for (uint32_t l = 0; l < cf.n_layer; ++l) {
    LayerW w;
    if ((rc = layer_weights(c, l, &w))) return rc;
    const GemmIn xn{c->pf_xn, c->pf_xn16};
    hipLaunchKernelGGL(k_pf_rmsnorm, dim3(T), dim3(256), 0, c->stream, c->pf_x, w.an, cf.rms_eps, n, c->pf_xn,
                       c->pf_xn16);
    enq_gemm(c, {{w.q, c->pf_qr, n}, {w.k, c->pf_kr, kv}, {w.v, c->pf_vr, kv}}, xn, T, 0);
    hipLaunchKernelGGL(k_pf_rope_kv, dim3((std::max(n, kv) / 4 + 255) / 256, T), dim3(256), 0, c->stream, c->pf_qr,
                       c->pf_kr, c->pf_vr, c->pf_q, c->kc[l], c->vc[l], c->rope, p0, n, cf.n_head, c->hd, kv);
    enq_pf_attn(c, l, T, p0);
    enq_gemm(c, {{w.o, c->pf_x, n}}, {c->pf_att, c->pf_att16}, T, 1);
    hipLaunchKernelGGL(k_pf_rmsnorm, dim3(T), dim3(256), 0, c->stream, c->pf_x, w.fn, cf.rms_eps, n, c->pf_xn,
                       c->pf_xn16);
    if (!enq_gateup_swiglu(c, w.g, w.u, xn, T)) {
      enq_gemm(c, {{w.g, c->pf_g, ff}, {w.u, c->pf_u, ff}}, xn, T, 0);
      const size_t cnt = (size_t)T * ff;
      hipLaunchKernelGGL(k_pf_swiglu, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, c->stream, c->pf_g,
                         c->pf_u, c->pf_h, c->pf_h16, cnt);
    }
    enq_gemm(c, {{w.d, c->pf_x, n}}, {c->pf_h, c->pf_h16}, T, 1);
  }
  HIPCHK(c, hipGetLastError());
  return TALOS_OK;
}

int check_ctx(talos_hip_ctx* c) {
  if (!c) return TALOS_ERR_ARG;
  c->err.clear();
  return TALOS_OK;
}

int set_device(talos_hip_ctx* c) {
  HIPCHK(c, hipSetDevice(c->cfg.device));
  return TALOS_OK;
}

}  // namespace

extern "C" {

int talos_hip_create(const talos_hip_cfg* cfg, talos_hip_ctx** out) {
  g_create_error.clear();
  if (!cfg || !out) return fail(nullptr, TALOS_ERR_ARG, "null cfg or out");
  *out = nullptr;
  const talos_hip_cfg& f = *cfg;
  if (!f.n_layer || !f.n_head || !f.n_head_kv || !f.n_embd || !f.n_ff || !f.vocab_size || !f.context_length)
    return fail(nullptr, TALOS_ERR_ARG, "config has a zero dimension");
  if (f.n_head % f.n_head_kv != 0)
    return fail(nullptr, TALOS_ERR_ARG, "head_count %u must be a positive multiple of head_count_kv %u", f.n_head,
                f.n_head_kv);
  // head_dim = n_embd / n_head, rounded down (src/model/config.rs); any
  // value of at least 1 is served (the generic-shape kernels take odd ones)
  const uint32_t hd = f.n_embd / f.n_head;
  if (hd == 0) return fail(nullptr, TALOS_ERR_ARG, "n_embd %u < n_head %u leaves no head dimension", f.n_embd, f.n_head);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0)
    return fail(nullptr, TALOS_ERR_HIP, "no HIP device available");
  if (f.device < 0 || f.device >= ndev) return fail(nullptr, TALOS_ERR_ARG, "device %d out of range", f.device);

  auto c = std::make_unique<talos_hip_ctx>();
  c->cfg = f;
  const char* env = getenv("TALOS_HIP_GRAPHS");
  c->use_graphs = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_MEGA");
  c->allow_mega = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_PREFETCH");
  c->mega_prefetch = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_BAR1");
  c->one_hop = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_COOP");
  c->mega_coop = env && env[0] == '1';
  env = getenv("TALOS_HIP_MFMA");
  c->allow_mfma = env && env[0] == '1';
  env = getenv("TALOS_HIP_DOT4");
  c->allow_dot4 = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_ATTN_WAIT");
  c->allow_attn_wait = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_DSPLIT");
  c->allow_dsplit = env && (env[0] == '0' || env[0] == '1') ? env[0] - '0' : 2;
  env = getenv("TALOS_HIP_BATCH");
  c->allow_batch = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_PF16");
  c->pf_f16 = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_PFA16");
  c->pf_attn16 = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_PF_TILED");
  c->pf_tiled = !(env && env[0] == '0');
  env = getenv("TALOS_HIP_ATTN_DIRECT");
  if (env) c->attn_direct = std::max(0, atoi(env));
  c->hd = hd;
  c->kv_dim = f.n_head_kv * hd;
  c->group = f.n_head / f.n_head_kv;
  // Slices of TALOS_ATTN_CHUNK positions, at most 512 per KV head; the
  // kernel uses ceil(seq / chunk) of them for the live sequence.  Past
  // 512 * chunk positions the slices grow to ceil(ctx / 512).
  uint32_t ns = (f.context_length + TALOS_ATTN_CHUNK - 1) / TALOS_ATTN_CHUNK;
  c->nsplit = ns < 1 ? 1 : (ns > 512 ? 512 : ns);
  // Longest live slice: up to TALOS_ATTN_CHUNK positions while the slice
  // count follows the sequence, ceil(ctx / nsplit) once it is capped (a
  // context that is not a multiple of the chunk still has chunk-long slices).
  c->max_chunk = std::max<uint32_t>(TALOS_ATTN_CHUNK, (f.context_length + c->nsplit - 1) / c->nsplit);
  hipError_t e = hipSetDevice(f.device);
  if (e != hipSuccess) return fail(nullptr, TALOS_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, f.device)) != hipSuccess)
    return fail(nullptr, TALOS_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  c->max_lds = prop.sharedMemPerBlock;
  const size_t need_lds = stage_lds_bytes((int)std::max(f.n_embd, f.n_ff), 3);
  if (need_lds > c->max_lds)
    return fail(nullptr, TALOS_ERR_ARG, "n_ff %u needs %zu B of LDS, device has %zu", f.n_ff, need_lds, c->max_lds);
  set_lds_attr_fmt<TALOS_FMT_F32>((int)c->max_lds);
  set_lds_attr_fmt<TALOS_FMT_Q4_0>((int)c->max_lds);
  set_lds_attr_fmt<TALOS_FMT_Q8_0>((int)c->max_lds);
  set_lds_attr_fmt<TALOS_FMT_Q6_K>((int)c->max_lds);
  set_pf_attn_lds((int)c->max_lds);
  for (const void* k : {(const void*)k_attn_scores, (const void*)k_attn<2>, (const void*)k_attn<3>, (const void*)k_attn<4>,
                        (const void*)k_attn<5>, (const void*)k_attn<6>, (const void*)k_attn<7>, (const void*)k_attn<8>})
    set_max_lds(k, (int)c->max_lds);
  if ((size_t)hd * 4 > c->max_lds)
    return fail(nullptr, TALOS_ERR_ARG, "head_dim %u needs %zu B of LDS, device has %zu", hd, (size_t)hd * 4,
                c->max_lds);
  if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess)
    return fail(nullptr, TALOS_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  // this GPU's address of the allocation-free sampler's scratch (the
  // device is current here)
  if ((e = scratch_setup(f.device)) != hipSuccess) {
    talos_hip_destroy(c.release());
    return fail(nullptr, TALOS_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  }


  // RoPE table, same expression as src/math/ops.rs:48-61 evaluated in f32
  // with the C library's powf/sinf/cosf.
  const uint32_t half = hd / 2;
  std::vector<float> rope((size_t)f.context_length * half * 2);
  for (uint32_t p = 0; p < f.context_length; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      const float expo = (-2.0f * (float)i) / (float)hd;
      const float theta = (float)p * powf(f.rope_freq_base, expo);
      rope[((size_t)p * half + i) * 2 + 0] = cosf(theta);
      rope[((size_t)p * half + i) * 2 + 1] = sinf(theta);
    }
  if ((e = hipMalloc(&c->rope, rope.size() * 4)) != hipSuccess ||
      (e = hipMemcpy(c->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
    talos_hip_destroy(c.release());
    return fail(nullptr, TALOS_ERR_HIP, "rope table: %s", hipGetErrorString(e));
  }
  *out = c.release();
  return TALOS_OK;
}

void talos_hip_destroy(talos_hip_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->cfg.device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  destroy_graphs(c);
  for (auto& kv : c->weights) (void)hipFree(kv.second.mem);
  if (c->pf_tile_pool) (void)hipFree(c->pf_tile_pool);
  for (float* p : c->kc) (void)hipFree(p);
  for (float* p : c->vc) (void)hipFree(p);
  void* dev[] = {c->io, c->q, c->atty, c->h, c->logits, c->hidden, c->part, c->count, c->tokens, c->rope,
                 c->samp_ka, c->samp_kb, c->samp_pb, c->samp_out, c->samp_u, c->nll, c->pf_x, c->pf_xn,
                 c->pf_qr, c->pf_q, c->pf_att, c->pf_kr, c->pf_vr, c->pf_g, c->pf_u, c->pf_h, c->pf_tok,
                 c->pf_kh, c->pf_kl, c->pf_vh, c->pf_vl, c->pf_xn16, c->pf_att16, c->pf_h16,
                 c->mv_x, c->mv_out, c->d_layers, c->d_sync, c->mact, c->mpart, c->qraw, c->kraw,
                 c->vraw, c->graw, c->uraw, c->scores};
  for (void* p : dev)
    if (p) (void)hipFree(p);
  if (c->h_io) (void)hipHostFree(c->h_io);
  if (c->h_out) (void)hipHostFree(c->h_out);
  if (c->h_tokens) (void)hipHostFree(c->h_tokens);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* talos_hip_last_error(const talos_hip_ctx* c) { return c ? c->err.c_str() : g_create_error.c_str(); }

int talos_hip_upload_weight(talos_hip_ctx* c, const char* name, const void* bytes, size_t len, uint32_t type,
                            size_t rows, size_t cols) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!name || !bytes) return fail(c, TALOS_ERR_ARG, "null name or bytes");
  if (!type_ok(type)) return fail(c, TALOS_ERR_DTYPE, "tensor \"%s\" has unsupported ggml type %u", name, type);
  if (!rows || !cols) return fail(c, TALOS_ERR_SHAPE, "tensor \"%s\" has an empty shape", name);
  const size_t be = block_elems(type);
  if (cols % be) return fail(c, TALOS_ERR_SHAPE, "tensor \"%s\": cols %zu not a multiple of block %zu", name, cols, be);
  const size_t want = rows * (cols / be) * block_bytes(type);
  if (len != want)
    return fail(c, TALOS_ERR_SHAPE, "tensor \"%s\": %zu bytes, [%zu, %zu] of type %u needs %zu", name, len, rows, cols,
                type, want);
  auto it = c->weights.find(name);
  if (it != c->weights.end() && it->second.len == len) return TALOS_OK;  // resident (metal/mod.rs:64-68)
  if ((rc = set_device(c))) return rc;
  Packed P;
  repack(static_cast<const uint8_t*>(bytes), type, rows, cols, P);
  DevWeight w;
  w.type = type;
  w.rows = rows;
  w.cols = cols;
  w.len = len;
  HIPCHK(c, hipMalloc(&w.mem, P.img.size()));
  hipError_t e = hipMemcpy(w.mem, P.img.data(), P.img.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(w.mem);
    return fail(c, TALOS_ERR_HIP, "upload of \"%s\": %s", name, hipGetErrorString(e));
  }
  uint8_t* base = static_cast<uint8_t*>(w.mem);
  w.mat.q = base + P.q_off;
  w.mat.d = type == TALOS_GGML_F32 ? nullptr : reinterpret_cast<const uint16_t*>(base + P.d_off);
  w.mat.sc = type == TALOS_GGML_Q6_K ? reinterpret_cast<const uint32_t*>(base + P.sc_off) : nullptr;
  w.mat.rows = (uint32_t)rows;
  w.mat.cols = (uint32_t)cols;
  w.mat.fmt = type;
  w.mat.nchunk = P.nchunk;
  w.f32 = type == TALOS_GGML_F32 ? reinterpret_cast<const float*>(base) : nullptr;
  if (it != c->weights.end()) {
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(it->second.mem);
    it->second = w;
  } else {
    c->weights.emplace(name, w);
  }
  destroy_graphs(c);  // graphs captured the old pointers
  pf_tile_drop(c);
  c->mega_ready = false;
  return TALOS_OK;
}

static int forward_host(talos_hip_ctx* c, const float* x_embed, uint32_t pos, float* out, GraphKind kind) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!x_embed || !out) return fail(c, TALOS_ERR_ARG, "null x_embed or output");
  if (pos >= c->cfg.context_length)
    return fail(c, TALOS_ERR_POS, "pos %u >= context_length %u", pos, c->cfg.context_length);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, kind, &g))) return rc;
  const uint32_t n = c->cfg.n_embd;
  memset(c->h_io, 0, 64);
  c->h_io[ST_POS] = (int32_t)pos;
  memcpy(c->h_io + 16, x_embed, (size_t)n * 4);
  HIPCHK(c, hipMemcpyAsync(c->io, c->h_io, 64 + (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
  if ((rc = run_step(c, kind, g))) return rc;
  const size_t out_n = kind == G_HIDDEN ? n : c->cfg.vocab_size;
  HIPCHK(c, hipMemcpyAsync(c->h_out, kind == G_HIDDEN ? c->hidden : c->logits, out_n * 4, hipMemcpyDeviceToHost,
                           c->stream));
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if ((rc = check_device_err(c))) return rc;
  memcpy(out, c->h_out, out_n * 4);
  return TALOS_OK;
}

int talos_hip_forward(talos_hip_ctx* c, const float* x_embed, uint32_t pos, float* logits) {
  return forward_host(c, x_embed, pos, logits, G_LOGITS);
}

int talos_hip_forward_hidden(talos_hip_ctx* c, const float* x_embed, uint32_t pos, float* hidden) {
  return forward_host(c, x_embed, pos, hidden, G_HIDDEN);
}

namespace {
int set_state(talos_hip_ctx* c, uint32_t token, uint32_t pos) {
  memset(c->h_io, 0, 64);
  c->h_io[ST_POS] = (int32_t)pos;
  c->h_io[ST_TOKEN] = (int32_t)token;
  c->h_io[ST_STEP] = 0;
  HIPCHK(c, hipMemcpyAsync(c->io, c->h_io, 64, hipMemcpyHostToDevice, c->stream));
  return TALOS_OK;
}
}  // namespace

int talos_hip_forward_token(talos_hip_ctx* c, uint32_t token, uint32_t pos, float* logits, uint32_t* argmax) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (pos >= c->cfg.context_length)
    return fail(c, TALOS_ERR_POS, "pos %u >= context_length %u", pos, c->cfg.context_length);
  if (token >= c->cfg.vocab_size)
    return fail(c, TALOS_ERR_TOKEN, "token %u >= vocab_size %u", token, c->cfg.vocab_size);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_TOKEN, &g))) return rc;
  if ((rc = set_state(c, token, pos))) return rc;
  if ((rc = run_step(c, G_TOKEN, g))) return rc;
  if (logits)
    HIPCHK(c, hipMemcpyAsync(c->h_out, c->logits, (size_t)c->cfg.vocab_size * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if ((rc = check_device_err(c))) return rc;
  if (logits) memcpy(logits, c->h_out, (size_t)c->cfg.vocab_size * 4);
  if (argmax) *argmax = (uint32_t)c->h_io[ST_ARGMAX];
  return TALOS_OK;
}

int talos_hip_decode_greedy(talos_hip_ctx* c, uint32_t token, uint32_t pos, uint32_t n_steps, uint32_t* tokens_out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!tokens_out && n_steps) return fail(c, TALOS_ERR_ARG, "null tokens_out");
  if ((uint64_t)pos + n_steps > c->cfg.context_length)
    return fail(c, TALOS_ERR_POS, "pos %u + %u steps exceeds context_length %u", pos, n_steps, c->cfg.context_length);
  if (token >= c->cfg.vocab_size)
    return fail(c, TALOS_ERR_TOKEN, "token %u >= vocab_size %u", token, c->cfg.vocab_size);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_GREEDY, &g))) return rc;
  if ((rc = set_state(c, token, pos))) return rc;
  for (uint32_t s = 0; s < n_steps; ++s)
    if ((rc = run_step(c, G_GREEDY, g))) return rc;
  if (n_steps)
    HIPCHK(c, hipMemcpyAsync(c->h_tokens, c->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if ((rc = check_device_err(c))) return rc;
  for (uint32_t s = 0; s < n_steps; ++s) tokens_out[s] = (uint32_t)c->h_tokens[s];
  return TALOS_OK;
}

int talos_hip_prefill(talos_hip_ctx* c, const uint32_t* tokens, uint32_t n, uint32_t pos, float* logits,
                      uint32_t* argmax) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (n == 0) return TALOS_OK;
  if (!tokens) return fail(c, TALOS_ERR_ARG, "null tokens");
  if ((uint64_t)pos + n > c->cfg.context_length)
    return fail(c, TALOS_ERR_POS, "pos %u + %u tokens exceeds context_length %u", pos, n, c->cfg.context_length);
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] >= c->cfg.vocab_size)
      return fail(c, TALOS_ERR_TOKEN, "tokens[%u] = %u >= vocab_size %u", i, tokens[i], c->cfg.vocab_size);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_FEED, &g))) return rc;
  bool batched = false;
  if ((rc = pf_supported(c, &batched))) return rc;
  if (batched) {
    // chunks of up to PF_CHUNK tokens through every layer at once; the last
    // token's row then takes the final norm, the output projection and the
    // argmax as a decode step's head does
    if ((rc = pf_reserve(c, std::min(n, (uint32_t)PF_CHUNK)))) return rc;
    if ((rc = pf_tile_weights(c))) return rc;
    uint32_t last = 0;
    for (uint32_t c0 = 0; c0 < n; c0 += PF_CHUNK) {
      const uint32_t T = std::min((uint32_t)PF_CHUNK, n - c0);
      if ((rc = pf_chunk(c, tokens + c0, T, pos + c0))) return rc;
      last = T - 1;
      if (c0 + T < n) HIPCHK(c, hipStreamSynchronize(c->stream));  // h_tokens is reused
    }
    const auto& cf = c->cfg;
    HIPCHK(c, hipMemcpyAsync(c->x, c->pf_x + (size_t)last * cf.n_embd, (size_t)cf.n_embd * 4,
                             hipMemcpyDeviceToDevice, c->stream));
    const DevWeight* wout;
    const float* onorm;
    if ((rc = need_norm(c, "output_norm.weight", cf.n_embd, &onorm)) ||
        (rc = need_matrix(c, "output.weight", cf.vocab_size, cf.n_embd, &wout)))
      return rc;
    memset(c->h_io, 0, 64);
    c->h_io[ST_POS] = (int32_t)(pos + n - 1);
    c->h_io[ST_TOKEN] = (int32_t)tokens[n - 1];
    HIPCHK(c, hipMemcpyAsync(c->io, c->h_io, 64, hipMemcpyHostToDevice, c->stream));
    enq_output(c, wout, onorm);
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, c->stream, c->logits, cf.vocab_size, c->io, c->tokens, 0);
    HIPCHK(c, hipGetLastError());
    if (logits)
      HIPCHK(c, hipMemcpyAsync(c->h_out, c->logits, (size_t)cf.vocab_size * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (logits) memcpy(logits, c->h_out, (size_t)cf.vocab_size * 4);
    if (argmax) *argmax = (uint32_t)c->h_io[ST_ARGMAX];
    return TALOS_OK;
  }
  for (uint32_t i = 0; i < n; ++i) c->h_tokens[i] = (int32_t)tokens[i];
  HIPCHK(c, hipMemcpyAsync(c->tokens, c->h_tokens, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
  memset(c->h_io, 0, 64);
  c->h_io[ST_POS] = (int32_t)pos;
  c->h_io[ST_TOKEN] = (int32_t)tokens[0];
  c->h_io[ST_NFEED] = (int32_t)n;
  HIPCHK(c, hipMemcpyAsync(c->io, c->h_io, 64, hipMemcpyHostToDevice, c->stream));
  for (uint32_t i = 0; i < n; ++i)
    if ((rc = run_step(c, G_FEED, g))) return rc;
  if (logits)
    HIPCHK(c, hipMemcpyAsync(c->h_out, c->logits, (size_t)c->cfg.vocab_size * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if ((rc = check_device_err(c))) return rc;
  if (logits) memcpy(logits, c->h_out, (size_t)c->cfg.vocab_size * 4);
  if (argmax) *argmax = (uint32_t)c->h_io[ST_ARGMAX];
  return TALOS_OK;
}

int talos_hip_kv_reset(talos_hip_ctx* c) { return check_ctx(c); }

int talos_hip_sample(talos_hip_ctx* c, float temperature, uint32_t top_k, float top_p, float u, uint32_t* token) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!token) return fail(c, TALOS_ERR_ARG, "null token");
  if ((rc = samp_check(c, temperature, top_p, u))) return rc;
  if ((rc = set_device(c))) return rc;
  if ((rc = alloc_acts(c))) return rc;
  const uint32_t n = c->cfg.vocab_size;
  if ((rc = samp_reserve(c, n))) return rc;
  enq_sample(c, c->logits, n, temperature, top_k, top_p, u, nullptr, c->samp_ka, c->samp_kb, c->samp_pb, c->samp_out,
             nullptr, nullptr);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->samp_out, 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  *token = (uint32_t)c->h_io[0];
  return TALOS_OK;
}

int talos_hip_sample_dev(talos_hip_ctx* c, const float* d_logits, uint32_t n, float temperature, uint32_t top_k,
                         float top_p, float u, uint32_t* d_token) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!d_logits || !d_token || n == 0) return fail(c, TALOS_ERR_ARG, "null logits or token, or n == 0");
  if ((rc = samp_check(c, temperature, top_p, u))) return rc;
  if ((rc = set_device(c))) return rc;
  if ((rc = samp_reserve(c, n))) return rc;
  enq_sample(c, d_logits, n, temperature, top_k, top_p, u, nullptr, c->samp_ka, c->samp_kb, c->samp_pb, d_token,
             nullptr, nullptr);
  HIPCHK(c, hipGetLastError());
  return TALOS_OK;
}

int talos_hip_sample_noalloc(talos_hip_ctx* c, const float* d_logits, uint32_t n, float temperature, uint32_t top_k,
                             float top_p, float u, uint32_t* d_token) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!d_logits || !d_token || n == 0) return fail(c, TALOS_ERR_ARG, "null logits or token, or n == 0");
  if (n > TALOS_SAMPLE_NOALLOC_MAX)
    return fail(c, TALOS_ERR_SHAPE, "n %u exceeds the allocation-free sampler's maximum %u", n,
                TALOS_SAMPLE_NOALLOC_MAX);
  if ((rc = samp_check(c, temperature, top_p, u))) return rc;
  if ((rc = set_device(c))) return rc;
  uint8_t* sp = scratch_ptr(c->cfg.device);
  if (!sp) return fail(c, TALOS_ERR_HIP, "sampling scratch of device %d not set up", c->cfg.device);
  uint64_t* ka = reinterpret_cast<uint64_t*>(sp);
  uint64_t* kb = reinterpret_cast<uint64_t*>(sp + (size_t)TALOS_SAMPLE_NOALLOC_MAX * 8);
  float* pb = reinterpret_cast<float*>(sp + (size_t)TALOS_SAMPLE_NOALLOC_MAX * 16);
  enq_sample(c, d_logits, n, temperature, top_k, top_p, u, nullptr, ka, kb, pb, d_token, nullptr, nullptr);
  HIPCHK(c, hipGetLastError());
  return TALOS_OK;
}

int talos_hip_decode_sample(talos_hip_ctx* c, uint32_t token, uint32_t pos, uint32_t n_steps, float temperature,
                            uint32_t top_k, float top_p, const float* u, uint32_t* tokens_out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (n_steps && (!tokens_out || !u)) return fail(c, TALOS_ERR_ARG, "null u or tokens_out");
  if ((uint64_t)pos + n_steps > c->cfg.context_length)
    return fail(c, TALOS_ERR_POS, "pos %u + %u steps exceeds context_length %u", pos, n_steps, c->cfg.context_length);
  if (token >= c->cfg.vocab_size)
    return fail(c, TALOS_ERR_TOKEN, "token %u >= vocab_size %u", token, c->cfg.vocab_size);
  for (uint32_t s = 0; s < n_steps; ++s)
    if ((rc = samp_check(c, temperature, top_p, u[s]))) return rc;
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_TOKEN, &g))) return rc;
  const uint32_t n = c->cfg.vocab_size;
  if ((rc = samp_reserve(c, n))) return rc;
  if (c->samp_u_cap < n_steps) {
    if (c->samp_u) (void)hipFree(c->samp_u);
    c->samp_u = nullptr;
    c->samp_u_cap = 0;
    HIPCHK(c, hipMalloc(&c->samp_u, (size_t)std::max(n_steps, 1u) * 4));
    c->samp_u_cap = std::max(n_steps, 1u);
  }
  if (n_steps) HIPCHK(c, hipMemcpyAsync(c->samp_u, u, (size_t)n_steps * 4, hipMemcpyHostToDevice, c->stream));
  if ((rc = set_state(c, token, pos))) return rc;
  // each step: the forward (its argmax is not used), then the draw, which
  // sets the next token and advances the position on the device
  for (uint32_t s = 0; s < n_steps; ++s) {
    if ((rc = run_step(c, G_TOKEN, g))) return rc;
    enq_sample(c, c->logits, n, temperature, top_k, top_p, 0.f, c->samp_u, c->samp_ka, c->samp_kb, c->samp_pb,
               nullptr, c->io, c->tokens);
  }
  HIPCHK(c, hipGetLastError());
  if (n_steps)
    HIPCHK(c, hipMemcpyAsync(c->h_tokens, c->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->io, 64, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if ((rc = check_device_err(c))) return rc;
  for (uint32_t s = 0; s < n_steps; ++s) tokens_out[s] = (uint32_t)c->h_tokens[s];
  return TALOS_OK;
}

int talos_hip_perplexity(talos_hip_ctx* c, const uint32_t* tokens, uint32_t n, float* ppl, float* nll_out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!tokens || !ppl) return fail(c, TALOS_ERR_ARG, "null tokens or ppl");
  if (n < 2) return fail(c, TALOS_ERR_ARG, "perplexity needs at least 2 tokens, got %u", n);
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] >= c->cfg.vocab_size)
      return fail(c, TALOS_ERR_TOKEN, "tokens[%u] = %u >= vocab_size %u", i, tokens[i], c->cfg.vocab_size);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_FEED, &g))) return rc;
  const uint32_t ctx = c->cfg.context_length;
  // scored positions: every chunk of ctx tokens with at least two scores
  // its len - 1 next tokens (src/eval.rs:35-52)
  uint32_t scored = 0;
  for (uint32_t c0 = 0; c0 < n; c0 += ctx) {
    const uint32_t len = std::min(ctx, n - c0);
    if (len < 2) break;
    scored += len - 1;
  }
  if (c->nll_cap < scored) {
    if (c->nll) (void)hipFree(c->nll);
    c->nll = nullptr;
    c->nll_cap = 0;
    HIPCHK(c, hipMalloc(&c->nll, (size_t)scored * 4));
    c->nll_cap = scored;
  }
  uint32_t k = 0;
  for (uint32_t c0 = 0; c0 < n; c0 += ctx) {
    const uint32_t len = std::min(ctx, n - c0);
    if (len < 2) break;
    // a fresh cache per chunk (positions restart at 0; rows are
    // position-indexed, so nothing needs clearing); the feed advances the
    // position and takes each next input from the device copy
    for (uint32_t i = 0; i < len; ++i) c->h_tokens[i] = (int32_t)tokens[c0 + i];
    HIPCHK(c, hipMemcpyAsync(c->tokens, c->h_tokens, (size_t)len * 4, hipMemcpyHostToDevice, c->stream));
    memset(c->h_io, 0, 64);
    c->h_io[ST_TOKEN] = (int32_t)tokens[c0];
    c->h_io[ST_NFEED] = (int32_t)len;
    HIPCHK(c, hipMemcpyAsync(c->io, c->h_io, 64, hipMemcpyHostToDevice, c->stream));
    for (uint32_t i = 0; i + 1 < len; ++i) {
      if ((rc = run_step(c, G_FEED, g))) return rc;
      hipLaunchKernelGGL(k_nll, dim3(1), dim3(256), 0, c->stream, c->logits, c->cfg.vocab_size, tokens[c0 + i + 1],
                         c->nll + k++);
    }
    // the host token buffer is reused by the next chunk
    HIPCHK(c, hipStreamSynchronize(c->stream));
  }
  HIPCHK(c, hipGetLastError());
  std::vector<float> h(scored);
  HIPCHK(c, hipMemcpy(h.data(), c->nll, (size_t)scored * 4, hipMemcpyDeviceToHost));
  HIPCHK(c, hipMemcpy(c->h_io, c->io, 64, hipMemcpyDeviceToHost));
  if ((rc = check_device_err(c))) return rc;
  double sum = 0.0;
  for (uint32_t i = 0; i < scored; ++i) sum += (double)h[i];
  *ppl = (float)std::exp(sum / (double)scored);
  if (nll_out) memcpy(nll_out, h.data(), (size_t)scored * 4);
  return TALOS_OK;
}

int talos_hip_kv_read(talos_hip_ctx* c, uint32_t n_pos, float* k_out, float* v_out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!k_out || !v_out) return fail(c, TALOS_ERR_ARG, "null output");
  if (n_pos > c->cfg.context_length) return fail(c, TALOS_ERR_POS, "n_pos %u > context_length", n_pos);
  if ((rc = set_device(c))) return rc;
  if ((rc = alloc_acts(c))) return rc;
  const size_t row = (size_t)n_pos * c->kv_dim;
  for (uint32_t l = 0; l < c->cfg.n_layer; ++l) {
    HIPCHK(c, hipMemcpyAsync(k_out + l * row, c->kc[l], row * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(v_out + l * row, c->vc[l], row * 4, hipMemcpyDeviceToHost, c->stream));
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return TALOS_OK;
}

int talos_hip_kv_write(talos_hip_ctx* c, uint32_t n_pos, const float* k, const float* v) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!k || !v) return fail(c, TALOS_ERR_ARG, "null input");
  if (n_pos > c->cfg.context_length) return fail(c, TALOS_ERR_POS, "n_pos %u > context_length", n_pos);
  if ((rc = set_device(c))) return rc;
  if ((rc = alloc_acts(c))) return rc;
  const size_t row = (size_t)n_pos * c->kv_dim;
  for (uint32_t l = 0; l < c->cfg.n_layer; ++l) {
    HIPCHK(c, hipMemcpyAsync(c->kc[l], k + l * row, row * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->vc[l], v + l * row, row * 4, hipMemcpyHostToDevice, c->stream));
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return TALOS_OK;
}

static int enqueue_matvec(talos_hip_ctx* c, const DevWeight* w, const float* d_x, float* d_out) {
  RowParams R{};
  R.m = w->mat;
  R.x = d_x;
  R.n = (uint32_t)w->cols;
  R.out = d_out;
  R.accumulate = 0;
  R.units = (uint32_t)((w->rows + mv_rows(w->mat.fmt) - 1) / mv_rows(w->mat.fmt));
  R.need = layout_need(w->mat.fmt);
  const size_t lds = stage_lds_bytes((int)w->cols, R.need);
  if (lds > c->max_lds) return fail(c, TALOS_ERR_SHAPE, "cols %zu needs %zu B of LDS", w->cols, lds);
  uint32_t blocks;
  if (w->mat.fmt == TALOS_FMT_F32) {
    // two rows per wave: twice the waves of mv_rows(F32) = 4, more bytes in
    // flight per CU (a standalone F32 matvec of 4096 x 4096 streams at ~0.68
    // of peak this way, ~0.56 with four rows)
    R.units = (uint32_t)((w->rows + 1) / 2);
    plan(R.units, R.upw, blocks);
    const int u = mv_u(w->mat.nchunk);
    if (u >= 4) hipLaunchKernelGGL((k_rows<TALOS_FMT_F32, 2, 4>), dim3(blocks), dim3(256), lds, c->stream, R);
    else if (u == 2) hipLaunchKernelGGL((k_rows<TALOS_FMT_F32, 2, 2>), dim3(blocks), dim3(256), lds, c->stream, R);
    else hipLaunchKernelGGL((k_rows<TALOS_FMT_F32, 2, 1>), dim3(blocks), dim3(256), lds, c->stream, R);
    HIPCHK(c, hipGetLastError());
    return TALOS_OK;
  }
  if (const int nr = iq_rounds(c, w->mat.fmt, w->cols)) {
    plan(R.units, R.upw, blocks);
    TALOS_MV_LAUNCH_IQ(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), nr, dim3(blocks), dim3(256),
                       rows_iq_lds_bytes(w->cols), c->stream, R);
    HIPCHK(c, hipGetLastError());
    return TALOS_OK;
  }
  plan(R.units, R.upw, blocks);
  TALOS_MV_LAUNCH(k_rows, w->mat.fmt, mv_u(w->mat.nchunk), dim3(blocks), dim3(256), lds, c->stream, R);
  HIPCHK(c, hipGetLastError());
  return TALOS_OK;
}

int talos_hip_matvec(talos_hip_ctx* c, const char* name, const void* bytes, size_t len, uint32_t type, size_t rows,
                     size_t cols, const float* x, float* out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!x || !out) return fail(c, TALOS_ERR_ARG, "null x or out");
  if ((rc = talos_hip_upload_weight(c, name, bytes, len, type, rows, cols))) return rc;
  const DevWeight* w = find_w(c, name);
  if (w->rows != rows || w->cols != cols)
    return fail(c, TALOS_ERR_SHAPE, "resident \"%s\" is [%zu, %zu], call asks [%zu, %zu]", name, w->rows, w->cols,
                rows, cols);
  if (c->mv_x_cap < cols) {
    if (c->mv_x) (void)hipFree(c->mv_x);
    c->mv_x = nullptr;
    HIPCHK(c, hipMalloc(&c->mv_x, cols * 4));
    c->mv_x_cap = cols;
  }
  if (c->mv_out_cap < rows) {
    if (c->mv_out) (void)hipFree(c->mv_out);
    c->mv_out = nullptr;
    HIPCHK(c, hipMalloc(&c->mv_out, rows * 4));
    c->mv_out_cap = rows;
  }
  HIPCHK(c, hipMemcpyAsync(c->mv_x, x, cols * 4, hipMemcpyHostToDevice, c->stream));
  if ((rc = enqueue_matvec(c, w, c->mv_x, c->mv_out))) return rc;
  HIPCHK(c, hipMemcpyAsync(out, c->mv_out, rows * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return TALOS_OK;
}

int talos_hip_matvec_dev(talos_hip_ctx* c, const char* name, const float* d_x, float* d_out) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!name || !d_x || !d_out) return fail(c, TALOS_ERR_ARG, "null argument");
  const DevWeight* w = find_w(c, name);
  if (!w) return fail(c, TALOS_ERR_MISSING_WEIGHT, "weight \"%s\" is not resident", name);
  return enqueue_matvec(c, w, d_x, d_out);
}

int talos_hip_bench_matvec(talos_hip_ctx* c, const char* const* names, uint32_t n_names, uint32_t reps,
                           float* avg_us, double* bytes) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!names || !n_names || !reps || !avg_us || !bytes) return fail(c, TALOS_ERR_ARG, "bad argument");
  if ((rc = set_device(c))) return rc;
  std::vector<const DevWeight*> ws(n_names);
  for (uint32_t i = 0; i < n_names; ++i) {
    ws[i] = names[i] ? find_w(c, names[i]) : nullptr;
    if (!ws[i]) return fail(c, TALOS_ERR_MISSING_WEIGHT, "weight \"%s\" is not resident", names[i] ? names[i] : "");
    if (ws[i]->rows != ws[0]->rows || ws[i]->cols != ws[0]->cols)
      return fail(c, TALOS_ERR_SHAPE, "bench matrices must share one shape");
  }
  const size_t rows = ws[0]->rows, cols = ws[0]->cols;
  float *x = nullptr, *out = nullptr;
  HIPCHK(c, hipMalloc(&x, cols * 4));
  if (hipMalloc(&out, rows * 4) != hipSuccess) {
    (void)hipFree(x);
    return fail(c, TALOS_ERR_HIP, "hipMalloc failed");
  }
  HIPCHK(c, hipMemsetAsync(x, 0, cols * 4, c->stream));
  hipEvent_t e0, e1;
  HIPCHK(c, hipEventCreate(&e0));
  HIPCHK(c, hipEventCreate(&e1));
  rc = enqueue_matvec(c, ws[0], x, out);  // warm
  if (!rc) HIPCHK(c, hipEventRecord(e0, c->stream));
  for (uint32_t r = 0; r < reps && !rc; ++r) rc = enqueue_matvec(c, ws[(r + 1) % n_names], x, out);
  if (!rc) {
    HIPCHK(c, hipEventRecord(e1, c->stream));
    HIPCHK(c, hipEventSynchronize(e1));
  }
  float ms = 0;
  if (!rc) HIPCHK(c, hipEventElapsedTime(&ms, e0, e1));
  (void)hipStreamSynchronize(c->stream);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipFree(x);
  (void)hipFree(out);
  if (rc) return rc;
  *avg_us = ms * 1000.f / (float)reps;
  *bytes = (double)ws[0]->len + 4.0 * (double)(rows + cols);
  return TALOS_OK;
}

int talos_hip_bench_kernel(talos_hip_ctx* c, const char* kind, uint32_t reps, float* avg_us, double* bytes) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!kind || !avg_us || !bytes || !reps) return fail(c, TALOS_ERR_ARG, "bad argument");
  if ((rc = set_device(c))) return rc;
  if ((rc = alloc_acts(c))) return rc;
  const std::string k(kind);
  const auto& cf = c->cfg;
  std::vector<LayerW> lw(cf.n_layer);
  for (uint32_t l = 0; l < cf.n_layer; ++l)
    if ((rc = layer_weights(c, l, &lw[l]))) return rc;
  const float* onorm = nullptr;
  const DevWeight* wout = nullptr;
  if (k == "output") {
    if ((rc = need_norm(c, "output_norm.weight", cf.n_embd, &onorm))) return rc;
    if ((rc = need_matrix(c, "output.weight", cf.vocab_size, cf.n_embd, &wout))) return rc;
  }
  const double act = 4.0 * cf.n_embd;
  double b = 0;
  if (k == "qkv") b = (double)(lw[0].q->len + lw[0].k->len + lw[0].v->len) + 2 * act + 4.0 * 2 * c->kv_dim;
  else if (k == "oproj") b = (double)lw[0].o->len + 3 * act;
  else if (k == "gateup") b = (double)(lw[0].g->len + lw[0].u->len) + 2 * act + 4.0 * cf.n_ff;
  else if (k == "down") b = (double)lw[0].d->len + 4.0 * cf.n_ff + 2 * act;
  else if (k == "output") b = (double)wout->len + 2 * act + 4.0 * cf.vocab_size;
  else return fail(c, TALOS_ERR_ARG, "unknown kernel kind \"%s\" (qkv, oproj, gateup, down, output)", kind);
  // The qkv kernel appends K/V at the device position: start from pos 0.
  if ((rc = set_state(c, 0, 0))) return rc;
  hipEvent_t e0, e1;
  HIPCHK(c, hipEventCreate(&e0));
  HIPCHK(c, hipEventCreate(&e1));
  auto launch = [&](uint32_t r) {
    const uint32_t l = r % cf.n_layer;
    if (k == "qkv") enq_qkv(c, l, lw[l]);
    else if (k == "oproj") enq_resid(c, lw[l].o, c->atty, cf.n_embd, c->q);
    else if (k == "gateup") enq_gateup(c, lw[l]);
    else if (k == "down") enq_resid(c, lw[l].d, c->h, cf.n_ff, c->q);
    else enq_output(c, wout, onorm);
  };
  launch(0);  // warm
  HIPCHK(c, hipEventRecord(e0, c->stream));
  for (uint32_t r = 0; r < reps; ++r) launch(r + 1);
  HIPCHK(c, hipEventRecord(e1, c->stream));
  HIPCHK(c, hipEventSynchronize(e1));
  float ms = 0;
  HIPCHK(c, hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *avg_us = ms * 1000.f / (float)reps;
  *bytes = b;
  return TALOS_OK;
}

int talos_hip_bench_token(talos_hip_ctx* c, uint32_t token, uint32_t pos, uint32_t reps, float* avg_us,
                          double* bytes) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!avg_us || !bytes || !reps) return fail(c, TALOS_ERR_ARG, "bad argument");
  const auto& cf = c->cfg;
  if (pos >= cf.context_length) return fail(c, TALOS_ERR_POS, "pos %u >= context_length %u", pos, cf.context_length);
  if (token >= cf.vocab_size) return fail(c, TALOS_ERR_TOKEN, "token %u >= vocab_size %u", token, cf.vocab_size);
  if ((rc = set_device(c))) return rc;
  // Algorithmic bytes of one step: every weight once (the embedding row
  // only), the K/V rows 0..pos read, the K/V row at pos written, the logits.
  double b = 0;
  for (uint32_t l = 0; l < cf.n_layer; ++l) {
    LayerW w;
    if ((rc = layer_weights(c, l, &w))) return rc;
    b += (double)(w.q->len + w.k->len + w.v->len + w.o->len + w.g->len + w.u->len + w.d->len) + 8.0 * cf.n_embd;
  }
  const DevWeight *wout, *emb;
  const float* onorm;
  if ((rc = need_matrix(c, "output.weight", cf.vocab_size, cf.n_embd, &wout)) ||
      (rc = need_norm(c, "output_norm.weight", cf.n_embd, &onorm)) ||
      (rc = need_matrix(c, "token_embd.weight", cf.vocab_size, cf.n_embd, &emb)))
    return rc;
  const double kv_row = 2.0 * 4.0 * c->kv_dim;  // K and V, f32
  b += (double)wout->len + 4.0 * cf.n_embd + (double)emb->len / cf.vocab_size;
  b += (double)cf.n_layer * kv_row * ((double)pos + 2.0) + 4.0 * cf.vocab_size;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_TOKEN, &g))) return rc;
  if ((rc = set_state(c, token, pos))) return rc;
  if ((rc = run_step(c, G_TOKEN, g))) return rc;  // warm
  hipEvent_t e0, e1;
  HIPCHK(c, hipEventCreate(&e0));
  HIPCHK(c, hipEventCreate(&e1));
  HIPCHK(c, hipEventRecord(e0, c->stream));
  for (uint32_t r = 0; r < reps && rc == TALOS_OK; ++r) rc = run_step(c, G_TOKEN, g);
  HIPCHK(c, hipEventRecord(e1, c->stream));
  HIPCHK(c, hipEventSynchronize(e1));
  float ms = 0;
  HIPCHK(c, hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  HIPCHK(c, hipMemcpy(c->h_io, c->io, 64, hipMemcpyDeviceToHost));
  if ((rc = check_device_err(c))) return rc;
  *avg_us = ms * 1000.f / (float)reps;
  *bytes = b;
  return TALOS_OK;
}

int talos_hip_bench_copy(talos_hip_ctx* c, size_t nbytes, uint32_t reps, float* avg_us) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!avg_us || !reps || nbytes < 16 || nbytes % 16) return fail(c, TALOS_ERR_ARG, "bad argument");
  if ((rc = set_device(c))) return rc;
  void *src = nullptr, *dst = nullptr;
  HIPCHK(c, hipMalloc(&src, nbytes));
  if (hipMalloc(&dst, nbytes) != hipSuccess) {
    (void)hipFree(src);
    return fail(c, TALOS_ERR_HIP, "hipMalloc of %zu bytes failed", nbytes);
  }
  const size_t n16 = nbytes / 16;
  hipDeviceProp_t prop;
  HIPCHK(c, hipGetDeviceProperties(&prop, c->cfg.device));
  const uint32_t grid = (uint32_t)prop.multiProcessorCount * 8;
  hipEvent_t e0, e1;
  HIPCHK(c, hipEventCreate(&e0));
  HIPCHK(c, hipEventCreate(&e1));
  k_fill<<<grid, 256, 0, c->stream>>>(reinterpret_cast<u4*>(src), n16);
  k_copy<<<grid, 256, 0, c->stream>>>(reinterpret_cast<const u4*>(src), reinterpret_cast<u4*>(dst), n16);
  HIPCHK(c, hipEventRecord(e0, c->stream));
  for (uint32_t r = 0; r < reps; ++r)
    k_copy<<<grid, 256, 0, c->stream>>>(reinterpret_cast<const u4*>(src), reinterpret_cast<u4*>(dst), n16);
  HIPCHK(c, hipEventRecord(e1, c->stream));
  HIPCHK(c, hipEventSynchronize(e1));
  float ms = 0;
  HIPCHK(c, hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipFree(src);
  (void)hipFree(dst);
  *avg_us = ms * 1000.f / (float)reps;
  return TALOS_OK;
}

int talos_hip_phase_timeline(talos_hip_ctx* c, uint32_t token, uint32_t pos, uint64_t* marks, size_t cap,
                             uint32_t* nblocks, uint32_t* slots, double* tick_ns) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!marks || !nblocks || !slots || !tick_ns) return fail(c, TALOS_ERR_ARG, "null argument");
  if (pos >= c->cfg.context_length) return fail(c, TALOS_ERR_POS, "pos %u >= context_length", pos);
  if (token >= c->cfg.vocab_size) return fail(c, TALOS_ERR_TOKEN, "token %u >= vocab_size", token);
  if ((rc = set_device(c))) return rc;
  hipGraphExec_t g;
  if ((rc = get_graph(c, G_TOKEN, &g))) return rc;
  if (!c->mega_fn) return fail(c, TALOS_ERR_ARG, "the persistent kernel is not in use for this model");
  const size_t per = MEGA_TL_SLOTS(c->cfg.n_layer), n = per * c->mega_blocks;
  *nblocks = c->mega_blocks;
  *slots = (uint32_t)per;
  if (cap < n) return fail(c, TALOS_ERR_ARG, "timeline needs %zu entries", n);
  uint64_t* d = nullptr;
  HIPCHK(c, hipMalloc(&d, n * 8));
  HIPCHK(c, hipMemsetAsync(d, 0, n * 8, c->stream));
  if ((rc = set_state(c, token, pos))) {
    (void)hipFree(d);
    return rc;
  }
  rc = mega_launch(c, G_TOKEN, d);
  if (!rc) {
    hipError_t e = hipMemcpyAsync(marks, d, n * 8, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) rc = fail(c, TALOS_ERR_HIP, "timeline copy: %s", hipGetErrorString(e));
  }
  (void)hipFree(d);
  int rate_khz = 0;
  (void)hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, c->cfg.device);
  *tick_ns = rate_khz > 0 ? 1e6 / rate_khz : 10.0;
  return rc;
}

int talos_hip_set_spin_limit(talos_hip_ctx* c, uint32_t polls) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  c->spin_limit = polls ? polls : TALOS_SPIN_LIMIT;
  return TALOS_OK;
}

int talos_hip_path(talos_hip_ctx* c, int* path) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  if (!path) return fail(c, TALOS_ERR_ARG, "null path");
  if ((rc = set_device(c))) return rc;
  if ((rc = prepare(c))) return rc;
  *path = c->path;
  return TALOS_OK;
}

void* talos_hip_stream(talos_hip_ctx* c) { return c ? (void*)c->stream : nullptr; }

int talos_hip_sync(talos_hip_ctx* c) {
  int rc;
  if ((rc = check_ctx(c))) return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return TALOS_OK;
}

}  // extern "C"
