// sample.h -- token sampling and per-token NLL on the device.
//
// k_sample restates src/sample.rs:19-76 for one row of logits in one
// 1024-thread workgroup: temperature <= 0 is the greedy argmax (ties to the
// last index); otherwise the logits are sorted descending (total_cmp order,
// equal logits by descending index), cut to top_k, turned into
// temperature-scaled softmax probabilities over the kept set, cut to the
// shortest prefix whose cumulative probability reaches top_p, and the token
// whose cumulative probability first reaches u times the kept mass is drawn
// (u: the caller's uniform draw, the reference's rng.gen::<f32>()).
//
// The sort is a stable LSD radix sort of 64-bit keys (the logit's total_cmp
// key above its index, complemented so that an ascending sort is the
// wanted order), four bits per pass, each thread owning a contiguous run of
// elements; passes whose digit is the same for every element are skipped
// (the high index bits).  Sums and prefix sums run per thread over its run,
// then across threads in thread order: deterministic, and within float
// rounding of the reference's sequential sums.
//
// k_nll restates src/eval.rs:17-22: -log softmax(logits)[target] with the
// max in f32 and the exponential sum in f64.
#pragma once
#include "device_common.h"

#define SAMPLE_NT 1024
#define SAMPLE_NW (SAMPLE_NT / 64)

struct SampleArgs {
  const float* logits;
  uint32_t n;
  float temperature;
  uint32_t top_k;  // 0: no top-k cut
  float top_p;     // > 1 or NaN: no top-p cut
  float u;         // the uniform draw in [0, 1) (used when u_dev is null)
  const float* u_dev;  // optional: draws per step, u_dev[state[ST_STEP]] (the device decode loop)
  uint64_t* ka;    // scratch: n keys
  uint64_t* kb;    // scratch: n keys
  float* pb;       // scratch: n floats
  uint32_t* out;   // the drawn token (nullable)
  int32_t* state;  // optional: device token state to advance (decode loop)
  int32_t* tokens;
};

// Block-wide exclusive scan of one uint32 per thread (SAMPLE_NT threads);
// returns the exclusive prefix, *total the sum.  Uses sh[SAMPLE_NW + 1].
__device__ __forceinline__ uint32_t block_excl_scan_u(uint32_t v, uint32_t* sh, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0;
    for (int w = 0; w < SAMPLE_NW; ++w) {
      const uint32_t t = sh[w];
      sh[w] = a;
      a += t;
    }
    sh[SAMPLE_NW] = a;
  }
  __syncthreads();
  const uint32_t r = sh[wave] + x - v;
  *total = sh[SAMPLE_NW];
  __syncthreads();
  return r;
}

// The same for floats, summed in thread order (fixed association).
__device__ __forceinline__ float block_excl_scan_f(float v, float* sh, float* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = 0.f;
    for (int w = 0; w < SAMPLE_NW; ++w) {
      const float t = sh[w];
      sh[w] = a;
      a += t;
    }
    sh[SAMPLE_NW] = a;
  }
  __syncthreads();
  // exclusive within the wave: x - v would round differently; shift instead
  float ex = __shfl_up(x, 1, 64);
  if (lane == 0) ex = 0.f;
  const float r = sh[wave] + ex;
  *total = sh[SAMPLE_NW];
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_min_u(uint32_t v, uint32_t* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o, 64));
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  uint32_t m = sh[0];
  for (int w = 1; w < SAMPLE_NW; ++w) m = min(m, sh[w]);
  __syncthreads();
  return m;
}

// Largest total_cmp key, ties to the larger index (src/sample.rs:7-14).
__device__ __forceinline__ uint32_t block_argmax(const float* logits, uint32_t n, int32_t* shk, int32_t* shi) {
  int32_t bk = INT32_MIN, bi = -1;
  for (uint32_t i = threadIdx.x; i < n; i += SAMPLE_NT) {
    const int32_t k = total_key(logits[i]);
    if (k > bk || (k == bk && (int32_t)i > bi)) {
      bk = k;
      bi = (int32_t)i;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int32_t ok = __shfl_xor(bk, o, 64), oi = __shfl_xor(bi, o, 64);
    if (ok > bk || (ok == bk && oi > bi)) {
      bk = ok;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    shk[wave] = bk;
    shi[wave] = bi;
  }
  __syncthreads();
  bk = shk[0];
  bi = shi[0];
  for (int w = 1; w < SAMPLE_NW; ++w)
    if (shk[w] > bk || (shk[w] == bk && shi[w] > bi)) {
      bk = shk[w];
      bi = shi[w];
    }
  __syncthreads();
  return (uint32_t)bi;
}

// Element i's sort key: ascending order of the key is descending total_cmp
// order of the logit, equal logits by descending index.
__device__ __forceinline__ uint64_t sample_key(float l, uint32_t i) {
  const uint32_t k = (uint32_t)total_key(l) ^ 0x80000000u;  // unsigned, monotone
  return ~(((uint64_t)k << 32) | i);
}

__global__ __launch_bounds__(SAMPLE_NT) void k_sample(SampleArgs A) {
  __shared__ uint32_t cnt[16][SAMPLE_NT];  // per-thread digit counts, then their exclusive offsets
  __shared__ uint32_t shu[SAMPLE_NW + 1];
  __shared__ uint32_t dtot[16];
  __shared__ float shf[SAMPLE_NW + 1];
  __shared__ int32_t shk[SAMPLE_NW], shi[SAMPLE_NW];
  const uint32_t n = A.n, tid = threadIdx.x;
  int32_t step = 0;
  if (A.state) step = A.state[3];  // ST_STEP
  const float u = A.u_dev ? A.u_dev[step] : A.u;
  uint32_t token;
  if (!(A.temperature > 0.f)) {
    token = block_argmax(A.logits, n, shk, shi);
  } else {
    // contiguous run of C elements per thread
    const uint32_t C = (n + SAMPLE_NT - 1) / SAMPLE_NT;
    const uint32_t e0 = min(n, tid * C), e1 = min(n, e0 + C);
    for (uint32_t i = e0; i < e1; ++i) A.ka[i] = sample_key(A.logits[i], i);
    uint64_t* src = A.ka;
    uint64_t* dst = A.kb;
    __threadfence();
    __syncthreads();
    for (int shift = 0; shift < 64; shift += 4) {
      uint32_t c[16];
#pragma unroll
      for (int d = 0; d < 16; ++d) c[d] = 0;
      for (uint32_t i = e0; i < e1; ++i) {
        const uint32_t d = (uint32_t)(src[i] >> shift) & 15u;
#pragma unroll
        for (int k = 0; k < 16; ++k) c[k] += d == (uint32_t)k;
      }
#pragma unroll
      for (int d = 0; d < 16; ++d) cnt[d][tid] = c[d];
      __syncthreads();
      // exclusive scan of cnt in digit-major order: thread t scans row
      // t / 64, entries [16 (t % 64), +16)
      const uint32_t row = tid >> 6, seg = (tid & 63) * 16;
      uint32_t loc[16], sum = 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        loc[k] = sum;
        sum += cnt[row][seg + k];
      }
      // digit totals: row d is wave d's 64 segments
      uint32_t dsum = sum;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) dsum += __shfl_xor(dsum, o, 64);
      if ((tid & 63) == 0) dtot[row] = dsum;
      uint32_t total;
      const uint32_t base = block_excl_scan_u(sum, shu, &total);
      // a digit shared by every element leaves the order as it is
      bool skip = false;
#pragma unroll
      for (int d = 0; d < 16; ++d) skip = skip || dtot[d] == n;
#pragma unroll
      for (int k = 0; k < 16; ++k) cnt[row][seg + k] = base + loc[k];
      __syncthreads();
      if (!skip) {
        uint32_t off[16];
#pragma unroll
        for (int d = 0; d < 16; ++d) off[d] = cnt[d][tid];
        for (uint32_t i = e0; i < e1; ++i) {
          const uint64_t v = src[i];
          const uint32_t d = (uint32_t)(v >> shift) & 15u;
          uint32_t o = 0;
#pragma unroll
          for (int k = 0; k < 16; ++k)
            if (d == (uint32_t)k) o = off[k]++;
          dst[o] = v;
        }
        // other threads read these keys next pass: agent-scope fence (the
        // vector L1 may hold lines of this buffer from two passes ago)
        __threadfence();
        __syncthreads();
        uint64_t* t = src;
        src = dst;
        dst = t;
      }
      __syncthreads();
    }
    // src: sorted keys.  Kept set, probabilities, cut, draw.
    const uint32_t K = A.top_k == 0 ? n : min(max(A.top_k, 1u), n);
    const uint32_t CK = (K + SAMPLE_NT - 1) / SAMPLE_NT;
    const uint32_t j0 = min(K, tid * CK), j1 = min(K, j0 + CK);
    const float maxv = A.logits[(uint32_t)(~src[0])];
    float ps = 0.f;
    for (uint32_t j = j0; j < j1; ++j) {
      const float p = expf((A.logits[(uint32_t)(~src[j])] - maxv) / A.temperature);
      A.pb[j] = p;
      ps += p;
    }
    float S;
    (void)block_excl_scan_f(ps, shf, &S);
    // cumulative normalised probabilities
    float cs = 0.f;
    for (uint32_t j = j0; j < j1; ++j) cs += A.pb[j] / S;
    float tot;
    float run = block_excl_scan_f(cs, shf, &tot);
    for (uint32_t j = j0; j < j1; ++j) {
      run += A.pb[j] / S;
      A.pb[j] = run;
    }
    __threadfence();
    __syncthreads();
    uint32_t m = K;
    if (A.top_p <= 1.0f) {  // NaN or > 1: no cut
      uint32_t first = 0xFFFFFFFFu;
      for (uint32_t j = j0; j < j1; ++j)
        if (A.pb[j] >= A.top_p) {
          first = j;
          break;
        }
      first = block_min_u(first, shu);
      if (first != 0xFFFFFFFFu) m = first + 1;
    }
    const float r = u * A.pb[m - 1];
    uint32_t pick = 0xFFFFFFFFu;
    for (uint32_t j = j0; j < min(j1, m); ++j)
      if (A.pb[j] >= r) {
        pick = j;
        break;
      }
    pick = block_min_u(pick, shu);
    if (pick == 0xFFFFFFFFu) pick = m - 1;
    token = (uint32_t)(~src[pick]);
  }
  if (threadIdx.x == 0) {
    if (A.out) A.out[0] = token;
    if (A.state) {  // the decode loop: this token is the next input (advance_state mode 2)
      A.state[2] = (int32_t)token;  // ST_ARGMAX slot keeps the drawn token
      A.tokens[step] = (int32_t)token;
      A.state[1] = (int32_t)token;  // ST_TOKEN
      A.state[0] = A.state[0] + 1;  // ST_POS
      A.state[3] = step + 1;        // ST_STEP
    }
  }
}

// nll[0] = -log softmax(logits)[target] (src/eval.rs:17-22).
__global__ __launch_bounds__(256) void k_nll(const float* __restrict__ logits, uint32_t n, uint32_t target,
                                             float* __restrict__ nll) {
  __shared__ float shm[4];
  __shared__ double shd[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = -INFINITY;
  for (uint32_t i = threadIdx.x; i < n; i += 256) m = fmaxf(m, logits[i]);
  m = wave_max(m);
  if (lane == 0) shm[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(shm[0], shm[1]), fmaxf(shm[2], shm[3]));
  double s = 0.0;
  for (uint32_t i = threadIdx.x; i < n; i += 256) s += exp((double)(logits[i] - m));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0) shd[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double sum = ((shd[0] + shd[1]) + shd[2]) + shd[3];
    const double lp = (double)(logits[target] - m) - log(sum);
    nll[0] = (float)(-lp);
  }
}
