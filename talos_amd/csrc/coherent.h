// coherent.h -- cross-workgroup data exchange inside one persistent kernel.
//
// The per-XCD L2 caches of MI355X are not coherent with each other while a
// kernel runs.  Data one workgroup produces for another is written with
// agent-scope relaxed atomic stores (global_store ... sc1, written through),
// and the producer waits for its stores to complete (s_waitcnt) before it
// signals.  A buffer written once per launch and read only after the barrier
// that follows the write can then be read with ordinary cached loads: caches
// are invalidated at kernel start, so no cache holds a copy of a line that
// nobody read before it was written.  Words rewritten within a launch (flags,
// counters) move with relaxed atomic loads (sc1).  Every wait is bounded: on
// timeout the kernel records an error and stops waiting, so it always drains.
#pragma once
#include "device_common.h"

__device__ __forceinline__ float ld_coh(const float* p) {
  return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coh_u(const uint32_t* p) {
  return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u(uint32_t* p, uint32_t v) {
  __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coh_i(const int32_t* p) {
  return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_i(int32_t* p, int32_t v) {
  __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes as two 8-byte coherent accesses (p 16-byte aligned).
__device__ __forceinline__ f4 ld_coh4(const float* p) {
  const uint64_t a = __hip_atomic_load(gptr(reinterpret_cast<const uint64_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b =
      __hip_atomic_load(gptr(reinterpret_cast<const uint64_t*>(p + 2)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return f4{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
            __uint_as_float((uint32_t)(b >> 32))};
}
__device__ __forceinline__ void st_coh4(float* p, f4 v) {
  const uint64_t a = (uint64_t)__float_as_uint(v.x) | ((uint64_t)__float_as_uint(v.y) << 32);
  const uint64_t b = (uint64_t)__float_as_uint(v.z) | ((uint64_t)__float_as_uint(v.w) << 32);
  __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(p)), a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(p + 2)), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this thread's outstanding memory operations have completed.
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// Default poll limit of every bounded wait (MegaParams::spin_limit).
#define TALOS_SPIN_LIMIT (1u << 20)

struct GridSync {
  uint32_t* flags;   // [nblocks * 16]: one 64-byte line per block
  uint32_t* go;      // release word written by block 0
  uint32_t* err;     // set to 1 when a wait timed out
  uint32_t* packed;  // [nblocks rounded up to 4], 8-byte aligned: the same arrivals, one word per block
  uint32_t nblocks;
  uint32_t spin;     // polls before a wait gives up
  int one_hop;       // grid_wait: every block reads the packed arrivals itself
};

// Shared flag: a wait timed out before this barrier, so it is skipped.
__device__ __forceinline__ uint32_t& barrier_skip() {
  __shared__ uint32_t timed_out;
  return timed_out;
}

// Grid barrier with epoch `ep` (monotonic, compared modulo 2^32), in two
// halves so that a block can issue independent loads between them.
// grid_arrive: all threads' prior stores are complete, then the block
// publishes its arrival.  grid_wait: block 0 gathers all arrivals and
// publishes `go`; the others wait for `go`.  Vector memory operations of a
// wave complete in issue order, so loads issued between the halves delay
// that wave's view of the barrier; block 0 must not issue any.
__device__ __forceinline__ void grid_arrive(const GridSync& g, uint32_t ep) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    barrier_skip() = ld_coh_u(g.err);
    st_coh_u(g.flags + blockIdx.x * 16, ep);
    st_coh_u(g.packed + blockIdx.x, ep);
  }
}

// Arrival words b0 .. b0 + 3 of the packed array have reached ep (words at
// or beyond nblocks count as reached).
__device__ __forceinline__ bool packed_reached(const GridSync& g, uint32_t b0, uint32_t ep) {
  const uint64_t* p = reinterpret_cast<const uint64_t*>(g.packed + b0);
  const uint64_t a = __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t c = __hip_atomic_load(gptr(p + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t w[4] = {(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)c, (uint32_t)(c >> 32)};
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 4; ++i) ok &= b0 + i >= g.nblocks || (int32_t)(w[i] - ep) >= 0;
  return ok;
}

__device__ __forceinline__ void grid_wait(const GridSync& g, uint32_t ep) {
  __syncthreads();
  const bool skip = barrier_skip() != 0;
  if (g.one_hop) {
    // wave 0 reads all arrivals, four words per lane per pass (nblocks <=
    // 8192); a lane stops reading words that have arrived, so a long wait
    // ends up polling only the stragglers' words
    if (threadIdx.x < 64 && !skip) {
      uint32_t pending = 0;  // bit k: words 4 * lane + 256 k .. +3 not all arrived yet
      for (uint32_t k = 0, b0 = threadIdx.x * 4; b0 < g.nblocks && k < 32; b0 += 256, ++k) pending |= 1u << k;
      uint32_t s = 0;
      for (;;) {
        for (uint32_t p = pending; p; p &= p - 1) {
          const uint32_t k = __builtin_ctz(p);
          if (packed_reached(g, threadIdx.x * 4 + 256 * k, ep)) pending &= ~(1u << k);
        }
        if (__all(pending == 0)) break;
        if (++s > g.spin) {
          if (threadIdx.x == 0) st_coh_u(g.err, 1u);
          break;
        }
      }
    }
  } else if (blockIdx.x == 0) {
    if (!skip) {
      for (uint32_t w = threadIdx.x; w < g.nblocks; w += blockDim.x) {
        uint32_t s = 0;
        while ((int32_t)(ld_coh_u(g.flags + w * 16) - ep) < 0) {
          if (++s > g.spin) {
            st_coh_u(g.err, 1u);
            break;
          }
        }
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) st_coh_u(g.go, ep);
  } else if (threadIdx.x == 0 && !skip) {
    uint32_t s = 0;
    while ((int32_t)(ld_coh_u(g.go) - ep) < 0) {
      if (++s > g.spin) {
        st_coh_u(g.err, 1u);
        break;
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void grid_barrier(const GridSync& g, uint32_t ep) {
  grid_arrive(g, ep);
  grid_wait(g, ep);
}
