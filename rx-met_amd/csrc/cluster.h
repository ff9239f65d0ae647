// cluster.h — workgroup clusters inside one cooperative launch.
//
// A persistent recurrence splits one batch tile's hidden units over G workgroups (a cluster).
// Each step the members exchange the new hidden codes through global memory and meet at a
// counter in global memory.  The launch is cooperative, so every workgroup is resident; the
// wait is still bounded: after a limit of polls a member gives up, raises the timeout flag
// and stops stepping, so every wave of the grid reaches the end of the kernel.
#pragma once

#include <cstdlib>

#include <hip/hip_runtime.h>

namespace rxmet {
namespace cluster {

constexpr unsigned kSpinLimit = 1u << 20;  // about a second of polling

// Words between two clusters' barrier counters: each counter has a 256-byte line of its own.
// Counters sharing a line serialise every cluster's arrivals and polls at that line; with the
// 32 clusters of the two-direction c3 GRU forward on one line, a step whose workgroups reach
// the barrier early took 1.55 ms against 0.82 ms with the counters apart.  A launch of n
// clusters takes kCounterStride * n + 1 words: the counters, then the timeout flag.
constexpr int kCounterStride = 64;

// The poll limit a launch passes to its waits: kSpinLimit, or RXMET_TEST_SPIN_LIMIT from the
// environment.  Tests of the timeout path set it to 0, so that a wait that has to poll gives
// up at once: the launch then takes the path of a real timeout (flag raised, members stop
// stepping, every wave reaches the end of the kernel, outputs poisoned with NaN).
inline unsigned spin_limit() {
  const char *s = std::getenv("RXMET_TEST_SPIN_LIMIT");
  return s != nullptr ? static_cast<unsigned>(std::strtoul(s, nullptr, 10)) : kSpinLimit;
}

struct Place {
  int cluster, member;
};

// Block index -> (cluster, member).  The dispatcher deals workgroups round-robin over the
// eight XCDs, so members that share blockIdx % 8 share an L2; the mapping keeps a cluster on
// one XCD when the cluster count is a multiple of 8.  Correctness does not depend on it.
__device__ __forceinline__ Place place(int G, int nclusters) {
  const int b = blockIdx.x;
  if (nclusters % 8 == 0) {
    const int xcd = b % 8, slot = b / 8;
    return {xcd + 8 * (slot / G), slot % G};
  }
  return {b / G, b % G};
}

// Cluster barrier.  Every thread of the workgroup calls it after its stores of exchanged data;
// the counter counts arrivals monotonically, so `arrivals` is G times the barrier's ordinal.
// Returns false when the wait timed out (the caller then stops stepping).
//
// Exchanged data must be written with store_coherent and read with load_coherent (agent-scope
// atomic accesses, which bypass the non-coherent caches).  Arrival waits for the wave's own
// stores to complete before the workgroup barrier, so every exchanged store of the workgroup
// is complete before thread 0 increments the counter; a member that has seen the count reach
// `arrivals` then reads the new values from the coherence point.  No L2 writeback or
// invalidation is needed, because nothing exchanged lives in a non-coherent cache line.
//
// The ordering rests on the ISA rather than on the language memory model: the exchanged
// stores and loads are agent-scope atomics (global_store/global_load with sc1), and
// s_waitcnt vmcnt(0) returns only once a wave's sc1 stores are complete at the coherence
// point.  The language-level form — a release fetch_add and an acquire fence after the poll
// — compiles on gfx950 to buffer_wbl2 sc1 before the increment and buffer_inv sc1 after the
// wait (write back, then invalidate, the whole XCD's L2), issued by every workgroup at every
// step.  Measured on the c3 GRU step: 6.10 ms against 3.50 ms; c4 LSTM step 4.41 against
// 3.37 ms.  Nothing here needs that cache maintenance.
__device__ __forceinline__ bool sync(unsigned *counter, unsigned arrivals, int *timeout,
                                     unsigned limit) {
  __shared__ int ok;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int good = 1;
    unsigned spins = 0;
    while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < arrivals) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > limit) {
        good = 0;
        __hip_atomic_store(timeout, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    ok = good;
  }
  __syncthreads();
  return ok != 0;
}

// The barrier in two halves, so that stores the other members do not read (outputs,
// checkpoints) can be issued between them and drain while the workgroup waits.
// arrive: every thread calls it after its exchanged stores; wait: every thread calls it once,
// after arrive, and gets false when the wait timed out.
__device__ __forceinline__ void arrive(unsigned *counter) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool wait(unsigned *counter, unsigned arrivals, int *timeout,
                                     unsigned limit) {
  __shared__ int ok;
  if (threadIdx.x == 0) {
    int good = 1;
    unsigned spins = 0;
    while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < arrivals) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > limit) {
        good = 0;
        __hip_atomic_store(timeout, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    ok = good;
  }
  __syncthreads();
  return ok != 0;
}

__device__ __forceinline__ void store_coherent(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes at a 16-byte aligned address, as two coherent 8-byte loads.
__device__ __forceinline__ int4 load_coherent16(const void *p) {
  const unsigned long long *q = static_cast<const unsigned long long *>(p);
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_int4(static_cast<int>(a), static_cast<int>(a >> 32), static_cast<int>(b),
                   static_cast<int>(b >> 32));
}

// Buffer resource over `bytes` bytes at `base` (raw addressing, 32-bit offsets).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

// 16 bytes at a 16-byte aligned byte offset of a buffer in one instruction, with the cache policy
// of an agent-scope atomic load (sc1: served from the coherence point, never from a stale
// non-coherent line).  The 16 bytes are not one atomic access; the exchange never needs that,
// since every exchanged store is complete before the barrier that precedes the load.
__device__ __forceinline__ int4 load_coherent16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  constexpr int kSc1 = 16;  // cache-policy operand: sc1
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
  return make_int4(static_cast<int>(v[0]), static_cast<int>(v[1]), static_cast<int>(v[2]),
                   static_cast<int>(v[3]));
}

// Store one byte per lane as packed 32-bit words: lanes 4k..4k+3 (which hold consecutive
// bytes of the destination) combine into lane 4k, which writes the word at `dst4` (the
// address of lane 4k's byte; lanes 4k+1..3 pass an ignored pointer).
__device__ __forceinline__ void store_bytes_coherent(unsigned char *dst4, int byte) {
  const int lane = threadIdx.x % 64;
  byte &= 255;
  const int b1 = __shfl_down(byte, 1, 64), b2 = __shfl_down(byte, 2, 64),
            b3 = __shfl_down(byte, 3, 64);
  if ((lane & 3) == 0)
    store_coherent(reinterpret_cast<unsigned *>(dst4),
                   static_cast<unsigned>(byte | (b1 << 8) | (b2 << 16) | (b3 << 24)));
}

// Zero `n` words (counters and flags) on the stream; used instead of a memset node so the
// sequence stays capturable.
[[maybe_unused]] static __global__ void zero_words(unsigned *p, int n) {
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

// Blocks of 256 threads for zero_words over n words (grid-strided, at most 1024 blocks).
[[maybe_unused]] static inline unsigned zero_blocks(int64_t n) {
  const int64_t b = (n + 1023) / 1024;
  return static_cast<unsigned>(b < 1 ? 1 : (b > 1024 ? 1024 : b));
}

// A launch whose cluster wait timed out leaves untrustworthy outputs: overwrite `n` floats
// with NaN when the timeout flag is set (a no-op otherwise).
[[maybe_unused]] static __global__ void poison_nan(const int *timeout, int64_t n, float *p) {
  if (*timeout == 0) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = NAN;
}

// The same for two outputs of n floats each (q may be null).
[[maybe_unused]] static __global__ void poison_nan2(const int *timeout, int64_t n, float *p, float *q) {
  if (*timeout == 0) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    p[i] = NAN;
    if (q) q[i] = NAN;
  }
}

// Every output of a computation whose recurrence timed out: up to 12 float buffers (null
// entries are skipped), all overwritten with NaN when the flag is set.  Launched after the
// last kernel that writes any of them, so nothing downstream of a stuck launch (weight and
// input gradients built from partly written gate gradients included) can look finite.
struct PoisonList {
  float *p[12];
  int64_t n[12];
  int count;
};

[[maybe_unused]] static __global__ void poison_list(const int *timeout, PoisonList l) {
  if (*timeout == 0) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int k = 0; k < l.count; ++k) {
    float *p = l.p[k];
    if (p == nullptr) continue;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < l.n[k];
         i += stride)
      p[i] = NAN;
  }
}

// Launch a clustered recurrence.  The launch is cooperative, which guarantees that every
// workgroup of the grid is resident at once.  With RXMET_PLAIN_LAUNCH set it is an ordinary
// launch of the same grid (for profilers that cannot trace cooperative launches): residency
// then holds only while nothing else occupies the GPU, and a wait that times out poisons the
// outputs with NaN instead of hanging.
inline hipError_t launch(const void *fn, dim3 grid, dim3 block, void **args, unsigned lds,
                         hipStream_t stream) {
  if (std::getenv("RXMET_PLAIN_LAUNCH") != nullptr)
    return hipLaunchKernel(fn, grid, block, args, lds, stream);
  return hipLaunchCooperativeKernel(fn, grid, block, args, lds, stream);
}

}  // namespace cluster
}  // namespace rxmet
