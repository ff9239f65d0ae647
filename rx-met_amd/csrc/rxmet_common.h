// rxmet_common.h — shared host/device helpers of the MI355X quantization library:
// error reporting for the C ABI, HIP error checks and wavefront reductions (gfx950,
// 64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>

namespace rxmet {

// Thread-local message of the last failing C-ABI call.
void set_error(const std::string &msg);
void clear_error();

struct Status {
  int code = 0;
};

// Asynchronous host -> device copy of a small per-call table (through pinned staging; the
// source may be reused as soon as the call returns).  0 or a negative error (message set).
int upload(void *dst, const void *src, size_t bytes, hipStream_t stream);

namespace prof {
// Brackets the launches made during its lifetime with a pair of hipEvents on `stream`
// when event timing is enabled (rxmet_prof_enable); `name` must be a string literal.
bool enabled();
class Scope {
 public:
  Scope(const char *name, hipStream_t stream);
  ~Scope();
  Scope(const Scope &) = delete;
  Scope &operator=(const Scope &) = delete;

 private:
  const char *name_;
  hipStream_t stream_;
  hipEvent_t start_ = nullptr;
};
}  // namespace prof

}  // namespace rxmet

#define RXMET_CHECK_ARG(cond, msg)          \
  do {                                      \
    if (!(cond)) {                          \
      rxmet::set_error(std::string(msg));   \
      return -22;                           \
    }                                       \
  } while (0)

#define RXMET_CHECK_HIP(expr)                                                        \
  do {                                                                               \
    hipError_t err__ = (expr);                                                       \
    if (err__ != hipSuccess) {                                                       \
      rxmet::set_error(std::string(#expr) + ": " + hipGetErrorString(err__));        \
      return -5;                                                                     \
    }                                                                                \
  } while (0)

// Launch-error check after a kernel launch (asynchronous errors surface later on the
// caller's stream synchronisation).
#define RXMET_CHECK_LAUNCH() RXMET_CHECK_HIP(hipGetLastError())

namespace rxmet {

constexpr int kWave = 64;

// Native 4-wide fp32 vector (maps to 128-bit global loads/stores and is accepted by
// the nontemporal builtins).
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// NaN-propagating min/max (a NaN anywhere makes the result NaN, like torch.min/max).
__device__ __forceinline__ float nan_min(float a, float b) {
  return (b < a || b != b) ? b : a;
}
__device__ __forceinline__ float nan_max(float a, float b) {
  return (b > a || b != b) ? b : a;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = nan_min(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, kWave));
  return v;
}

// Clamp that keeps NaN (torch.clamp semantics): comparisons with NaN are false, so a
// NaN input falls through unchanged.
__device__ __forceinline__ float clamp_keep_nan(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

}  // namespace rxmet
