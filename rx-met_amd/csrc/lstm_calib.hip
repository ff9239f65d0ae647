// lstm_calib.hip — float LSTM forward with MinMax statistics (PTQ calibration pass) and the
// plain float forward, behind rxmet_lstm_forward_calibrate / rxmet_lstm_forward_float.
//
// Reference: CalibrationSession.collect -> LstmCalibrationCollector::collect
// (src/lstm/calibration.cc:154-240) over lstmForwardFloatCpu (src/lstm/forward_float_cpu.cc:
// 57-153); the CUDA session runs the same observation set on device traces
// (src/lstm/calibration_cuda.cu:372-480).  One workgroup per sequence keeps h and c in LDS
// and walks the T steps with the reference's summation order (bias first, then the
// products in index order); exp and tanh are evaluated in double and rounded once to float.
// Observed: x, h (h0 or zeros, then every h_t), c (c0 or zeros, then every c_t), both
// linears, the four gate inputs and outputs, tanh(c), and per-channel parameter ranges.
// Non-finite values are counted (the reference rejects them) instead of entering a range.
#include <cfloat>

#include "rxmet_common.h"
#include "rxmet_lstm.h"

namespace rxmet {
namespace lstm {

constexpr int kCalThreads = 256;
constexpr int kN = RXMET_LSTM_NOPS;

__device__ __forceinline__ unsigned f2ord(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(unsigned u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

struct Obs {
  float mn[kN], mx[kN];
  unsigned bad;
};

__device__ __forceinline__ void observe(Obs &o, int op, float v) {
  if (isfinite(v)) {
    o.mn[op] = fminf(o.mn[op], v);
    o.mx[op] = fmaxf(o.mx[op], v);
  } else {
    ++o.bad;
  }
}

__device__ __forceinline__ float sigm(float x) {
  if (x >= 0.0f) {
    const float e = static_cast<float>(exp(-static_cast<double>(x)));
    return 1.0f / (1.0f + e);
  }
  const float e = static_cast<float>(exp(static_cast<double>(x)));
  return e / (1.0f + e);
}
__device__ __forceinline__ float tnh(float x) { return static_cast<float>(tanh(static_cast<double>(x))); }

template <bool STATS>
__global__ __launch_bounds__(kCalThreads) void lstm_float_forward(
    int T, int B, int I, int H, const float *__restrict__ Wi, const float *__restrict__ Wh,
    const float *__restrict__ bi, const float *__restrict__ bh, const float *__restrict__ x,
    const float *__restrict__ h0, const float *__restrict__ c0, float *__restrict__ out,
    float *__restrict__ hn, float *__restrict__ cn, unsigned *__restrict__ gstat /* 2*kN + 1 */) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = 4 * H;
  float *hs = reinterpret_cast<float *>(smem);  // [H]
  float *cs = hs + H;                           // [H]
  float *gates = cs + H;                        // [4H]
  __shared__ unsigned smin[kN], smax[kN], sbad;
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid < kN) {
    smin[tid] = f2ord(INFINITY);
    smax[tid] = f2ord(-INFINITY);
  }
  if (tid == 0) sbad = 0;
  Obs o;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    o.mn[i] = INFINITY;
    o.mx[i] = -INFINITY;
  }
  o.bad = 0;
  for (int j = tid; j < H; j += kCalThreads) {
    const size_t s = static_cast<size_t>(b) * H + j;
    hs[j] = h0 ? h0[s] : 0.0f;
    cs[j] = c0 ? c0[s] : 0.0f;
    if (STATS) {
      observe(o, RXMET_LSTM_OUTPUT, hs[j]);
      observe(o, RXMET_LSTM_CELL_STATE, cs[j]);
    }
  }
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const float *xt = x + (static_cast<size_t>(t) * B + b) * I;
    if (STATS)
      for (int k = tid; k < I; k += kCalThreads) observe(o, RXMET_LSTM_INPUT, xt[k]);
    for (int c = tid; c < C; c += kCalThreads) {
      float li = bi ? bi[c] : 0.0f, lh = bh ? bh[c] : 0.0f;
      const float *wi = Wi + static_cast<size_t>(c) * I, *wh = Wh + static_cast<size_t>(c) * H;
      for (int k = 0; k < I; ++k) li += wi[k] * xt[k];
      for (int k = 0; k < H; ++k) lh += wh[k] * hs[k];
      const float gsum = li + lh;
      gates[c] = gsum;
      if (STATS) {
        observe(o, RXMET_LSTM_IH_LINEAR, li);
        observe(o, RXMET_LSTM_HH_LINEAR, lh);
        observe(o, RXMET_LSTM_I_GATE_IN + c / H, gsum);
      }
    }
    __syncthreads();
    for (int j = tid; j < H; j += kCalThreads) {
      const float ig = sigm(gates[j]), fg = sigm(gates[H + j]);
      const float gg = tnh(gates[2 * H + j]), og = sigm(gates[3 * H + j]);
      const float cnew = fg * cs[j] + ig * gg;
      const float ct = tnh(cnew);
      const float hv = og * ct;
      cs[j] = cnew;
      hs[j] = hv;  // every gate of this step is already in `gates`
      out[(static_cast<size_t>(t) * B + b) * H + j] = hv;
      if (STATS) {
        observe(o, RXMET_LSTM_I_GATE_OUT, ig);
        observe(o, RXMET_LSTM_F_GATE_OUT, fg);
        observe(o, RXMET_LSTM_G_GATE_OUT, gg);
        observe(o, RXMET_LSTM_O_GATE_OUT, og);
        observe(o, RXMET_LSTM_CELL_STATE, cnew);
        observe(o, RXMET_LSTM_CELL_TANH, ct);
        observe(o, RXMET_LSTM_OUTPUT, hv);
      }
    }
    __syncthreads();
  }
  for (int j = tid; j < H; j += kCalThreads) {
    const size_t s = static_cast<size_t>(b) * H + j;
    hn[s] = hs[j];
    cn[s] = cs[j];
  }
  if (!STATS) return;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    if (o.mn[i] <= o.mx[i]) {
      atomicMin(&smin[i], f2ord(o.mn[i]));
      atomicMax(&smax[i], f2ord(o.mx[i]));
    }
  }
  if (o.bad) atomicAdd(&sbad, o.bad);
  __syncthreads();
  if (tid < kN) {
    atomicMin(&gstat[tid], smin[tid]);
    atomicMax(&gstat[kN + tid], smax[tid]);
  }
  if (tid == 0 && sbad) atomicAdd(&gstat[2 * kN], sbad);
}

__global__ void lstm_stats_init(unsigned *o) {
  const int i = threadIdx.x;
  if (i < kN) {
    o[i] = f2ord(INFINITY);
    o[kN + i] = f2ord(-INFINITY);
  }
  if (i == 0) o[2 * kN] = 0u;
}

__global__ void lstm_stats_merge(const unsigned *o, float *s, int64_t count_index) {
  const int i = threadIdx.x;
  if (i < kN) {
    const float lo = ord2f(o[i]), hi = ord2f(o[kN + i]);
    s[i] = fminf(s[i], lo);
    s[kN + i] = fmaxf(s[kN + i], hi);
  }
  if (i == 0) s[count_index] += static_cast<float>(o[2 * kN]);
}

// Per-channel ranges of W_ih / W_hh rows and biases, merged into the running ranges; a
// non-finite parameter value is counted.
__global__ __launch_bounds__(64) void lstm_param_stats(int I, int H, const float *Wi,
                                                       const float *Wh, const float *bi,
                                                       const float *bh, float *chan,
                                                       unsigned *bad) {
  const int C = 4 * H;
  const int c = blockIdx.x, l = threadIdx.x;
  const float *src[4] = {Wi + static_cast<size_t>(c) * I, Wh + static_cast<size_t>(c) * H,
                         bi ? bi + c : nullptr, bh ? bh + c : nullptr};
  const int n[4] = {I, H, 1, 1};
  unsigned nb = 0;
  for (int k = 0; k < 4; ++k) {
    if (!src[k]) continue;
    float lo = INFINITY, hi = -INFINITY;
    for (int e = l; e < n[k]; e += 64) {
      const float v = src[k][e];
      if (isfinite(v)) {
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      } else {
        ++nb;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    if (l == 0) {
      float *mn = chan + static_cast<size_t>(k) * 2 * C, *mx = mn + C;
      mn[c] = fminf(mn[c], lo);
      mx[c] = fmaxf(mx[c], hi);
    }
  }
  if (nb) atomicAdd(bad, nb);
}

}  // namespace lstm
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::lstm;

extern "C" {

int64_t rxmet_lstm_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  (void)T; (void)B; (void)I; (void)H;
  return static_cast<int64_t>(sizeof(unsigned) * (2 * kN + 1));
}

static int launch_float(bool stats, int T, int B, int I, int H, const float *Wi, const float *Wh,
                        const float *bi, const float *bh, const float *x, const float *h0,
                        const float *c0, float *out, float *hn, float *cn, unsigned *ord,
                        hipStream_t stream) {
  const size_t lds = sizeof(float) * 6 * static_cast<size_t>(H);
  const void *fn = stats ? reinterpret_cast<const void *>(&lstm_float_forward<true>)
                         : reinterpret_cast<const void *>(&lstm_float_forward<false>);
  if (lds > 64 * 1024)
    RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
  if (stats)
    hipLaunchKernelGGL(lstm_float_forward<true>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I,
                       H, Wi, Wh, bi, bh, x, h0, c0, out, hn, cn, ord);
  else
    hipLaunchKernelGGL(lstm_float_forward<false>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I,
                       H, Wi, Wh, bi, bh, x, h0, c0, out, hn, cn, ord);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_lstm_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                                 const float *W_hh, const float *b_ih, const float *b_hh,
                                 const float *x, const float *h0, const float *c0,
                                 float *output, float *h_n, float *c_n, float *stats,
                                 void *workspace, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 8192, "hidden_size above 8192 is not supported by the calibration pass");
  RXMET_CHECK_ARG(W_ih && W_hh && x && output && h_n && c_n && stats && workspace,
                  "required pointer is null");
  RXMET_CHECK_ARG((h0 == nullptr) == (c0 == nullptr), "h0 and c0 must be given together");
  RXMET_CHECK_ARG((b_ih == nullptr) == (b_hh == nullptr), "b_ih and b_hh must be given together");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  unsigned *ord = static_cast<unsigned *>(workspace);
  hipLaunchKernelGGL(lstm_stats_init, dim3(1), dim3(64), 0, stream, ord);
  RXMET_CHECK_LAUNCH();
  {
    rxmet::prof::Scope ps__("lstm_calibrate_forward", stream);
    if (int rc = launch_float(true, T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, output, h_n, c_n,
                              ord, stream))
      return rc;
  }
  hipLaunchKernelGGL(lstm_param_stats, dim3(4 * H), dim3(64), 0, stream, I, H, W_ih, W_hh, b_ih,
                     b_hh, stats + 2 * kN, ord + 2 * kN);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(lstm_stats_merge, dim3(1), dim3(64), 0, stream, ord, stats,
                     rxmet_lstm_stats_size(H) - 1);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_lstm_forward_float(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0, float *output,
                             float *h_n, float *c_n, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 8192, "hidden_size above 8192 is not supported by the float forward");
  RXMET_CHECK_ARG(W_ih && W_hh && x && output && h_n && c_n, "required pointer is null");
  RXMET_CHECK_ARG((h0 == nullptr) == (c0 == nullptr), "h0 and c0 must be given together");
  RXMET_CHECK_ARG((b_ih == nullptr) == (b_hh == nullptr), "b_ih and b_hh must be given together");
  return launch_float(false, T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, output, h_n, c_n,
                      nullptr, static_cast<hipStream_t>(stream_));
}

}  // extern "C"
