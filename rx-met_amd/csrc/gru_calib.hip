// gru_calib.hip — float GRU forward with MinMax statistics (PTQ calibration pass),
// behind rxmet_gru_forward_calibrate.
//
// The same kernel without statistics is the float forward behind rxmet_gru_forward_fp.
//
// Reference: forwardWithCalibrationCPU (operators/quant-gru/src/gru_forward_cpu.cc:58-151)
// and its GPU counterpart forwardWithCalibrationGPU (src/gru_interface.cc:930-1024).
// One workgroup per sequence keeps h in LDS and walks the T steps; the two linears use
// the reference's sequential fp32 summation order (sum over k, then + bias), sigmoid is
// evaluated in double as the reference's CPU template does, so h, v and the statistics
// match the CPU reference up to the device's tanhf/exp last-ulp behaviour.  Statistics
// of the 13 activations ignore non-finite values, are reduced with atomic min/max on
// order-preserving integer images of the floats and then merged into the caller's
// running ranges; per-channel ranges of W, R, bw and br are reduced
// by a separate kernel.
#include <cfloat>

#include "rxmet_common.h"
#include "rxmet_gru.h"

namespace rxmet {
namespace gru {

constexpr int kCalThreads = 256;
constexpr int kNStat = RXMET_GRU_NGRIDS;

// Order-preserving float <-> uint for atomic min/max on floats.
__device__ __forceinline__ unsigned f2ord(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(unsigned u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

__device__ __forceinline__ void observe(float v, float &mn, float &mx) {
  if (isfinite(v)) {
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
}

template <bool STATS>
__global__ __launch_bounds__(kCalThreads) void calib_forward(
    int T, int B, int I, int H, const float *__restrict__ W, const float *__restrict__ R,
    const float *__restrict__ bw, const float *__restrict__ br, const float *__restrict__ x,
    const float *__restrict__ h0, float *__restrict__ hout, float *__restrict__ v,
    unsigned *__restrict__ gstat /* 2 x 13 ordered (min, max) */) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = 3 * H;
  float *hbuf = reinterpret_cast<float *>(smem);  // [2][H], h_t and h_{t+1}
  float *wx = hbuf + 2 * H;                       // [3H]
  float *rh = wx + C;                             // [3H]
  __shared__ unsigned smin[kNStat], smax[kNStat];
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid < kNStat) {
    smin[tid] = f2ord(FLT_MAX);
    smax[tid] = f2ord(-FLT_MAX);
  }
  const size_t BH = static_cast<size_t>(B) * H;
  for (int j = tid; j < H; j += kCalThreads) {
    const float v0 = h0 ? h0[static_cast<size_t>(b) * H + j] : 0.0f;
    hbuf[j] = v0;
    hout[static_cast<size_t>(b) * H + j] = v0;
  }
  float mn[kNStat], mx[kNStat];
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    mn[i] = FLT_MAX;
    mx[i] = -FLT_MAX;
  }
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const float *hs = hbuf + (t & 1) * H;
    float *hn_s = hbuf + ((t + 1) & 1) * H;
    const float *xt = x + (static_cast<size_t>(t) * B + b) * I;
    if (STATS)
      for (int k = tid; k < I; k += kCalThreads) observe(xt[k], mn[RXMET_GRU_X], mx[RXMET_GRU_X]);
    for (int c = tid; c < C; c += kCalThreads) {
      float si = 0.0f, sh = 0.0f;
      for (int k = 0; k < I; ++k) si += xt[k] * W[static_cast<size_t>(k) * C + c];
      for (int k = 0; k < H; ++k) sh += hs[k] * R[static_cast<size_t>(k) * C + c];
      const float a = si + bw[c], r = sh + br[c];
      wx[c] = a;
      rh[c] = r;
      if (STATS) {
        observe(a, mn[RXMET_GRU_WX], mx[RXMET_GRU_WX]);
        observe(r, mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
      }
    }
    __syncthreads();
    for (int j = tid; j < H; j += kCalThreads) {
      const float zp = wx[j] + rh[j];
      const float rp = wx[H + j] + rh[H + j];
      const float z = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(zp))));
      const float r = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(rp))));
      const float rec = rh[2 * H + j];
      const float rhm = r * rec;
      const float np = wx[2 * H + j] + rhm;
      const float n = tanhf(np);
      const float oldc = z * hs[j];
      const float newc = (1.0f - z) * n;
      const float hn = oldc + newc;
      if (STATS) {
        observe(zp, mn[RXMET_GRU_Z_IN], mx[RXMET_GRU_Z_IN]);
        observe(rp, mn[RXMET_GRU_R_IN], mx[RXMET_GRU_R_IN]);
        observe(np, mn[RXMET_GRU_N_IN], mx[RXMET_GRU_N_IN]);
        observe(z, mn[RXMET_GRU_Z_OUT], mx[RXMET_GRU_Z_OUT]);
        observe(r, mn[RXMET_GRU_R_OUT], mx[RXMET_GRU_R_OUT]);
        observe(n, mn[RXMET_GRU_N_OUT], mx[RXMET_GRU_N_OUT]);
        observe(rhm, mn[RXMET_GRU_MUL_RH], mx[RXMET_GRU_MUL_RH]);
        observe(newc, mn[RXMET_GRU_MUL_NEW], mx[RXMET_GRU_MUL_NEW]);
        observe(oldc, mn[RXMET_GRU_MUL_OLD], mx[RXMET_GRU_MUL_OLD]);
        observe(hn, mn[RXMET_GRU_H], mx[RXMET_GRU_H]);
      }
      hout[(t + 1) * BH + static_cast<size_t>(b) * H + j] = hn;
      if (v) {
        float *vb = v + (static_cast<size_t>(t) * B + b) * 4 * H + j;
        vb[0] = z;
        vb[H] = r;
        vb[2 * H] = n;
        vb[3 * H] = rec;
      }
      hn_s[j] = hn;
    }
    __syncthreads();
  }
  if (!STATS) return;
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    if (mn[i] <= mx[i]) {
      atomicMin(&smin[i], f2ord(mn[i]));
      atomicMax(&smax[i], f2ord(mx[i]));
    }
  }
  __syncthreads();
  if (tid < kNStat) {
    atomicMin(&gstat[tid], smin[tid]);
    atomicMax(&gstat[kNStat + tid], smax[tid]);
  }
}

// This call's ranges start empty (min=FLT_MAX, max=-FLT_MAX) in ordered-uint form.
__global__ void stats_init(unsigned *o) {
  const int i = threadIdx.x;
  if (i < kNStat) {
    o[i] = f2ord(FLT_MAX);
    o[kNStat + i] = f2ord(-FLT_MAX);
  }
}
// Merge this call's ranges into the running ones.  A tensor without any finite value
// contributes the range [0, 0], as the reference's min/max update does.
__global__ void stats_merge(const unsigned *o, float *s) {
  const int i = threadIdx.x;
  if (i < kNStat) {
    float lo = ord2f(o[i]), hi = ord2f(o[kNStat + i]);
    if (lo > hi) lo = hi = 0.0f;
    s[i] = lo < s[i] ? lo : s[i];
    s[kNStat + i] = hi > s[kNStat + i] ? hi : s[kNStat + i];
  }
}

// Per-channel min/max of W [I,3H], R [H,3H], bw, br merged into the running ranges.
__global__ __launch_bounds__(256) void calib_params(int I, int H, const float *W, const float *R,
                                                    const float *bw, const float *br,
                                                    float *chan /* 4 x (min[C], max[C]) */) {
  const int C = 3 * H;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const float *src[4] = {W, R, bw, br};
  const int rows[4] = {I, H, 1, 1};
  for (int k = 0; k < 4; ++k) {
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (int r = 0; r < rows[k]; ++r) {
      const float v = src[k][static_cast<size_t>(r) * C + c];
      if (isfinite(v)) {
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      }
    }
    if (lo > hi) lo = hi = 0.0f;
    float *mn = chan + static_cast<size_t>(k) * 2 * C, *mx = mn + C;
    mn[c] = lo < mn[c] ? lo : mn[c];
    mx[c] = hi > mx[c] ? hi : mx[c];
  }
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int64_t rxmet_gru_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  (void)T; (void)B; (void)I; (void)H;
  return static_cast<int64_t>(sizeof(unsigned) * 2 * kNStat);
}

int rxmet_gru_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W,
                                const float *R, const float *bw, const float *br,
                                const float *x, const float *h0, float *h, float *v,
                                float *stats, void *workspace, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 4096, "hidden_size above 4096 is not supported by the calibration pass");
  RXMET_CHECK_ARG(W && R && bw && br && x && h && stats && workspace, "required pointer is null");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  unsigned *ord = static_cast<unsigned *>(workspace);
  hipLaunchKernelGGL(stats_init, dim3(1), dim3(64), 0, stream, ord);
  RXMET_CHECK_LAUNCH();
  const size_t lds = sizeof(float) * 8 * static_cast<size_t>(H);
  if (lds > 64 * 1024)
    RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&calib_forward<true>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
  {
    rxmet::prof::Scope ps__("gru_calibrate_forward", stream);
    hipLaunchKernelGGL(calib_forward<true>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I, H, W, R, bw,
                       br, x, h0, h, v, ord);
  }
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(stats_merge, dim3(1), dim3(64), 0, stream, ord, stats);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(calib_params, dim3((3 * H + 255) / 256), dim3(256), 0, stream, I, H, W, R, bw,
                     br, stats + 2 * kNStat);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_gru_forward_fp(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                         const float *W, const float *R, const float *bw, const float *br,
                         const float *x, const float *h0, float *h, float *v, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 4096, "hidden_size above 4096 is not supported by the float forward");
  RXMET_CHECK_ARG(W && R && bw && br && x && h, "required pointer is null");
  RXMET_CHECK_ARG(!is_training || v, "v is required when is_training is set");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const size_t lds = sizeof(float) * 8 * static_cast<size_t>(H);
  if (lds > 64 * 1024)
    RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&calib_forward<false>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
  hipLaunchKernelGGL(calib_forward<false>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I, H, W,
                     R, bw, br, x, h0, h, is_training ? v : nullptr, nullptr);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
