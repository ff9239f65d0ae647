// qdq.hip — MI355X (gfx950) streaming fake-quantization kernels behind rxmet_qdq.h.
//
// The AIMET reference runs QuantizeDequantize as a chain of PyTorch elementwise ops
// (src/aimet_torch/v2/quantization/affine/backends/torch_builtins.py:618-691): about seven
// full HBM passes forward and ten backward plus broadcast reductions.  Here each
// direction is one pass:
//   forward  : read x, write y                                   (8 B/element)
//   backward : read x and g, write dx, reduce encoding gradients (12 B/element)
//   min/max  : read x                                            (4 B/element)
//
// Work decomposition.  The tensor is [outer, C, inner]; a "run" is one contiguous
// stretch of `inner` elements sharing one encoding.  When runs are long (or the
// encoding is per-tensor) every workgroup streams one CHUNK of one run with f4
// accesses and wave-uniform (scalar) encoding loads.  When runs are short (per-channel
// on a trailing axis) a "column" decomposition is used instead: threads own columns of
// the [outer, C*inner] matrix and walk rows, so accesses stay coalesced.  Reductions
// write one fp64 partial per workgroup (or per column and row-chunk) and a second
// kernel folds the partials of each encoding in a fixed order, so results are
// deterministic and need no atomics.
#include <mutex>
#include <string>

#include "rxmet_common.h"
#include "rxmet_qdq.h"

namespace rxmet {
namespace qdq {

enum Op { OP_QDQ_LEARN = 0, OP_QDQ_FROZEN = 1, OP_Q = 2, OP_DQ = 3 };

constexpr int kThreads = 256;
constexpr int kVecPerThread = 8;                            // f4 per thread per chunk
constexpr int64_t kChunk = kThreads * kVecPerThread * 4;    // 8192 elements
constexpr int64_t kMinRun = 1024;                           // shorter runs use columns
constexpr int kColTargetBlocks = 2048;

struct Enc {
  float s, o, inv_s, zp, qmin, qmax;
};

__device__ __forceinline__ Enc load_enc(const float *scale, const float *offset, int64_t c,
                                        float qmin, float qmax) {
  Enc e;
  e.s = scale[c];
  e.o = offset ? offset[c] : 0.0f;
  e.inv_s = 1.0f / e.s;  // torch's fake_quantize kernels multiply by fp32 1/scale
  e.zp = -truncf(e.o);   // zero point = -offset.to(int32)
  e.qmin = qmin;
  e.qmax = qmax;
  return e;
}

template <int OP>
__device__ __forceinline__ float fwd_elem(float x, const Enc &e) {
  if constexpr (OP == OP_QDQ_LEARN) {
    const float r = rintf(x / e.s) - e.o;
    return (clamp_keep_nan(r, e.qmin, e.qmax) + e.o) * e.s;
  } else if constexpr (OP == OP_QDQ_FROZEN) {
    const float r = rintf(x * e.inv_s) + e.zp;
    return (clamp_keep_nan(r, e.qmin, e.qmax) - e.zp) * e.s;
  } else if constexpr (OP == OP_Q) {
    const float r = rintf(x / e.s) - e.o;
    return clamp_keep_nan(r, e.qmin, e.qmax);
  } else {
    return (x + e.o) * e.s;
  }
}

// One element of the backward: returns dx and adds this element's encoding-gradient
// terms to (ds, dof).
template <int OP>
__device__ __forceinline__ float bwd_elem(float x, float g, const Enc &e, double &ds,
                                          double &dof) {
  if constexpr (OP == OP_QDQ_LEARN) {
    const float xs = x / e.s;
    const float rr = rintf(xs);
    const float r = rr - e.o;
    const float m = (r >= e.qmin && r <= e.qmax) ? 1.0f : 0.0f;
    const float lo = e.o + e.qmin, hi = e.o + e.qmax;
    ds += static_cast<double>(g * (clamp_keep_nan(rr, lo, hi) - xs * m));
    dof += static_cast<double>(g * ((1.0f - m) * e.s));
    return g * m;
  } else if constexpr (OP == OP_QDQ_FROZEN) {
    const float r = rintf(x * e.inv_s) + e.zp;
    const float m = (r >= e.qmin && r <= e.qmax) ? 1.0f : 0.0f;
    return g * m;
  } else if constexpr (OP == OP_Q) {
    const float r = rintf(x / e.s) - e.o;
    const float m = (r >= e.qmin && r <= e.qmax) ? 1.0f : 0.0f;
    const float mg = g * m;
    const float gs = mg / e.s;
    ds += static_cast<double>(-gs * (x / e.s));
    dof += static_cast<double>(-mg);
    return gs;
  } else {
    const float gs = g * e.s;
    ds += static_cast<double>(g * (x + e.o));
    dof += static_cast<double>(gs);
    return gs;
  }
}

// ---------------------------------------------------------------------------------
// Block-wide reductions (256 threads = 4 waves).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void block_sum2(double &a, double &b) {
  __shared__ double sa[kThreads / kWave], sb[kThreads / kWave];
  a = wave_sum(a);
  b = wave_sum(b);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  if (lane == 0) {
    sa[w] = a;
    sb[w] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    a = sa[0];
    b = sb[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i) {
      a += sa[i];
      b += sb[i];
    }
  }
}

__device__ __forceinline__ void block_minmax(float &mn, float &mx) {
  __shared__ float smn[kThreads / kWave], smx[kThreads / kWave];
  mn = wave_min(mn);
  mx = wave_max(mx);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  if (lane == 0) {
    smn[w] = mn;
    smx[w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    mn = smn[0];
    mx = smx[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i) {
      mn = nan_min(mn, smn[i]);
      mx = nan_max(mx, smx[i]);
    }
  }
}

// ---------------------------------------------------------------------------------
// Run decomposition: block b handles chunk (b % splits) of run (b / splits).
// ---------------------------------------------------------------------------------
template <int OP>
__global__ __launch_bounds__(kThreads) void fwd_runs(const float *__restrict__ x,
                                                     float *__restrict__ y, int64_t inner,
                                                     int64_t C, int64_t splits,
                                                     const float *__restrict__ scale,
                                                     const float *__restrict__ offset,
                                                     float qmin, float qmax, int vec4) {
  const int64_t b = blockIdx.x;
  const int64_t run = b / splits, sp = b % splits;
  const Enc e = load_enc(scale, offset, run % C, qmin, qmax);
  const int64_t beg = sp * kChunk;
  const int64_t end = min(inner, beg + kChunk);
  const int64_t base = run * inner + beg;
  if (vec4) {
    const f4 *xv = reinterpret_cast<const f4 *>(x + base);
    f4 *yv = reinterpret_cast<f4 *>(y + base);
    const int nv = static_cast<int>((end - beg) >> 2);
    f4 v[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) v[k] = __builtin_nontemporal_load(xv + i);
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) {
        f4 o;
        o.x = fwd_elem<OP>(v[k].x, e);
        o.y = fwd_elem<OP>(v[k].y, e);
        o.z = fwd_elem<OP>(v[k].z, e);
        o.w = fwd_elem<OP>(v[k].w, e);
        __builtin_nontemporal_store(o, yv + i);
      }
    }
  } else {
    const int n = static_cast<int>(end - beg);
    for (int i = threadIdx.x; i < n; i += kThreads) y[base + i] = fwd_elem<OP>(x[base + i], e);
  }
}

template <int OP, bool ENC>
__global__ __launch_bounds__(kThreads) void bwd_runs(
    const float *__restrict__ x, const float *__restrict__ g, float *__restrict__ dx,
    int64_t inner, int64_t C, int64_t splits, const float *__restrict__ scale,
    const float *__restrict__ offset, float qmin, float qmax, int vec4,
    double2 *__restrict__ partial) {
  const int64_t b = blockIdx.x;
  const int64_t run = b / splits, sp = b % splits;
  const Enc e = load_enc(scale, offset, run % C, qmin, qmax);
  const int64_t beg = sp * kChunk;
  const int64_t end = min(inner, beg + kChunk);
  const int64_t base = run * inner + beg;
  double ds = 0.0, dof = 0.0;
  if (vec4) {
    const f4 *xv = reinterpret_cast<const f4 *>(x + base);
    const f4 *gv = reinterpret_cast<const f4 *>(g + base);
    f4 *dv = reinterpret_cast<f4 *>(dx + base);
    const int nv = static_cast<int>((end - beg) >> 2);
    f4 xr[kVecPerThread], gr[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) {
        xr[k] = __builtin_nontemporal_load(xv + i);
        gr[k] = __builtin_nontemporal_load(gv + i);
      }
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) {
        f4 o;
        o.x = bwd_elem<OP>(xr[k].x, gr[k].x, e, ds, dof);
        o.y = bwd_elem<OP>(xr[k].y, gr[k].y, e, ds, dof);
        o.z = bwd_elem<OP>(xr[k].z, gr[k].z, e, ds, dof);
        o.w = bwd_elem<OP>(xr[k].w, gr[k].w, e, ds, dof);
        __builtin_nontemporal_store(o, dv + i);
      }
    }
  } else {
    const int n = static_cast<int>(end - beg);
    for (int i = threadIdx.x; i < n; i += kThreads)
      dx[base + i] = bwd_elem<OP>(x[base + i], g[base + i], e, ds, dof);
  }
  if constexpr (ENC) {
    block_sum2(ds, dof);
    if (threadIdx.x == 0) partial[b] = make_double2(ds, dof);
  }
}

__global__ __launch_bounds__(kThreads) void minmax_runs(const float *__restrict__ x,
                                                        int64_t inner, int64_t splits,
                                                        int vec4, float2 *__restrict__ partial) {
  const int64_t b = blockIdx.x;
  const int64_t run = b / splits, sp = b % splits;
  const int64_t beg = sp * kChunk;
  const int64_t end = min(inner, beg + kChunk);
  const int64_t base = run * inner + beg;
  float mn = INFINITY, mx = -INFINITY;
  if (vec4) {
    const f4 *xv = reinterpret_cast<const f4 *>(x + base);
    const int nv = static_cast<int>((end - beg) >> 2);
    f4 v[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) v[k] = __builtin_nontemporal_load(xv + i);
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) {
        mn = nan_min(nan_min(mn, v[k].x), nan_min(v[k].y, nan_min(v[k].z, v[k].w)));
        mx = nan_max(nan_max(mx, v[k].x), nan_max(v[k].y, nan_max(v[k].z, v[k].w)));
      }
    }
  } else {
    const int n = static_cast<int>(end - beg);
    for (int i = threadIdx.x; i < n; i += kThreads) {
      mn = nan_min(mn, x[base + i]);
      mx = nan_max(mx, x[base + i]);
    }
  }
  block_minmax(mn, mx);
  if (threadIdx.x == 0) partial[b] = make_float2(mn, mx);
}

// ---------------------------------------------------------------------------------
// Column decomposition for short runs: matrix [M = outer, K = C * inner]; block b owns
// columns [tile * 256, +256) of rows [chunk * rows_per_chunk, +rows_per_chunk).
// ---------------------------------------------------------------------------------
template <int OP>
__global__ __launch_bounds__(kThreads) void fwd_elementwise(const float *__restrict__ x,
                                                            float *__restrict__ y, int64_t n,
                                                            int64_t C, int64_t inner,
                                                            const float *__restrict__ scale,
                                                            const float *__restrict__ offset,
                                                            float qmin, float qmax) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    const Enc e = load_enc(scale, offset, (i / inner) % C, qmin, qmax);
    y[i] = fwd_elem<OP>(x[i], e);
  }
}

template <int OP, bool ENC>
__global__ __launch_bounds__(kThreads) void bwd_cols(
    const float *__restrict__ x, const float *__restrict__ g, float *__restrict__ dx,
    int64_t M, int64_t K, int64_t inner, int64_t col_tiles, int64_t rows_per_chunk,
    const float *__restrict__ scale, const float *__restrict__ offset, float qmin,
    float qmax, double2 *__restrict__ partial) {
  const int64_t tile = blockIdx.x % col_tiles, chunk = blockIdx.x / col_tiles;
  const int64_t j = tile * kThreads + threadIdx.x;
  if (j >= K) return;
  const Enc e = load_enc(scale, offset, j / inner, qmin, qmax);
  const int64_t r0 = chunk * rows_per_chunk;
  const int64_t r1 = min(M, r0 + rows_per_chunk);
  double ds = 0.0, dof = 0.0;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t i = r * K + j;
    dx[i] = bwd_elem<OP>(x[i], g[i], e, ds, dof);
  }
  if constexpr (ENC) partial[chunk * K + j] = make_double2(ds, dof);
}

__global__ __launch_bounds__(kThreads) void minmax_cols(const float *__restrict__ x, int64_t M,
                                                        int64_t K, int64_t col_tiles,
                                                        int64_t rows_per_chunk,
                                                        float2 *__restrict__ partial) {
  const int64_t tile = blockIdx.x % col_tiles, chunk = blockIdx.x / col_tiles;
  const int64_t j = tile * kThreads + threadIdx.x;
  if (j >= K) return;
  const int64_t r0 = chunk * rows_per_chunk;
  const int64_t r1 = min(M, r0 + rows_per_chunk);
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t r = r0; r < r1; ++r) {
    const float v = x[r * K + j];
    mn = nan_min(mn, v);
    mx = nan_max(mx, v);
  }
  partial[chunk * K + j] = make_float2(mn, mx);
}

// ---------------------------------------------------------------------------------
// Partial folding: one wavefront per encoding c.  Partial p of encoding c lives at
//   runs:    ((o * C + c) * splits + s)    for o < outer, s < splits
//   columns: (h * K + c * inner + k)       for h < chunks, k < inner
// Each lane folds a fixed, strided subset; lanes are then combined by a fixed butterfly.
// ---------------------------------------------------------------------------------
struct FoldMap {
  int64_t a_count, a_stride;  // outer loop (o or h)
  int64_t b_count, b_stride;  // inner loop (s or k)
  int64_t c_stride;           // encoding stride
};

__device__ __forceinline__ int64_t fold_index(const FoldMap &f, int64_t c, int64_t p) {
  const int64_t a = p / f.b_count, bb = p % f.b_count;
  return a * f.a_stride + c * f.c_stride + bb * f.b_stride;
}

// NT threads per encoding (one wave, or four waves for encodings with many partials); the
// waves' sums are added in a fixed order.
template <int NT>
__global__ __launch_bounds__(NT) void fold_sum(const double2 *__restrict__ partial, FoldMap f,
                                               float *__restrict__ dscale,
                                               float *__restrict__ doffset) {
  __shared__ double red[2][NT / kWave];
  const int64_t c = blockIdx.x;
  const int64_t n = f.a_count * f.b_count;
  double a = 0.0, b = 0.0;
  for (int64_t p = threadIdx.x; p < n; p += NT) {
    const double2 v = partial[fold_index(f, c, p)];
    a += v.x;
    b += v.y;
  }
  a = wave_sum(a);
  b = wave_sum(b);
  if (NT > kWave) {
    if (threadIdx.x % kWave == 0) {
      red[0][threadIdx.x / kWave] = a;
      red[1][threadIdx.x / kWave] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0)
      for (int w = 1; w < NT / kWave; ++w) {
        a += red[0][w];
        b += red[1][w];
      }
  }
  if (threadIdx.x == 0) {
    if (dscale) dscale[c] = static_cast<float>(a);
    if (doffset) doffset[c] = static_cast<float>(b);
  }
}

__global__ __launch_bounds__(kWave) void fold_minmax(const float2 *__restrict__ partial, FoldMap f,
                                                     float *__restrict__ out_min,
                                                     float *__restrict__ out_max) {
  const int64_t c = blockIdx.x;
  const int64_t n = f.a_count * f.b_count;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t p = threadIdx.x; p < n; p += kWave) {
    const float2 v = partial[fold_index(f, c, p)];
    mn = nan_min(mn, v.x);
    mx = nan_max(mx, v.y);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if (threadIdx.x == 0) {
    out_min[c] = mn;
    out_max[c] = mx;
  }
}

// ---------------------------------------------------------------------------------
// Host-side planning.
// ---------------------------------------------------------------------------------
struct Plan {
  bool cols = false;
  int64_t outer = 0, C = 0, inner = 0;
  // runs
  int64_t runs = 0, splits = 0;
  // columns
  int64_t M = 0, K = 0, col_tiles = 0, rows_per_chunk = 0, chunks = 0;
  int64_t partial_slots = 0;
  FoldMap fold{};
};

static Plan make_plan(int64_t outer, int64_t C, int64_t inner) {
  Plan p;
  if (C == 1) {  // every element shares the encoding: one long run
    inner = outer * inner;
    outer = 1;
  }
  p.outer = outer;
  p.C = C;
  p.inner = inner;
  if (C == 1 || inner >= kMinRun) {
    p.cols = false;
    p.runs = outer * C;
    p.splits = (inner + kChunk - 1) / kChunk;
    p.partial_slots = p.runs * p.splits;
    p.fold = FoldMap{outer, C * p.splits, p.splits, 1, p.splits};
  } else {
    p.cols = true;
    p.M = outer;
    p.K = C * inner;
    p.col_tiles = (p.K + kThreads - 1) / kThreads;
    int64_t chunks = kColTargetBlocks / p.col_tiles;
    chunks = chunks < 1 ? 1 : (chunks > p.M ? p.M : chunks);
    p.rows_per_chunk = (p.M + chunks - 1) / chunks;
    p.chunks = (p.M + p.rows_per_chunk - 1) / p.rows_per_chunk;
    p.partial_slots = p.chunks * p.K;
    p.fold = FoldMap{p.chunks, p.K, inner, 1, inner};
  }
  return p;
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int check_layout(int64_t outer, int64_t C, int64_t inner) {
  RXMET_CHECK_ARG(outer >= 0 && C >= 1 && inner >= 0, "invalid layout: need outer>=0, C>=1, inner>=0");
  RXMET_CHECK_ARG(outer <= (int64_t(1) << 40) / (C * (inner > 0 ? inner : 1)),
                  "tensor too large");
  return 0;
}

template <int OP>
static int launch_forward(const float *x, float *y, int64_t outer, int64_t C, int64_t inner,
                          const float *scale, const float *offset, float qmin, float qmax,
                          hipStream_t stream) {
  const Plan p = make_plan(outer, C, inner);
  const int64_t n = p.outer * p.C * p.inner;
  if (n == 0) return 0;
  rxmet::prof::Scope ps__("qdq_forward_stream", stream);
  if (!p.cols) {
    const int vec4 = (p.inner % 4 == 0) && aligned16(x) && aligned16(y);
    hipLaunchKernelGGL(fwd_runs<OP>, dim3(static_cast<unsigned>(p.runs * p.splits)),
                       dim3(kThreads), 0, stream, x, y, p.inner, p.C, p.splits, scale, offset,
                       qmin, qmax, vec4);
  } else {
    int64_t blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fwd_elementwise<OP>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                       0, stream, x, y, n, p.C, p.inner, scale, offset, qmin, qmax);
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}

template <int OP, bool ENC>
static int launch_backward_impl(const Plan &p, const float *x, const float *g, float *dx,
                                float *dscale, float *doffset, const float *scale,
                                const float *offset, float qmin, float qmax, double2 *ws,
                                hipStream_t stream) {
  {
    rxmet::prof::Scope ps__("qdq_backward_stream", stream);
    if (!p.cols) {
      const int vec4 = (p.inner % 4 == 0) && aligned16(x) && aligned16(g) && aligned16(dx);
      hipLaunchKernelGGL((bwd_runs<OP, ENC>), dim3(static_cast<unsigned>(p.runs * p.splits)),
                         dim3(kThreads), 0, stream, x, g, dx, p.inner, p.C, p.splits, scale,
                         offset, qmin, qmax, vec4, ws);
    } else {
      hipLaunchKernelGGL((bwd_cols<OP, ENC>), dim3(static_cast<unsigned>(p.col_tiles * p.chunks)),
                         dim3(kThreads), 0, stream, x, g, dx, p.M, p.K, p.inner, p.col_tiles,
                         p.rows_per_chunk, scale, offset, qmin, qmax, ws);
    }
  }
  RXMET_CHECK_LAUNCH();
  if constexpr (ENC) {
    rxmet::prof::Scope ps__("qdq_backward_fold", stream);
    if (p.fold.a_count * p.fold.b_count >= 1024)
      hipLaunchKernelGGL(fold_sum<4 * kWave>, dim3(static_cast<unsigned>(p.C)), dim3(4 * kWave), 0,
                         stream, ws, p.fold, dscale, doffset);
    else
      hipLaunchKernelGGL(fold_sum<kWave>, dim3(static_cast<unsigned>(p.C)), dim3(kWave), 0, stream,
                         ws, p.fold, dscale, doffset);
    RXMET_CHECK_LAUNCH();
  }
  return 0;
}

__global__ __launch_bounds__(256) void zero_enc_grads(int64_t C, float *dscale, float *doffset) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= C) return;
  if (dscale) dscale[i] = 0.0f;
  if (doffset) doffset[i] = 0.0f;
}

template <int OP>
static int launch_backward(const float *x, const float *g, float *dx, float *dscale,
                           float *doffset, int64_t outer, int64_t C, int64_t inner,
                           const float *scale, const float *offset, float qmin, float qmax,
                           void *workspace, hipStream_t stream) {
  const Plan p = make_plan(outer, C, inner);
  const int64_t n = p.outer * p.C * p.inner;
  const bool enc = dscale != nullptr || doffset != nullptr;
  if (n == 0) {
    // zeroed by a kernel, not a memset node, so a captured training step replays correctly
    if (enc && C > 0) {
      hipLaunchKernelGGL(zero_enc_grads, dim3(static_cast<unsigned>((C + 255) / 256)), dim3(256), 0,
                         stream, C, dscale, doffset);
      RXMET_CHECK_LAUNCH();
    }
    return 0;
  }
  if (enc) {
    RXMET_CHECK_ARG(workspace != nullptr, "encoding gradients need a workspace");
    return launch_backward_impl<OP, true>(p, x, g, dx, dscale, doffset, scale, offset, qmin,
                                          qmax, static_cast<double2 *>(workspace), stream);
  }
  return launch_backward_impl<OP, false>(p, x, g, dx, nullptr, nullptr, scale, offset, qmin,
                                         qmax, nullptr, stream);
}

static int check_grid(int64_t qmin, int64_t qmax) {
  RXMET_CHECK_ARG(qmin <= qmax, "qmin must be <= qmax");
  RXMET_CHECK_ARG(qmin >= -(int64_t(1) << 24) && qmax <= (int64_t(1) << 24),
                  "grid not exactly representable in fp32 (|q| > 2^24)");
  return 0;
}

// Encodings of learnable min / max, one thread per encoding (see rxmet_qdq_encoding_forward).
__global__ __launch_bounds__(256) void encoding_fwd(int64_t n, const float *__restrict__ mn,
                                                    const float *__restrict__ mx, float inv_steps,
                                                    float qmin, float qmax, int symmetric,
                                                    float sym_offset, float min_scale,
                                                    float *__restrict__ scale,
                                                    float *__restrict__ offset) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  // a tensor divided by a scalar is evaluated on the GPU as a product with the rounded
  // reciprocal of the scalar
  float s = fabsf((mx[c] - mn[c]) * inv_steps);
  s = s < min_scale ? min_scale : s;  // clamp_min keeps NaN
  scale[c] = s;
  if (symmetric) {
    offset[c] = sym_offset;
  } else {
    float o = rintf(mn[c] / s) - qmin;
    o = o < -qmax ? -qmax : o;
    o = o > -qmin ? -qmin : o;
    offset[c] = o;
  }
}

__global__ __launch_bounds__(256) void encoding_bwd(int64_t n, const float *__restrict__ mn,
                                                    const float *__restrict__ mx,
                                                    const float *__restrict__ g_scale,
                                                    const float *__restrict__ g_offset, float inv_steps,
                                                    float qmin, float qmax, int symmetric,
                                                    float min_scale, float *__restrict__ d_min,
                                                    float *__restrict__ d_max) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  const float raw = (mx[c] - mn[c]) * inv_steps, a = fabsf(raw);
  const float s = a < min_scale ? min_scale : a;
  float gs = g_scale ? g_scale[c] : 0.0f, gmin = 0.0f;
  if (!symmetric && g_offset) {
    const float o = rintf(mn[c] / s) - qmin;
    const float gr = (o >= -qmax && o <= -qmin) ? g_offset[c] : 0.0f;  // clamp, then STE round
    gmin += gr / s;                                                   // d(min / s) / d min
    gs += -gr * ((mn[c] / s) / s);                                    // d(min / s) / d s
  }
  const float ga = a >= min_scale ? gs : 0.0f;  // clamp_min
  const float sg = raw > 0.0f ? 1.0f : (raw < 0.0f ? -1.0f : 0.0f);
  const float gr2 = (ga * sg) * inv_steps;      // d|raw| and d((max - min) / steps)
  d_max[c] = gr2;
  d_min[c] = gmin - gr2;
}

}  // namespace qdq
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::qdq;

namespace rxmet {
namespace qdq {

// Scratch of rxmet_qdq_backward_noalloc: the per-block partial sums of the encoding
// gradients, in a file-scope device array instead of a caller workspace.  Each device holds
// its own copy for the life of the process.  Every slot a call uses is written by its block
// before the fold reads it, so nothing needs clearing between calls.
constexpr int64_t kNoAllocScratchBytes = RXMET_QDQ_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) double2 scratch[kNoAllocScratchBytes / sizeof(double2)];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void *scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device (the array's
// host-side name is not a device address).
static int scratch_address(void **out) {
  int dev = 0;
  RXMET_CHECK_HIP(hipGetDevice(&dev));
  RXMET_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_dev[dev] == nullptr) {
    void *p = nullptr;
    RXMET_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    RXMET_CHECK_ARG(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return 0;
}

}  // namespace qdq
}  // namespace rxmet

extern "C" {

int64_t rxmet_qdq_workspace_bytes(int64_t outer, int64_t C, int64_t inner) {
  if (outer < 0 || C < 1 || inner < 0) return 0;
  const Plan p = make_plan(outer, C, inner);
  return p.partial_slots * static_cast<int64_t>(sizeof(double2));
}

int rxmet_qdq_minmax(const float *x, int64_t outer, int64_t C, int64_t inner, float *out_min,
                     float *out_max, void *workspace, void *stream_) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  RXMET_CHECK_ARG(out_min && out_max, "out_min/out_max must be non-null");
  const Plan p = make_plan(outer, C, inner);
  RXMET_CHECK_ARG(p.outer * p.C * p.inner > 0, "min/max of an empty tensor");
  RXMET_CHECK_ARG(workspace != nullptr, "min/max needs a workspace");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  float2 *ws = static_cast<float2 *>(workspace);
  rxmet::prof::Scope ps__("qdq_minmax", stream);
  if (!p.cols) {
    const int vec4 = (p.inner % 4 == 0) && aligned16(x);
    hipLaunchKernelGGL(minmax_runs, dim3(static_cast<unsigned>(p.runs * p.splits)), dim3(kThreads),
                       0, stream, x, p.inner, p.splits, vec4, ws);
  } else {
    hipLaunchKernelGGL(minmax_cols, dim3(static_cast<unsigned>(p.col_tiles * p.chunks)),
                       dim3(kThreads), 0, stream, x, p.M, p.K, p.col_tiles, p.rows_per_chunk, ws);
  }
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(fold_minmax, dim3(static_cast<unsigned>(p.C)), dim3(kWave), 0, stream, ws,
                     p.fold, out_min, out_max);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_qdq_forward(const float *x, float *y, int64_t outer, int64_t C, int64_t inner,
                      const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                      int mode, void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  const float lo = static_cast<float>(qmin), hi = static_cast<float>(qmax);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mode == RXMET_QDQ_LEARNABLE)
    return launch_forward<OP_QDQ_LEARN>(x, y, outer, C, inner, scale, offset, lo, hi, s);
  if (mode == RXMET_QDQ_FROZEN)
    return launch_forward<OP_QDQ_FROZEN>(x, y, outer, C, inner, scale, offset, lo, hi, s);
  set_error("unknown qdq mode");
  return -22;
}

int rxmet_qdq_backward(const float *x, const float *g, float *dx, float *dscale, float *doffset,
                       int64_t outer, int64_t C, int64_t inner, const float *scale,
                       const float *offset, int64_t qmin, int64_t qmax, int mode,
                       void *workspace, void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  const float lo = static_cast<float>(qmin), hi = static_cast<float>(qmax);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mode == RXMET_QDQ_LEARNABLE)
    return launch_backward<OP_QDQ_LEARN>(x, g, dx, dscale, doffset, outer, C, inner, scale,
                                         offset, lo, hi, workspace, s);
  if (mode == RXMET_QDQ_FROZEN) {
    RXMET_CHECK_ARG(dscale == nullptr && doffset == nullptr,
                    "frozen encodings have no encoding gradients");
    return launch_backward<OP_QDQ_FROZEN>(x, g, dx, nullptr, nullptr, outer, C, inner, scale,
                                          offset, lo, hi, workspace, s);
  }
  set_error("unknown qdq mode");
  return -22;
}

int rxmet_qdq_backward_noalloc(const float *x, const float *g, float *dx, float *dscale,
                               float *doffset, int64_t outer, int64_t C, int64_t inner,
                               const float *scale, const float *offset, int64_t qmin,
                               int64_t qmax, int mode, void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  RXMET_CHECK_ARG(mode == RXMET_QDQ_LEARNABLE || mode == RXMET_QDQ_FROZEN, "unknown qdq mode");
  void *ws = nullptr;
  if ((dscale != nullptr || doffset != nullptr) && outer * inner > 0) {
    const int64_t need = rxmet_qdq_workspace_bytes(outer, C, inner);
    if (need > kNoAllocScratchBytes) {
      set_error("rxmet_qdq_backward_noalloc: the encoding-gradient partials of this layout need " +
                std::to_string(need) + " bytes, more than the " +
                std::to_string(kNoAllocScratchBytes) +
                "-byte scratch; call rxmet_qdq_backward with a workspace instead");
      return -22;
    }
    if (int rc = scratch_address(&ws)) return rc;
  }
  return rxmet_qdq_backward(x, g, dx, dscale, doffset, outer, C, inner, scale, offset, qmin, qmax,
                            mode, ws, stream);
}

int rxmet_quantize_forward(const float *x, float *q, int64_t outer, int64_t C, int64_t inner,
                           const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                           void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  return launch_forward<OP_Q>(x, q, outer, C, inner, scale, offset, static_cast<float>(qmin),
                              static_cast<float>(qmax), static_cast<hipStream_t>(stream));
}

int rxmet_quantize_backward(const float *x, const float *g, float *dx, float *dscale,
                            float *doffset, int64_t outer, int64_t C, int64_t inner,
                            const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                            void *workspace, void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  return launch_backward<OP_Q>(x, g, dx, dscale, doffset, outer, C, inner, scale, offset,
                               static_cast<float>(qmin), static_cast<float>(qmax), workspace,
                               static_cast<hipStream_t>(stream));
}

int rxmet_dequantize_forward(const float *q, float *y, int64_t outer, int64_t C, int64_t inner,
                             const float *scale, const float *offset, void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  return launch_forward<OP_DQ>(q, y, outer, C, inner, scale, offset, 0.f, 0.f,
                               static_cast<hipStream_t>(stream));
}

int rxmet_dequantize_backward(const float *q, const float *g, float *dq, float *dscale,
                              float *doffset, int64_t outer, int64_t C, int64_t inner,
                              const float *scale, const float *offset, void *workspace,
                              void *stream) {
  clear_error();
  if (int rc = check_layout(outer, C, inner)) return rc;
  RXMET_CHECK_ARG(scale != nullptr, "scale must be non-null");
  return launch_backward<OP_DQ>(q, g, dq, dscale, doffset, outer, C, inner, scale, offset, 0.f,
                                0.f, workspace, static_cast<hipStream_t>(stream));
}

int rxmet_qdq_encoding_forward(const float *mn, const float *mx, int64_t n, int64_t qmin,
                               int64_t qmax, int32_t symmetric, float sym_offset,
                               float min_scale, float *scale, float *offset, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(n >= 1 && mn && mx && scale && offset, "bad encoding arguments");
  if (int rc = check_grid(qmin, qmax)) return rc;
  hipLaunchKernelGGL(encoding_fwd, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n, mn, mx,
                     1.0f / static_cast<float>(qmax - qmin), static_cast<float>(qmin),
                     static_cast<float>(qmax), symmetric, sym_offset,
                     min_scale, scale, offset);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_qdq_encoding_backward(const float *mn, const float *mx, const float *g_scale,
                                const float *g_offset, int64_t n, int64_t qmin, int64_t qmax,
                                int32_t symmetric, float min_scale, float *d_min, float *d_max,
                                void *stream) {
  clear_error();
  RXMET_CHECK_ARG(n >= 1 && mn && mx && d_min && d_max, "bad encoding arguments");
  if (int rc = check_grid(qmin, qmax)) return rc;
  hipLaunchKernelGGL(encoding_bwd, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n, mn, mx, g_scale, g_offset,
                     1.0f / static_cast<float>(qmax - qmin), static_cast<float>(qmin),
                     static_cast<float>(qmax), symmetric, min_scale, d_min, d_max);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
