// qdq.hip — C ABI of the MI355X (gfx950) fake-quantization kernels (rxmet_qdq.h).
//
// The AIMET reference runs QuantizeDequantize as a chain of PyTorch elementwise ops
// (src/aimet_torch/v2/quantization/affine/backends/torch_builtins.py:618-691): about seven
// full HBM passes forward and ten backward plus broadcast reductions.  Here each
// direction is one pass:
//   forward  : read x, write y                                   (2 * sizeof(T) B/element)
//   backward : read x and g, write dx, reduce encoding gradients (3 * sizeof(T) B/element)
//   min/max  : read x                                            (sizeof(T) B/element)
// The kernels and their work decompositions are in qdq_kernels.h, instantiated per
// tensor type in qdq_f32.hip / qdq_f16.hip / qdq_bf16.hip.  This file plans a call
// (layout normalization, decomposition, partial-sum layout), checks its arguments, and
// folds the per-block partial sums of the encoding gradients and min/max.
#include <mutex>
#include <string>

#include "qdq_kernels.h"

namespace rxmet {
namespace qdq {

// ---------------------------------------------------------------------------------
// Partial folding.  The partials of encoding c are at base(c) + l0 * s0 + l1 * s1 + l2 * s2
// for p = (l0 * n1 + l1) * n2 + l2 < n0 * n1 * n2.  Each thread folds a fixed, strided
// subset of p (kFoldUnroll loads in flight), the lanes are combined by a fixed butterfly and
// the waves in a fixed order, so results do not depend on timing.  Three shapes:
//   many partials per encoding (>= 8192): one 1024-thread workgroup per encoding;
//   (1024 .. 8191): one 256-thread workgroup per encoding;
//   some (64 .. 1023): one wave per encoding;
//   few (< 64, e.g. per-channel runs with one chunk per channel): one thread per encoding,
//   the partials in order.
// A single strided run of partials (n0 = n1 = 1, every runs decomposition with one
// encoding group) is indexed without divisions.
// ---------------------------------------------------------------------------------
constexpr int kFoldUnroll = 8;

__device__ __forceinline__ int64_t fold_base(const FoldMap &f, int64_t c) {
  return (c / f.C1) * f.sc0 + (c % f.C1) * f.sc1;
}

__device__ __forceinline__ int64_t fold_offset(const FoldMap &f, int64_t p) {
  if (f.n0 * f.n1 == 1) return p * f.s2;
  const int64_t l2 = p % f.n2, t = p / f.n2;
  const int64_t l1 = t % f.n1, l0 = t / f.n1;
  return l0 * f.s0 + l1 * f.s1 + l2 * f.s2;
}

// Thread-strided fold of encoding c's partials from position `first` in steps of `step`.
template <typename Acc, typename Add>
__device__ __forceinline__ Acc fold_strided(const Acc *__restrict__ partial, const FoldMap &f,
                                            int64_t c, int64_t first, int64_t step, Acc a,
                                            Add add) {
  const int64_t n = f.n0 * f.n1 * f.n2, base = fold_base(f, c);
  for (int64_t p0 = first; p0 < n; p0 += kFoldUnroll * step) {
    Acc v[kFoldUnroll];
#pragma unroll
    for (int k = 0; k < kFoldUnroll; ++k) {
      const int64_t p = p0 + k * step;
      if (p < n) v[k] = partial[base + fold_offset(f, p)];
    }
#pragma unroll
    for (int k = 0; k < kFoldUnroll; ++k)
      if (p0 + k * step < n) add(a, v[k]);
  }
  return a;
}

// Folded min / max written out.
struct PutMinMax {
  float *out_min, *out_max;
  __device__ void operator()(const MinMax &v, int64_t c) const {
    out_min[c] = v.mn;
    out_max[c] = v.mx;
  }
};

// Folded min / max of one statistics update taken into a TF-scheme quantizer's running
// statistics (std::min / std::max with the previous ones, or in their place after a reset),
// and optionally its TfEncodings derived from them in the same thread.
struct PutStats {
  StatsSink k;
  __device__ void operator()(const MinMax &v, int64_t c) const {
    float mn = v.mn, mx = v.mx;
    if (!k.reset) {
      const float a = k.st_min[c], u = k.st_max[c];
      mn = mn < a ? mn : a;
      mx = u < mx ? mx : u;
    }
    k.st_min[c] = mn;
    k.st_max[c] = mx;
    if (k.enc) tf_encoding(mn, mx, k.bw, k.sym, k.strict, k.unsigned_sym, k.enc64, k.enc32, c);
  }
};

struct AddSum {
  __device__ void operator()(Sum2 &a, const Sum2 &v) const { acc_add(a, v); }
};
struct AddMinMax {
  __device__ void operator()(MinMax &a, const MinMax &v) const { acc_add(a, v); }
};

// NT threads per encoding (a wave or a workgroup).
template <int NT, typename Acc, typename Add, typename Put>
__device__ __forceinline__ void fold_block(const Acc *__restrict__ partial, const FoldMap &f,
                                           Acc zero, Add add, Put put) {
  __shared__ Acc red[NT / kWave];
  const int64_t c = blockIdx.x;
  Acc a = fold_strided(partial, f, c, threadIdx.x, NT, zero, add);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) add(a, acc_shfl(a, off));
  if (NT > kWave) {
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = a;
    __syncthreads();
    if (threadIdx.x == 0)
      for (int w = 1; w < NT / kWave; ++w) add(a, red[w]);
  }
  if (threadIdx.x == 0) put(a, c);
}

template <int NT, typename Put>
__global__ __launch_bounds__(NT) void fold_sum(const Sum2 *__restrict__ partial, FoldMap f,
                                               Put put) {
  fold_block<NT>(partial, f, Sum2{0.0, 0.0}, AddSum{}, put);
}

template <int NT, typename Put>
__global__ __launch_bounds__(NT) void fold_minmax(const MinMax *__restrict__ partial, FoldMap f,
                                                  Put put) {
  fold_block<NT>(partial, f, MinMax{INFINITY, -INFINITY}, AddMinMax{}, put);
}

// One thread per encoding, its partials in order.
template <typename Put>
__global__ __launch_bounds__(256) void fold_sum_thread(const Sum2 *__restrict__ partial,
                                                       FoldMap f, int64_t C, Put put) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= C) return;
  put(fold_strided(partial, f, c, 0, 1, Sum2{0.0, 0.0}, AddSum{}), c);
}

template <typename Put>
__global__ __launch_bounds__(256) void fold_minmax_thread(const MinMax *__restrict__ partial,
                                                          FoldMap f, int64_t C, Put put) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= C) return;
  put(fold_strided(partial, f, c, 0, 1, MinMax{INFINITY, -INFINITY}, AddMinMax{}), c);
}

// Launch the fold of C encodings' partials with the shape their count calls for.
template <typename Put>
static void launch_fold_sum(const Sum2 *ws, const FoldMap &f, int64_t C, Put put,
                            hipStream_t s) {
  const int64_t n = f.n0 * f.n1 * f.n2;
  if (n >= 8192)
    hipLaunchKernelGGL((fold_sum<16 * kWave, Put>), dim3(static_cast<unsigned>(C)),
                       dim3(16 * kWave), 0, s, ws, f, put);
  else if (n >= 1024)
    hipLaunchKernelGGL((fold_sum<4 * kWave, Put>), dim3(static_cast<unsigned>(C)),
                       dim3(4 * kWave), 0, s, ws, f, put);
  else if (n >= 64)
    hipLaunchKernelGGL((fold_sum<kWave, Put>), dim3(static_cast<unsigned>(C)), dim3(kWave), 0, s,
                       ws, f, put);
  else
    hipLaunchKernelGGL((fold_sum_thread<Put>), dim3(static_cast<unsigned>((C + 255) / 256)),
                       dim3(256), 0, s, ws, f, C, put);
}

template <typename Put>
static void launch_fold_minmax(const MinMax *ws, const FoldMap &f, int64_t C, Put put,
                               hipStream_t s) {
  const int64_t n = f.n0 * f.n1 * f.n2;
  if (n >= 8192)
    hipLaunchKernelGGL((fold_minmax<16 * kWave, Put>), dim3(static_cast<unsigned>(C)),
                       dim3(16 * kWave), 0, s, ws, f, put);
  else if (n >= 1024)
    hipLaunchKernelGGL((fold_minmax<4 * kWave, Put>), dim3(static_cast<unsigned>(C)),
                       dim3(4 * kWave), 0, s, ws, f, put);
  else if (n >= 64)
    hipLaunchKernelGGL((fold_minmax<kWave, Put>), dim3(static_cast<unsigned>(C)), dim3(kWave), 0,
                       s, ws, f, put);
  else
    hipLaunchKernelGGL((fold_minmax_thread<Put>), dim3(static_cast<unsigned>((C + 255) / 256)),
                       dim3(256), 0, s, ws, f, C, put);
}

__global__ __launch_bounds__(256) void zero_enc_grads(int64_t C, float *dscale, float *doffset) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= C) return;
  if (dscale) dscale[i] = 0.0f;
  if (doffset) doffset[i] = 0.0f;
}

// ---------------------------------------------------------------------------------
// Planning.
// ---------------------------------------------------------------------------------

// Normalize a [outer, C0, mid, C1, inner] layout (one encoding group -> C0 = outer = 1;
// one encoding -> a single run) and choose the decomposition.
static Plan make_plan(int64_t outer, int64_t C0, int64_t mid, int64_t C1, int64_t inner,
                      int esize, int vec) {
  Plan p;
  p.esize = esize;
  if (C0 == 1) {
    mid *= outer;
    outer = 1;
  } else if (mid == 1) {  // adjacent groups
    mid = outer;
    outer = 1;
    C1 *= C0;
    C0 = 1;
  } else if (C1 == 1) {
    inner *= mid;
    mid = outer;
    outer = 1;
    C1 = C0;
    C0 = 1;
  }
  if (C0 == 1 && C1 == 1) {  // one encoding: one run
    inner *= mid;
    mid = 1;
  }
  p.outer = outer;
  p.C0 = C0;
  p.mid = mid;
  p.C1 = C1;
  p.inner = inner;
  p.n = outer * C0 * mid * C1 * inner;
  p.runs = outer * C0 * mid * C1;
  p.geo = Geo{inner, C1, mid * C1, C0};
  const int64_t chunk = int64_t(kThreads) * vec * (16 / esize);
  if ((C0 == 1 && C1 == 1) || inner >= kMinRun) {
    p.kind = KIND_RUNS;
    // many encodings of one run each, runs of a few chunks: whole runs per workgroup; one
    // long run (the forward / backward passes): two chunks per workgroup
    const int64_t nchunks = inner > 0 ? (inner + chunk - 1) / chunk : 1;
    if (outer * mid == 1 && p.runs >= kWholeRunMinRuns && nchunks > 1 &&
        nchunks <= kWholeRunChunks)
      p.passes = static_cast<int>(nchunks);
    else if (p.runs == 1 && vec == kVecQdq && nchunks >= kSingleRunMinChunks)
      p.passes = kSingleRunPasses;
    p.splits = (nchunks + p.passes - 1) / p.passes;
    p.partial_slots = p.runs * p.splits;
    p.direct = p.splits == 1 && outer * mid == 1;
    p.fold = FoldMap{outer, mid, p.splits, C0 * mid * C1 * p.splits, C1 * p.splits, 1,
                     C1, mid * C1 * p.splits, p.splits};
  } else if (inner >= kMinSeg) {
    p.kind = KIND_SEGS;
    p.splits = 1;
    p.partial_slots = p.runs;
    p.fold = FoldMap{outer, mid, 1, C0 * mid * C1, C1, 0, C1, mid * C1, 1};
  } else {
    p.kind = KIND_COLS;
    const int64_t K = C1 * inner;
    int kt_shift = 0;
    while (kt_shift < 8 && (int64_t(1) << kt_shift) < K) ++kt_shift;
    const int64_t kt = int64_t(1) << kt_shift, rows_par = kThreads / kt;
    const int64_t col_tiles = (K + kt - 1) / kt;
    const int64_t bands = outer * C0;
    int64_t chunks = kColTargetBlocks / (bands * col_tiles > 0 ? bands * col_tiles : 1);
    const int64_t max_chunks = (mid + rows_par - 1) / rows_par;
    chunks = chunks < 1 ? 1 : (chunks > max_chunks ? max_chunks : chunks);
    if (chunks < 1) chunks = 1;
    const int64_t rpc = mid > 0 ? (mid + chunks - 1) / chunks : 1;
    chunks = mid > 0 ? (mid + rpc - 1) / rpc : 1;
    p.cg = ColGeo{mid, K, inner, C1, C0, col_tiles, chunks, rpc, kt_shift};
    p.col_blocks = bands * chunks * col_tiles;
    p.partial_slots = bands * chunks * K;
    p.fold = FoldMap{outer, chunks, inner, C0 * chunks * K, K, 1, C1, chunks * K, inner};
  }
  return p;
}

static int check_layout(int64_t outer, int64_t C0, int64_t mid, int64_t C1, int64_t inner) {
  RXMET_CHECK_ARG(outer >= 0 && mid >= 0 && inner >= 0 && C0 >= 1 && C1 >= 1,
                  "invalid layout: need outer, mid, inner >= 0 and C0, C1 >= 1");
  const int64_t lim = int64_t(1) << 40;
  int64_t n = 1;
  for (int64_t d : {outer, C0, mid, C1, inner}) {
    if (d == 0) return 0;
    RXMET_CHECK_ARG(n <= lim / d, "tensor too large");
    n *= d;
  }
  return 0;
}

static int esize_of(int32_t io) {
  return io == RXMET_QDQ_F64 ? 8 : io == RXMET_QDQ_F32 ? 4 : 2;
}

static int mantissa_bits(int32_t t) {
  return t == RXMET_QDQ_F64 ? 53 : t == RXMET_QDQ_F32 ? 24 : t == RXMET_QDQ_F16 ? 11 : 8;
}

// The grid's end points are exact integers of the type the arithmetic runs in.
static int check_grid(int64_t qmin, int64_t qmax, int32_t type) {
  RXMET_CHECK_ARG(qmin <= qmax, "qmin must be <= qmax");
  const int64_t lim = int64_t(1) << mantissa_bits(type);
  RXMET_CHECK_ARG(qmin >= -lim && qmax <= lim,
                  "grid not exactly representable in the arithmetic type (|q| > 2^" +
                      std::to_string(mantissa_bits(type)) + ")");
  return 0;
}

static bool is_io(int32_t t) {
  return t == RXMET_QDQ_F32 || t == RXMET_QDQ_F16 || t == RXMET_QDQ_BF16 || t == RXMET_QDQ_F64;
}

// Which internal type an op computes in under these numerics.
static int32_t arithmetic_type(int op, const rxmet_qdq_numerics &nm) {
  if (op == OP_QDQ_FROZEN) return RXMET_QDQ_F32;
  if (op == OP_DQ) return nm.io_dtype;
  return nm.internal_dtype;
}

static int check_numerics(int op, const rxmet_qdq_numerics &nm) {
  RXMET_CHECK_ARG(is_io(nm.io_dtype), "io_dtype must be RXMET_QDQ_F32, F16, BF16 or F64");
  const int32_t r = nm.internal_dtype;
  RXMET_CHECK_ARG(r == nm.io_dtype || r == RXMET_QDQ_F32 || r == RXMET_QDQ_F64,
                  "internal_dtype must be io_dtype, RXMET_QDQ_F32 or RXMET_QDQ_F64");
  RXMET_CHECK_ARG(nm.reserved == 0, "rxmet_qdq_numerics.reserved must be 0");
  RXMET_CHECK_ARG(nm.zero_point_shift == nm.zero_point_shift &&
                      nm.zero_point_shift > -1e30 && nm.zero_point_shift < 1e30,
                  "zero_point_shift must be finite");
  if (op != OP_QDQ_LEARN)
    RXMET_CHECK_ARG(nm.zero_point_shift == 0.0,
                    "zero_point_shift applies to learnable-mode quantize_dequantize only");
  if (op == OP_DQ)
    RXMET_CHECK_ARG(r == nm.io_dtype, "dequantize computes in the tensor's own type");
  return 0;
}

static Params make_params(int64_t qmin, int64_t qmax, const rxmet_qdq_numerics &nm) {
  return Params{static_cast<double>(qmin), static_cast<double>(qmax), nm.zero_point_shift,
                nm.scalar_scale ? 1 : 0};
}

static int dispatch(const Call &c, int32_t io, int what) {
  int rc = -22;
  if (io == RXMET_QDQ_F32) rc = run_f32(c, what);
  else if (io == RXMET_QDQ_F16) rc = run_f16(c, what);
  else if (io == RXMET_QDQ_BF16) rc = run_bf16(c, what);
  else if (io == RXMET_QDQ_F64) rc = run_f64(c, what);
  if (rc != 0) {
    set_error("qdq: no kernel for this op / io type / internal type combination");
    return rc;
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}

static int forward_impl(int op, const void *x, void *y, const rxmet_qdq_layout *l,
                        const rxmet_qdq_numerics *nm, const float *scale, const float *offset,
                        int64_t qmin, int64_t qmax, void *stream,
                        const MinMaxSrc *mm = nullptr) {
  RXMET_CHECK_ARG(l != nullptr && nm != nullptr, "layout and numerics must be non-null");
  if (int rc = check_layout(l->outer, l->C0, l->mid, l->C1, l->inner)) return rc;
  if (int rc = check_numerics(op, *nm)) return rc;
  if (op != OP_DQ)
    if (int rc = check_grid(qmin, qmax, arithmetic_type(op, *nm))) return rc;
  RXMET_CHECK_ARG(scale != nullptr || mm != nullptr, "scale must be non-null");
  const Plan p =
      make_plan(l->outer, l->C0, l->mid, l->C1, l->inner, esize_of(nm->io_dtype), kVecQdq);
  if (p.n == 0) return 0;
  RXMET_CHECK_ARG(x != nullptr && y != nullptr, "input/output must be non-null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Call c{&p, op, nm->internal_dtype, x, nullptr, y, scale, offset,
               make_params(qmin, qmax, *nm), nullptr, s, mm ? *mm : MinMaxSrc{}};
  rxmet::prof::Scope ps__("qdq_forward_stream", s);
  return dispatch(c, nm->io_dtype, WHAT_FORWARD);
}

// With mm (encodings derived from min / max in the kernels), d_min / d_max receive the
// gradients of min and max instead of dscale / doffset receiving those of scale and offset.
static int backward_impl(int op, const void *x, const void *g, void *dx, float *dscale,
                         float *doffset, const rxmet_qdq_layout *l, const rxmet_qdq_numerics *nm,
                         const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                         void *workspace, void *stream, const MinMaxSrc *mm = nullptr,
                         float *d_min = nullptr, float *d_max = nullptr) {
  RXMET_CHECK_ARG(l != nullptr && nm != nullptr, "layout and numerics must be non-null");
  if (int rc = check_layout(l->outer, l->C0, l->mid, l->C1, l->inner)) return rc;
  if (int rc = check_numerics(op, *nm)) return rc;
  if (op != OP_DQ)
    if (int rc = check_grid(qmin, qmax, arithmetic_type(op, *nm))) return rc;
  RXMET_CHECK_ARG(scale != nullptr || mm != nullptr, "scale must be non-null");
  if (op == OP_QDQ_FROZEN)
    RXMET_CHECK_ARG(dscale == nullptr && doffset == nullptr,
                    "frozen encodings have no encoding gradients");
  if (mm != nullptr)
    RXMET_CHECK_ARG(dscale == nullptr && doffset == nullptr && (d_min == nullptr) == (d_max == nullptr),
                    "min/max encodings give d_min and d_max together");
  const Plan p =
      make_plan(l->outer, l->C0, l->mid, l->C1, l->inner, esize_of(nm->io_dtype), kVecQdq);
  const bool enc = dscale != nullptr || doffset != nullptr || d_min != nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t C = l->C0 * l->C1;
  if (p.n == 0) {
    // zeroed by a kernel, not a memset node, so a captured training step replays correctly
    if (enc) {
      hipLaunchKernelGGL(zero_enc_grads, dim3(static_cast<unsigned>((C + 255) / 256)), dim3(256),
                         0, s, C, d_min ? d_min : dscale, d_min ? d_max : doffset);
      RXMET_CHECK_LAUNCH();
    }
    return 0;
  }
  RXMET_CHECK_ARG(x != nullptr && g != nullptr && dx != nullptr, "x, g and dx must be non-null");
  if (enc) RXMET_CHECK_ARG(workspace != nullptr, "encoding gradients need a workspace");
  Call c{&p, op, nm->internal_dtype, x, g, dx, scale, offset,
         make_params(qmin, qmax, *nm), enc ? workspace : nullptr, s,
         mm ? *mm : MinMaxSrc{}};
  const int32_t r = arithmetic_type(op, *nm);
  const int round16 = r == RXMET_QDQ_F16 ? 1 : (r == RXMET_QDQ_BF16 ? 2 : 0);
  if (enc && p.kind == KIND_RUNS && p.direct) {
    c.ff.direct = 1;
    c.ff.use_mm = mm != nullptr;
    c.ff.so = PutScaleOffset{dscale, doffset, round16};
    if (mm != nullptr) c.ff.mg = PutMinMaxGrad{*mm, d_min, d_max, round16};
  }
  {
    rxmet::prof::Scope ps__("qdq_backward_stream", s);
    if (int rc = dispatch(c, nm->io_dtype, WHAT_BACKWARD)) return rc;
  }
  if (enc && !c.ff.direct) {
    rxmet::prof::Scope ps__("qdq_backward_fold", s);
    const Sum2 *ws = static_cast<const Sum2 *>(workspace);
    if (mm != nullptr)
      launch_fold_sum(ws, p.fold, C, PutMinMaxGrad{*mm, d_min, d_max, round16}, s);
    else
      launch_fold_sum(ws, p.fold, C, PutScaleOffset{dscale, doffset, round16}, s);
    RXMET_CHECK_LAUNCH();
  }
  return 0;
}

// Min / max of every encoding's elements; `put` receives each folded pair.
template <typename Put>
static int minmax_impl(const void *x, int32_t io, const rxmet_qdq_layout *l, Put put,
                       void *workspace, void *stream, bool skip_nan = false) {
  RXMET_CHECK_ARG(l != nullptr, "layout must be non-null");
  if (int rc = check_layout(l->outer, l->C0, l->mid, l->C1, l->inner)) return rc;
  RXMET_CHECK_ARG(is_io(io), "io_dtype must be RXMET_QDQ_F32, F16, BF16 or F64");
  const Plan p = make_plan(l->outer, l->C0, l->mid, l->C1, l->inner, esize_of(io), kVecMinMax);
  RXMET_CHECK_ARG(p.n > 0, "min/max of an empty tensor");
  RXMET_CHECK_ARG(x != nullptr, "x must be non-null");
  RXMET_CHECK_ARG(workspace != nullptr, "min/max needs a workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  rxmet::prof::Scope ps__("qdq_minmax", s);
  rxmet_qdq_numerics nm{io, io, 0.0, 0, 0};
  const Call c{&p, OP_QDQ_LEARN, nm.internal_dtype, x, nullptr, nullptr, nullptr, nullptr,
               make_params(0, 0, nm), workspace, s};
  if (int rc = dispatch(c, io, skip_nan ? WHAT_MINMAX_SKIP_NAN : WHAT_MINMAX)) return rc;
  launch_fold_minmax(static_cast<const MinMax *>(workspace), p.fold, l->C0 * l->C1, put, s);
  RXMET_CHECK_LAUNCH();
  return 0;
}

// Shared with the ONNX Runtime op core (qc_quantize.hip).
int minmax_stats(const void *x, int32_t io, const rxmet_qdq_layout &l, const StatsSink &sink,
                 void *workspace, hipStream_t s) {
  RXMET_CHECK_ARG(sink.st_min && sink.st_max, "statistics must be non-null");
  RXMET_CHECK_ARG(!sink.enc || (sink.enc64 && sink.enc32), "encodings must be non-null");
  return minmax_impl(x, io, &l, PutStats{sink}, workspace, s, true);
}

int forward_tf(int op, const void *x, void *y, int32_t io, const rxmet_qdq_layout &l,
               const TfEnc32 *enc, hipStream_t s) {
  RXMET_CHECK_ARG(op == OP_NATIVE || op == OP_FP16, "forward_tf: OP_NATIVE or OP_FP16");
  RXMET_CHECK_ARG(io == RXMET_QDQ_F32 || io == RXMET_QDQ_F16, "io_dtype must be F32 or F16");
  if (int rc = check_layout(l.outer, l.C0, l.mid, l.C1, l.inner)) return rc;
  RXMET_CHECK_ARG(op == OP_FP16 || enc != nullptr, "encodings must be non-null");
  const Plan p = make_plan(l.outer, l.C0, l.mid, l.C1, l.inner, esize_of(io), kVecQdq);
  if (p.n == 0) return 0;
  RXMET_CHECK_ARG(x != nullptr && y != nullptr, "input/output must be non-null");
  const rxmet_qdq_numerics nm{io, RXMET_QDQ_F32, 0.0, 0, 0};
  const Call c{&p, op, RXMET_QDQ_F32, x, nullptr, y, reinterpret_cast<const float *>(enc),
               nullptr, make_params(0, 0, nm), nullptr, s, MinMaxSrc{}};
  rxmet::prof::Scope ps__(op == OP_NATIVE ? "qc_qdq_native" : "qc_qdq_fp16", s);
  return dispatch(c, io, WHAT_FORWARD);
}

// The three-argument fp32 layout [outer, C, inner] of the original entry points.
static rxmet_qdq_layout layout3(int64_t outer, int64_t C, int64_t inner) {
  return rxmet_qdq_layout{1, 1, outer, C, inner};
}
static const rxmet_qdq_numerics kF32{RXMET_QDQ_F32, RXMET_QDQ_F32, 0.0, 0, 0};

static int check_layout3(int64_t outer, int64_t C, int64_t inner) {
  RXMET_CHECK_ARG(outer >= 0 && C >= 1 && inner >= 0,
                  "invalid layout: need outer>=0, C>=1, inner>=0");
  return check_layout(1, 1, outer, C, inner);
}

// Encodings of learnable min / max, one thread per encoding (see rxmet_qdq_encoding_forward).
__global__ __launch_bounds__(256) void encoding_fwd(int64_t n, MinMaxSrc m,
                                                    float *__restrict__ scale,
                                                    float *__restrict__ offset) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  float s, o;
  minmax_scale_offset(m, c, s, o);
  scale[c] = s;
  offset[c] = o;
}

__global__ __launch_bounds__(256) void encoding_bwd(int64_t n, MinMaxSrc m,
                                                    const float *__restrict__ g_scale,
                                                    const float *__restrict__ g_offset,
                                                    float *__restrict__ d_min,
                                                    float *__restrict__ d_max) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  minmax_encoding_grad(m, c, g_scale ? g_scale[c] : 0.0f, g_offset ? g_offset + c : nullptr,
                       d_min[c], d_max[c]);
}

static MinMaxSrc minmax_src(const float *mn, const float *mx, int64_t qmin, int64_t qmax,
                            int32_t symmetric, float sym_offset, float min_scale) {
  return MinMaxSrc{mn, mx, 1.0f / static_cast<float>(qmax - qmin), static_cast<float>(qmin),
                   static_cast<float>(qmax), sym_offset, min_scale, symmetric ? 1 : 0};
}

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

using namespace rxmet;
using namespace rxmet::qdq;

extern "C" {

int64_t rxmet_qdq_workspace_bytes(int64_t outer, int64_t C, int64_t inner) {
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return rxmet_qdq_workspace_bytes_ex(&l, RXMET_QDQ_F32);
}

int64_t rxmet_qdq_workspace_bytes_ex(const rxmet_qdq_layout *l, int32_t io_dtype) {
  if (l == nullptr || !is_io(io_dtype) || l->outer < 0 || l->mid < 0 || l->inner < 0 ||
      l->C0 < 1 || l->C1 < 1)
    return 0;
  // the forward / backward plan has at least as many partials as the min / max plan (its
  // chunks are half as long; it takes two per workgroup only where min / max takes one)
  const Plan p = make_plan(l->outer, l->C0, l->mid, l->C1, l->inner, esize_of(io_dtype), kVecQdq);
  return p.partial_slots * static_cast<int64_t>(sizeof(Sum2));
}

int rxmet_qdq_minmax(const float *x, int64_t outer, int64_t C, int64_t inner, float *out_min,
                     float *out_max, void *workspace, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  RXMET_CHECK_ARG(out_min && out_max, "out_min/out_max must be non-null");
  return minmax_impl(x, RXMET_QDQ_F32, &l, PutMinMax{out_min, out_max}, workspace, stream);
}

int rxmet_qdq_minmax_ex(const void *x, int32_t io_dtype, const rxmet_qdq_layout *layout,
                        float *out_min, float *out_max, void *workspace, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(out_min && out_max, "out_min/out_max must be non-null");
  return minmax_impl(x, io_dtype, layout, PutMinMax{out_min, out_max}, workspace, stream);
}

static int qdq_op(int mode) {
  return mode == RXMET_QDQ_LEARNABLE ? OP_QDQ_LEARN : (mode == RXMET_QDQ_FROZEN ? OP_QDQ_FROZEN : -1);
}

int rxmet_qdq_forward(const float *x, float *y, int64_t outer, int64_t C, int64_t inner,
                      const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                      int mode, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return rxmet_qdq_forward_ex(x, y, &l, &kF32, scale, offset, qmin, qmax, mode, stream);
}

int rxmet_qdq_forward_ex(const void *x, void *y, const rxmet_qdq_layout *layout,
                         const rxmet_qdq_numerics *numerics, const float *scale,
                         const float *offset, int64_t qmin, int64_t qmax, int mode,
                         void *stream) {
  clear_error();
  const int op = qdq_op(mode);
  RXMET_CHECK_ARG(op >= 0, "unknown qdq mode");
  return forward_impl(op, x, y, layout, numerics, scale, offset, qmin, qmax, stream);
}

int rxmet_qdq_backward(const float *x, const float *g, float *dx, float *dscale, float *doffset,
                       int64_t outer, int64_t C, int64_t inner, const float *scale,
                       const float *offset, int64_t qmin, int64_t qmax, int mode,
                       void *workspace, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return rxmet_qdq_backward_ex(x, g, dx, dscale, doffset, &l, &kF32, scale, offset, qmin, qmax,
                               mode, workspace, stream);
}

int rxmet_qdq_backward_ex(const void *x, const void *g, void *dx, float *dscale, float *doffset,
                          const rxmet_qdq_layout *layout, const rxmet_qdq_numerics *numerics,
                          const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                          int mode, void *workspace, void *stream) {
  clear_error();
  const int op = qdq_op(mode);
  RXMET_CHECK_ARG(op >= 0, "unknown qdq mode");
  return backward_impl(op, x, g, dx, dscale, doffset, layout, numerics, scale, offset, qmin,
                       qmax, workspace, stream);
}

static int minmax_args(const rxmet_qdq_minmax_enc *enc, int64_t qmin, int64_t qmax, MinMaxSrc *mm) {
  RXMET_CHECK_ARG(enc != nullptr && enc->min != nullptr && enc->max != nullptr,
                  "min/max encodings must be non-null");
  RXMET_CHECK_ARG(enc->reserved == 0, "rxmet_qdq_minmax_enc.reserved must be 0");
  if (int rc = check_grid(qmin, qmax, RXMET_QDQ_F32)) return rc;
  RXMET_CHECK_ARG(qmax > qmin, "min/max encodings need qmax > qmin");
  *mm = minmax_src(enc->min, enc->max, qmin, qmax, enc->symmetric, enc->sym_offset,
                   enc->min_scale);
  return 0;
}

int rxmet_qdq_forward_minmax(const void *x, void *y, const rxmet_qdq_layout *layout,
                             const rxmet_qdq_numerics *numerics, const rxmet_qdq_minmax_enc *enc,
                             int64_t qmin, int64_t qmax, void *stream) {
  clear_error();
  MinMaxSrc mm;
  if (int rc = minmax_args(enc, qmin, qmax, &mm)) return rc;
  return forward_impl(OP_QDQ_LEARN, x, y, layout, numerics, nullptr, nullptr, qmin, qmax, stream,
                      &mm);
}

int rxmet_qdq_backward_minmax(const void *x, const void *g, void *dx, float *d_min,
                              float *d_max, const rxmet_qdq_layout *layout,
                              const rxmet_qdq_numerics *numerics, const rxmet_qdq_minmax_enc *enc,
                              int64_t qmin, int64_t qmax, void *workspace, void *stream) {
  clear_error();
  MinMaxSrc mm;
  if (int rc = minmax_args(enc, qmin, qmax, &mm)) return rc;
  return backward_impl(OP_QDQ_LEARN, x, g, dx, nullptr, nullptr, layout, numerics, nullptr,
                       nullptr, qmin, qmax, workspace, stream, &mm, d_min, d_max);
}

int rxmet_qdq_backward_noalloc(const float *x, const float *g, float *dx, float *dscale,
                               float *doffset, int64_t outer, int64_t C, int64_t inner,
                               const float *scale, const float *offset, int64_t qmin,
                               int64_t qmax, int mode, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  if (int rc = check_grid(qmin, qmax, RXMET_QDQ_F32)) return rc;
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
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return forward_impl(OP_Q, x, q, &l, &kF32, scale, offset, qmin, qmax, stream);
}

int rxmet_quantize_forward_ex(const void *x, void *q, const rxmet_qdq_layout *layout,
                              const rxmet_qdq_numerics *numerics, const float *scale,
                              const float *offset, int64_t qmin, int64_t qmax, void *stream) {
  clear_error();
  return forward_impl(OP_Q, x, q, layout, numerics, scale, offset, qmin, qmax, stream);
}

int rxmet_quantize_backward(const float *x, const float *g, float *dx, float *dscale,
                            float *doffset, int64_t outer, int64_t C, int64_t inner,
                            const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                            void *workspace, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return backward_impl(OP_Q, x, g, dx, dscale, doffset, &l, &kF32, scale, offset, qmin, qmax,
                       workspace, stream);
}

int rxmet_quantize_backward_ex(const void *x, const void *g, void *dx, float *dscale,
                               float *doffset, const rxmet_qdq_layout *layout,
                               const rxmet_qdq_numerics *numerics, const float *scale,
                               const float *offset, int64_t qmin, int64_t qmax,
                               void *workspace, void *stream) {
  clear_error();
  return backward_impl(OP_Q, x, g, dx, dscale, doffset, layout, numerics, scale, offset, qmin,
                       qmax, workspace, stream);
}

int rxmet_dequantize_forward(const float *q, float *y, int64_t outer, int64_t C, int64_t inner,
                             const float *scale, const float *offset, void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return forward_impl(OP_DQ, q, y, &l, &kF32, scale, offset, 0, 0, stream);
}

int rxmet_dequantize_forward_ex(const void *q, void *y, const rxmet_qdq_layout *layout,
                                const rxmet_qdq_numerics *numerics, const float *scale,
                                const float *offset, void *stream) {
  clear_error();
  return forward_impl(OP_DQ, q, y, layout, numerics, scale, offset, 0, 0, stream);
}

int rxmet_dequantize_backward(const float *q, const float *g, float *dq, float *dscale,
                              float *doffset, int64_t outer, int64_t C, int64_t inner,
                              const float *scale, const float *offset, void *workspace,
                              void *stream) {
  clear_error();
  if (int rc = check_layout3(outer, C, inner)) return rc;
  const rxmet_qdq_layout l = layout3(outer, C, inner);
  return backward_impl(OP_DQ, q, g, dq, dscale, doffset, &l, &kF32, scale, offset, 0, 0,
                       workspace, stream);
}

int rxmet_dequantize_backward_ex(const void *q, const void *g, void *dq, float *dscale,
                                 float *doffset, const rxmet_qdq_layout *layout,
                                 const rxmet_qdq_numerics *numerics, const float *scale,
                                 const float *offset, void *workspace, void *stream) {
  clear_error();
  return backward_impl(OP_DQ, q, g, dq, dscale, doffset, layout, numerics, scale, offset, 0, 0,
                       workspace, stream);
}

int rxmet_qdq_encoding_forward(const float *mn, const float *mx, int64_t n, int64_t qmin,
                               int64_t qmax, int32_t symmetric, float sym_offset,
                               float min_scale, float *scale, float *offset, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(n >= 1 && mn && mx && scale && offset, "bad encoding arguments");
  if (int rc = check_grid(qmin, qmax, RXMET_QDQ_F32)) return rc;
  hipLaunchKernelGGL(encoding_fwd, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n,
                     minmax_src(mn, mx, qmin, qmax, symmetric, sym_offset, min_scale), scale,
                     offset);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_qdq_encoding_backward(const float *mn, const float *mx, const float *g_scale,
                                const float *g_offset, int64_t n, int64_t qmin, int64_t qmax,
                                int32_t symmetric, float min_scale, float *d_min, float *d_max,
                                void *stream) {
  clear_error();
  RXMET_CHECK_ARG(n >= 1 && mn && mx && d_min && d_max, "bad encoding arguments");
  if (int rc = check_grid(qmin, qmax, RXMET_QDQ_F32)) return rc;
  hipLaunchKernelGGL(encoding_bwd, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n,
                     minmax_src(mn, mx, qmin, qmax, symmetric, 0.0f, min_scale), g_scale,
                     g_offset, d_min, d_max);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
