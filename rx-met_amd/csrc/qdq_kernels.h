// qdq_kernels.h — streaming fake-quantization kernels (MI355X, gfx950), shared by the
// per-element-type translation units qdq_f32.hip / qdq_f16.hip / qdq_bf16.hip.
//
// Element types.  Tensors hold fp32, fp16 or bf16 elements ("io" type T).  The arithmetic
// of the reference runs in an "internal" type R chosen by its numerical-stability rule
// (torch_builtins.py:85-101, 255-262): R = T for small grids, else fp32, else fp64.  Here
// every element is widened to fp32 (fp64 when R is fp64), each operation is evaluated
// there and its result rounded back to R, which is what PyTorch's 16-bit elementwise
// kernels do (fp32 "opmath", one rounding to the storage type per operation; for +, -, *, /
// of fp16/bf16 operands the fp32 result rounded once more is the correctly rounded
// 16-bit result, because fp32 carries more than 2p+2 bits).
//
// Work decompositions of a [outer, C0, mid, C1, inner] tensor whose element
// (o, c0, m, c1, k) uses encoding c0 * C1 + c1 (a "run" is one contiguous stretch of
// `inner` elements sharing an encoding):
//   runs : long runs (>= 1024 elements) or one encoding — each workgroup streams one
//          chunk of one run with 16-byte accesses and one scalar encoding load.
//   segs : medium runs (16..1023 elements, e.g. block quantization) — a power-of-two
//          segment of lanes per run, several runs per workgroup, one partial per run
//          reduced with lane shuffles inside the segment.
//   cols : short runs (< 16 elements, e.g. per-channel on the last axis) — the tensor is
//          outer*C0 bands of a [mid, C1*inner] matrix; threads own columns and walk the
//          rows of one band, several rows in parallel when the matrix is narrow.
// Reductions write one fp64 (or min/max) partial per workgroup, run or column chunk; a
// second kernel folds the partials of each encoding in a fixed order, so results are
// deterministic and need no atomics.  A backward whose workgroups each hold one whole
// encoding (per-channel runs of a few chunks) writes the encoding gradients itself.
#pragma once

#include <stdint.h>

#include <type_traits>

#include "div_rn.h"
#include "rxmet_common.h"
#include "rxmet_qc.h"
#include "rxmet_qdq.h"

namespace rxmet {
namespace qdq {

// OP_NATIVE: the libpymo form stableQuantizeDequantize (quantize_dequantize.hpp:35-46) on a
// TfEncoding, as the ONNX Runtime custom op runs it (trim_functions.cpp:646-668).  OP_FP16:
// the float16 round trip of a float quantizer (AimetOpUtils.cpp:60-66).  Forward only.
enum Op { OP_QDQ_LEARN = 0, OP_QDQ_FROZEN = 1, OP_Q = 2, OP_DQ = 3, OP_NATIVE = 4, OP_FP16 = 5 };

// One TfEncoding as OP_NATIVE reads it: min, max and delta rounded to fp32 (the reference
// casts the double encoding to the tensor type) and the correctly rounded fp32 1 / delta.
struct alignas(16) TfEnc32 {
  float mn, mx, delta, inv_delta;
};

__device__ __forceinline__ double dmin_std(double a, double b) { return b < a ? b : a; }
__device__ __forceinline__ double dmax_std(double a, double b) { return a < b ? b : a; }
__device__ __forceinline__ double dclamp_std(double v, double lo, double hi) {
  return v < lo ? lo : (hi < v ? hi : v);
}

// The TfEncoding of encoding c from its fp32 running statistics:
// MinMaxEncodingAnalyzer<float>::computeEncoding (MinMaxEncodingAnalyzer.cpp:72-96) and
// getComputedEncodings (quantization_utils.cpp:59-119), each step the correctly rounded double
// operation (std::min / max / clamp as their comparisons define them, C round), written as the
// double encoding and its fp32 form.
__device__ __forceinline__ void tf_encoding(float st_min, float st_max, int bw, int sym,
                                            int strict, int unsigned_sym, rxmet_tf_encoding *enc,
                                            TfEnc32 *enc32, int64_t c) {
  // zero inside the range; at least MIN_RANGE (the float 0.01) wide
  double mn = static_cast<double>(st_min < 0.0f ? st_min : 0.0f);
  double mx = static_cast<double>(0.0f < st_max ? st_max : 0.0f);
  mx = dmax_std(mx, mn + static_cast<double>(0.01f));

  double steps = ldexp(1.0, bw) - 1.0;
  if (sym && strict) steps -= 1.0;
  const double f32_lo = static_cast<double>(-3.40282346638528859812e+38f) * 0.99;
  const double f32_hi = static_cast<double>(3.40282346638528859812e+38f) * 0.99;
  mn = dclamp_std(mn, f32_lo, 0.0);
  mx = dclamp_std(mx, 0.0, f32_hi);
  const bool uns = unsigned_sym && mn >= 0.0;
  double delta, offset;
  if (sym && !uns) {
    const unsigned pos = static_cast<unsigned>(floor(steps / 2.0));
    const unsigned neg = static_cast<unsigned>(steps - static_cast<double>(pos));
    const unsigned extra = steps == 3.0 ? 1u : 0u;  // all bins usable at 2 bits
    delta = dmax_std(mx / static_cast<double>(pos + extra), -mn / static_cast<double>(neg));
    offset = -static_cast<double>(neg);
  } else {
    delta = (mx - mn) / steps;
    offset = dclamp_std(round(mn / delta), -steps, 0.0);
  }
  // the dequantized grid stays inside [0.99 lowest, 0.99 max] of fp32
  if (offset < 0.0) delta = dmin_std(delta, f32_lo / offset);
  if (offset + steps > 0.0) delta = dmin_std(delta, f32_hi / (offset + steps));
  rxmet_tf_encoding e;
  e.min = delta * offset;
  e.max = delta * (offset + steps);
  e.delta = delta;
  e.offset = offset;
  e.bw = bw;
  e.reserved = 0;
  enc[c] = e;
  TfEnc32 t;
  t.mn = static_cast<float>(e.min);
  t.mx = static_cast<float>(e.max);
  t.delta = static_cast<float>(delta);
  t.inv_delta = 1.0f / t.delta;  // correctly rounded (qdqReciprocal)
  enc32[c] = t;
}

constexpr int kThreads = 256;
// 16-byte vectors per thread per chunk (runs decomposition), per kind of pass.  Measured on
// c2 ([8192, 8192] fp32) as a forward + backward training step of QuantizeDequantize: 4 for the
// forward / backward passes (236-240 us) against 8 (241-244 us); 8 for the read-only min / max
// (45 us against 49 with 4).
constexpr int kVecQdq = 4;
constexpr int kVecMinMax = 8;
constexpr int64_t kMinRun = 1024;  // runs at least this long use the runs decomposition
constexpr int64_t kMinSeg = 16;    // shorter runs use the column decomposition
constexpr int kColTargetBlocks = 2048;
// Runs decomposition with many encodings (at least kWholeRunMinRuns runs, one per encoding):
// a run of up to kWholeRunChunks chunks is one workgroup's, so its encoding gradients are
// complete in that workgroup and no fold follows.  One long run (a single encoding, at least
// kSingleRunMinChunks chunks): kSingleRunPasses chunks per workgroup, interleaved.  Measured on
// c2 as a QuantizeDequantize training step, per tensor: 232 us with 2 chunks against 236
// with 1, 236 with 4 and 241 with 8 (the separate fold kernel reads half the partials); per
// channel with whole rows (two chunks): 226 us against 231 with one chunk per workgroup.
constexpr int kWholeRunChunks = 4;
constexpr int64_t kWholeRunMinRuns = 1024;
constexpr int kSingleRunPasses = 2;
constexpr int64_t kSingleRunMinChunks = 2048;

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------
// Element types and rounding.
// ---------------------------------------------------------------------------------
struct half_t {
  uint16_t b;
};
struct bf16_t {
  uint16_t b;
};

__device__ __forceinline__ float f16_to_f(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
// Round an fp32 value to fp16, nearest even.  The empty asm makes v an fp32 register first:
// without it the compiler folds the multiply or fma that produced v into the conversion
// (v_fma_mixlo_f16), which rounds the exact result to fp16 once instead of rounding it to
// fp32 and then to fp16 as the reference does — different on fp16 ties.
__device__ __forceinline__ uint32_t f_to_f16(float v) {
  __asm__("" : "+v"(v));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}
__device__ __forceinline__ float bf16_to_f(uint32_t b) {
  return __builtin_bit_cast(float, (b & 0xFFFFu) << 16);
}
// Round to nearest even on the bit pattern; NaN becomes the quiet NaN 0x7FC0, as torch's
// BFloat16 conversion does.
__device__ __forceinline__ uint32_t f_to_bf16(float v) {
  if (v != v) return 0x7FC0u;
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Loads, stores and 16-byte (un)packing of the io type, all through fp32 values.
template <typename T>
struct Io;

template <>
struct Io<float> {
  using V = float;             // the value type elements are computed in
  static constexpr int E = 4;  // elements per 16-byte vector
  __device__ static float ld(const float *p, int64_t i) { return p[i]; }
  __device__ static void st(float *p, int64_t i, float v) { p[i] = v; }
  __device__ static void unpack(const u4 &v, float (&a)[E]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // copy the element out first: __builtin_bit_cast of an ext-vector element lvalue
      // reads element 0
      const unsigned w = v[k];
      a[k] = __builtin_bit_cast(float, w);
    }
  }
  __device__ static u4 pack(const float (&a)[E]) {
    u4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __builtin_bit_cast(unsigned, a[k]);
    return v;
  }
  __device__ static float round(float v) { return v; }
};

// 16-bit io types: BF selects bf16 (else fp16).
template <typename Tag, bool BF>
struct Io16 {
  using V = float;
  static constexpr int E = 8;
  __device__ static float to_f(uint32_t b) { return BF ? bf16_to_f(b) : f16_to_f(b); }
  __device__ static uint32_t from_f(float v) { return BF ? f_to_bf16(v) : f_to_f16(v); }
  __device__ static float ld(const Tag *p, int64_t i) { return to_f(p[i].b); }
  __device__ static void st(Tag *p, int64_t i, float v) {
    Tag t;
    t.b = static_cast<uint16_t>(from_f(v));
    p[i] = t;
  }
  __device__ static void unpack(const u4 &v, float (&a)[E]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[2 * k] = to_f(v[k] & 0xFFFFu);
      a[2 * k + 1] = to_f(v[k] >> 16);
    }
  }
  __device__ static u4 pack(const float (&a)[E]) {
    u4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = from_f(a[2 * k]) | (from_f(a[2 * k + 1]) << 16);
    return v;
  }
  __device__ static float round(float v) { return to_f(from_f(v)); }
};

template <>
struct Io<half_t> : Io16<half_t, false> {};
template <>
struct Io<bf16_t> : Io16<bf16_t, true> {};

// fp64 tensors: elements stay in double (the reference computes in the tensor's own type).
template <>
struct Io<double> {
  using V = double;
  static constexpr int E = 2;
  __device__ static double ld(const double *p, int64_t i) { return p[i]; }
  __device__ static void st(double *p, int64_t i, double v) { p[i] = v; }
  __device__ static void unpack(const u4 &v, double (&a)[E]) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const unsigned lo = v[2 * k], hi = v[2 * k + 1];
      a[k] = __builtin_bit_cast(double, (static_cast<unsigned long long>(hi) << 32) | lo);
    }
  }
  __device__ static u4 pack(const double (&a)[E]) {
    u4 v;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const unsigned long long b = __builtin_bit_cast(unsigned long long, a[k]);
      v[2 * k] = static_cast<unsigned>(b);
      v[2 * k + 1] = static_cast<unsigned>(b >> 32);
    }
    return v;
  }
  __device__ static double round(double v) { return v; }
};

// Rounding of an intermediate result to the internal type R, in R's compute type A.
template <typename R>
struct Rnd {
  using A = float;
  __device__ static float r(float v) { return Io<R>::round(v); }
};
template <>
struct Rnd<double> {
  using A = double;
  __device__ static double r(double v) { return v; }
};

__device__ __forceinline__ float rint_a(float v) { return rintf(v); }
__device__ __forceinline__ double rint_a(double v) { return rint(v); }
__device__ __forceinline__ float fma_a(float a, float b, float c) { return fmaf(a, b, c); }
__device__ __forceinline__ double fma_a(double a, double b, double c) { return fma(a, b, c); }

// x / s in the internal type: fp32 by the correctly rounded reciprocal (div_rn.h), fp64 by
// the division.
__device__ __forceinline__ float div_a(float x, float s, float rs) { return div_rn(x, s, rs); }
__device__ __forceinline__ double div_a(double x, double s, float) { return x / s; }
template <typename A>
__device__ __forceinline__ A clamp_a(A v, A lo, A hi) {
  return v < lo ? lo : (v > hi ? hi : v);  // NaN falls through (torch.clamp)
}

// Per-launch scalars.
struct Params {
  double qmin, qmax;   // grid (exact in R)
  double alpha;        // zero_point_shift (0: none); taken to R where it is used
  int scalar_scale;    // the scale is a 0-dim tensor (see rxmet_qdq_numerics)
};

// Learnable min / max encodings (QuantizeDequantize's parameters) as the source of a launch's
// scale and offset: each block derives its encodings from min and max itself, as
// get_scale / _get_offset evaluate them on the GPU (quantizer.py:345-403), instead of reading
// scale and offset tensors made by separate launches.  mn == null: scale / offset are given.
struct MinMaxSrc {
  const float *mn, *mx;
  float inv_steps;  // fp32 reciprocal of (qmax - qmin): a tensor / scalar on the GPU
  float qmin, qmax, sym_offset, min_scale;
  int symmetric;
};

// scale = clamp_min(|(max - min) / steps|, min_scale); offset = the symmetric offset, or
// clamp(rint(min / scale) - qmin, -qmax, -qmin); all in fp32 (clamp_min keeps NaN).
__device__ __forceinline__ void minmax_scale_offset(const MinMaxSrc &m, int64_t c, float &s,
                                                    float &o) {
  s = fabsf((m.mx[c] - m.mn[c]) * m.inv_steps);
  s = s < m.min_scale ? m.min_scale : s;
  if (m.symmetric) {
    o = m.sym_offset;
  } else {
    o = rintf(m.mn[c] / s) - m.qmin;
    o = o < -m.qmax ? -m.qmax : o;
    o = o > -m.qmin ? -m.qmin : o;
  }
}

// Gradients of min and max from those of scale (gs) and offset (go; unused when symmetric):
// the autograd rules of the expressions above (STE through rint).
__device__ __forceinline__ void minmax_encoding_grad(const MinMaxSrc &m, int64_t c, float gs,
                                                     const float *go, float &d_min,
                                                     float &d_max) {
  const float mn = m.mn[c];
  const float raw = (m.mx[c] - mn) * m.inv_steps, a = fabsf(raw);
  const float s = a < m.min_scale ? m.min_scale : a;
  float gmin = 0.0f;
  if (!m.symmetric && go) {
    const float o = rintf(mn / s) - m.qmin;
    const float gr = (o >= -m.qmax && o <= -m.qmin) ? *go : 0.0f;  // clamp, then STE round
    gmin += gr / s;                                                // d(min / s) / d min
    gs += -gr * ((mn / s) / s);                                    // d(min / s) / d s
  }
  const float ga = a >= m.min_scale ? gs : 0.0f;  // clamp_min
  const float sg = raw > 0.0f ? 1.0f : (raw < 0.0f ? -1.0f : 0.0f);
  const float gr2 = (ga * sg) * m.inv_steps;      // d|raw| and d((max - min) / steps)
  d_max = gr2;
  d_min = gmin - gr2;
}

// One encoding as the element functions use it.
template <typename T, typename R>
struct Elem {
  using A = typename Rnd<R>::A;
  struct Enc {
    A s, o, qmin, qmax, lo, hi;  // internal-type values (lo/hi: o + qmin, o + qmax)
    float fs, inv_s, zp, s_io;   // fp32 forms (frozen path) and the scale rounded to T
  };

  __device__ static A r(A v) { return Rnd<R>::r(v); }

  __device__ static Enc enc(const float *scale, const float *offset, const MinMaxSrc &mm,
                            int64_t c, const Params &p) {
    Enc e;
    float s, o;
    if (mm.mn != nullptr) {
      // scale.to(R), offset.to(R) of the derived fp32 encodings
      minmax_scale_offset(mm, c, s, o);
      if constexpr (std::is_same<A, float>::value) {
        s = Rnd<R>::r(s);
        o = Rnd<R>::r(o);
      }
    } else {
      s = scale[c];
      o = offset ? offset[c] : 0.0f;
    }
    e.s = A(s);
    e.o = A(o);
    e.qmin = A(p.qmin);
    e.qmax = A(p.qmax);
    e.lo = r(e.o + e.qmin);
    e.hi = r(e.o + e.qmax);
    e.fs = s;
    // torch's fake_quantize kernels multiply by fp32 1/scale; with A = fp32 it is also the
    // correctly rounded reciprocal of e.s that div_a takes
    e.inv_s = 1.0f / s;
    e.zp = -truncf(o);   // zero point = -offset.to(int32)
    e.s_io = Io<T>::round(s);
    return e;
  }

  // The tensor QuantDequantFunc receives: x, or torch.sub(x, scale, alpha=shift).  With a
  // 0-dim scale and R wider than T, type promotion keeps that subtraction in T (the scale
  // is rounded to T first); otherwise it runs in R.
  __device__ static A shifted(typename Io<T>::V x, const Enc &e, const Params &p) {
    if (p.alpha == 0.0) return A(x);
    if constexpr (std::is_same<typename Io<T>::V, float>::value)
      if (p.scalar_scale) return A(Io<T>::round(fmaf(-static_cast<float>(p.alpha), e.s_io, x)));
    return r(fma_a(A(-p.alpha), e.s, A(x)));
  }

  // QuantDequantFunc.forward: (clamp(rint(v / s) - o) + o) * s, each step rounded to R.
  __device__ static A qdq(A v, const Enc &e) {
    const A t = r(div_a(v, e.s, e.inv_s));
    const A q = r(rint_a(t) - e.o);
    return r(r(clamp_a(q, e.qmin, e.qmax) + e.o) * e.s);
  }

  // torch.add(qdq, scale, alpha=shift) in R.
  __device__ static A unshift(A y, const Enc &e, const Params &p) {
    return p.alpha == 0.0 ? y : r(fma_a(A(p.alpha), e.s, y));
  }
};

// Forward value of one element (in the io type's value type V; the store rounds it to T).
template <int OP, typename T, typename R, typename V = typename Io<T>::V>
__device__ __forceinline__ V fwd_elem(V x, const typename Elem<T, R>::Enc &e, const Params &p) {
  using El = Elem<T, R>;
  using A = typename El::A;
  if constexpr (OP == OP_QDQ_LEARN) {
    return static_cast<V>(El::unshift(El::qdq(El::shifted(x, e, p), e), e, p));
  } else if constexpr (OP == OP_QDQ_FROZEN) {
    if constexpr (std::is_same<V, double>::value) {
      // torch's fake_quantize on an fp64 tensor: the code from x times the fp32 1 / scale in
      // double, then the clamp, zero point and scale in fp32
      const double qd = rint(x * static_cast<double>(e.inv_s)) + static_cast<double>(e.zp);
      const float q = static_cast<float>(qd);
      return static_cast<double>(
          (clamp_keep_nan(q, static_cast<float>(p.qmin), static_cast<float>(p.qmax)) - e.zp) * e.fs);
    } else {
      const float q = rintf(x * e.inv_s) + e.zp;
      return (clamp_keep_nan(q, static_cast<float>(p.qmin), static_cast<float>(p.qmax)) - e.zp) *
             e.fs;
    }
  } else if constexpr (OP == OP_Q) {
    const A t = El::r(div_a(A(x), e.s, e.inv_s));
    return static_cast<V>(clamp_a(El::r(rint_a(t) - e.o), e.qmin, e.qmax));
  } else if constexpr (OP == OP_NATIVE) {
    // NaN kept; clip in value space (fmax(fmin(v, max), min)); times fl(1 / delta); round
    // half to even; times delta
    if (x != x) return x;
    const float c = fmaxf(fminf(x, e.hi), e.lo);
    return rintf(c * e.inv_s) * e.fs;
  } else if constexpr (OP == OP_FP16) {
    return static_cast<V>(static_cast<_Float16>(x));  // round to nearest even, and back
  } else {
    return static_cast<V>(El::r(El::r(A(x) + e.o) * e.s));
  }
}

// One element of the backward: returns dx and adds this element's encoding-gradient terms
// (as the reference rounds them, in R) to the fp64 sums (ds, dof).
template <int OP, typename T, typename R, typename V = typename Io<T>::V>
__device__ __forceinline__ V bwd_elem(V x, V g, const typename Elem<T, R>::Enc &e, const Params &p,
                                      double &ds, double &dof) {
  using El = Elem<T, R>;
  using A = typename El::A;
  const A ga = A(g);
  if constexpr (OP == OP_QDQ_LEARN) {
    const A t = El::r(div_a(El::shifted(x, e, p), e.s, e.inv_s));
    const A rr = rint_a(t);
    const A q = El::r(rr - e.o);
    const A m = (q >= e.qmin && q <= e.qmax) ? A(1) : A(0);
    const A nm = A(1) - m;
    ds += static_cast<double>(El::r(ga * El::r(clamp_a(rr, e.lo, e.hi) - t * m)));
    dof += static_cast<double>(El::r(ga * El::r(nm * e.s)));
    // the shift's own scale terms: +alpha*g from the add, -alpha*g*mask through the sub
    if (p.alpha != 0.0)
      ds += static_cast<double>(A(p.alpha)) * static_cast<double>(ga * nm);
    return static_cast<V>(ga * m);
  } else if constexpr (OP == OP_QDQ_FROZEN) {
    if constexpr (std::is_same<V, double>::value) {
      const double q = rint(x * static_cast<double>(e.inv_s)) + static_cast<double>(e.zp);
      return (q >= p.qmin && q <= p.qmax) ? g : g * 0.0;
    } else {
      const float q = rintf(x * e.inv_s) + e.zp;
      const float m = (q >= p.qmin && q <= p.qmax) ? 1.0f : 0.0f;
      return g * m;
    }
  } else if constexpr (OP == OP_Q) {
    const A t = El::r(div_a(A(x), e.s, e.inv_s));
    const A q = El::r(rint_a(t) - e.o);
    const A m = (q >= e.qmin && q <= e.qmax) ? A(1) : A(0);
    const A mg = ga * m;
    const A gs = El::r(div_a(mg, e.s, e.inv_s));
    // QuantizeFunc.backward divides the saved input (type T) by the scale: in T when the
    // scale is 0-dim, in R otherwise
    const A xs = p.scalar_scale ? A(Io<T>::round(x / e.s_io)) : t;
    ds += static_cast<double>(El::r(-gs * xs));
    dof += static_cast<double>(-mg);
    return static_cast<V>(gs);
  } else {
    const A gs = El::r(ga * e.s);
    ds += static_cast<double>(El::r(ga * El::r(A(x) + e.o)));
    dof += static_cast<double>(gs);
    return static_cast<V>(gs);
  }
}

// ---------------------------------------------------------------------------------
// Accumulators.
// ---------------------------------------------------------------------------------
struct Sum2 {
  double a, b;
};
struct MinMax {
  float mn, mx;
};

__device__ __forceinline__ void acc_add(Sum2 &x, const Sum2 &y) {
  x.a += y.a;
  x.b += y.b;
}
__device__ __forceinline__ void acc_add(MinMax &x, const MinMax &y) {
  x.mn = nan_min(x.mn, y.mn);
  x.mx = nan_max(x.mx, y.mx);
}
__device__ __forceinline__ Sum2 acc_shfl(const Sum2 &x, int off) {
  return Sum2{__shfl_xor(x.a, off, kWave), __shfl_xor(x.b, off, kWave)};
}
__device__ __forceinline__ MinMax acc_shfl(const MinMax &x, int off) {
  return MinMax{__shfl_xor(x.mn, off, kWave), __shfl_xor(x.mx, off, kWave)};
}

// Rounding of a folded encoding gradient to the internal type (0: fp32, 1: fp16, 2: bf16),
// as the reference's gradient tensors carry it.
__device__ __forceinline__ float round_internal(float v, int round16) {
  if (round16 == 1) return Io<half_t>::round(v);
  if (round16 == 2) return Io<bf16_t>::round(v);
  return v;
}

// Folded encoding gradients, written as the gradients of scale and offset.
struct PutScaleOffset {
  float *dscale, *doffset;
  int round16;
  __device__ void operator()(const Sum2 &v, int64_t c) const {
    if (dscale) dscale[c] = round_internal(static_cast<float>(v.a), round16);
    if (doffset) doffset[c] = round_internal(static_cast<float>(v.b), round16);
  }
};

// Folded encoding gradients taken on to the min / max they were derived from.
struct PutMinMaxGrad {
  MinMaxSrc mm;
  float *d_min, *d_max;
  int round16;
  __device__ void operator()(const Sum2 &v, int64_t c) const {
    const float gs = round_internal(static_cast<float>(v.a), round16);
    const float go = round_internal(static_cast<float>(v.b), round16);
    float a, b;
    minmax_encoding_grad(mm, c, gs, &go, a, b);
    d_min[c] = a;
    d_max[c] = b;
  }
};

// A backward launch with encoding gradients completes them by a separate fold kernel over the
// partials, or (direct: one workgroup per encoding) each workgroup writes its own encoding's.
struct FusedFold {
  int direct;
  int use_mm;  // min / max gradients instead of scale / offset gradients
  PutScaleOffset so;
  PutMinMaxGrad mg;
  __device__ void put(const Sum2 &v, int64_t c) const {
    if (use_mm)
      mg(v, c);
    else
      so(v, c);
  }
};

// Whole-block reduction; thread 0 ends with the block's value (fixed order).
template <typename Acc>
__device__ __forceinline__ void block_reduce(Acc &a) {
  __shared__ Acc red[kThreads / kWave];
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) acc_add(a, acc_shfl(a, off));
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    a = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / kWave; ++i) acc_add(a, red[i]);
  }
}

// ---------------------------------------------------------------------------------
// Work policies: what one element / one 16-byte vector does.
// ---------------------------------------------------------------------------------
template <int OP, typename T, typename R>
struct FwdW {
  using El = Elem<T, R>;
  using Enc = typename El::Enc;
  using Acc = Sum2;  // unused
  static constexpr bool kReduce = false;
  static constexpr bool kFold = false;
  static constexpr int E = Io<T>::E;
  static constexpr int V = kVecQdq;
  const T *x;
  T *y;
  const float *scale, *offset;
  Params p;
  MinMaxSrc mm;

  __device__ Enc enc(int64_t c) const {
    if constexpr (OP == OP_NATIVE) {
      // `scale` holds the TfEnc32 array of the launch
      const TfEnc32 t = reinterpret_cast<const TfEnc32 *>(scale)[c];
      Enc e{};
      e.lo = t.mn;
      e.hi = t.mx;
      e.fs = t.delta;
      e.inv_s = t.inv_delta;
      return e;
    } else if constexpr (OP == OP_FP16) {
      return Enc{};
    } else {
      return El::enc(scale, offset, mm, c, p);
    }
  }
  __device__ static Acc zero() { return Sum2{0.0, 0.0}; }
  __device__ void elem(const Enc &e, int64_t i, Acc &) const {
    Io<T>::st(y, i, fwd_elem<OP, T, R>(Io<T>::ld(x, i), e, p));
  }
  // Non-temporal loads and stores.  Ordinary stores time about 6 % faster in a loop of one
  // pass, but leave the output in the caches to be written back during the next pass: a
  // forward + backward training step measured 255-263 us with them against 236-240 us.
  __device__ void compute(const Enc &e, const u4 &v, int64_t vi) const {
    typename Io<T>::V a[E];
    Io<T>::unpack(v, a);
#pragma unroll
    for (int k = 0; k < E; ++k) a[k] = fwd_elem<OP, T, R>(a[k], e, p);
    __builtin_nontemporal_store(Io<T>::pack(a), reinterpret_cast<u4 *>(y) + vi);
  }
  __device__ void vec1(const Enc &e, int64_t vi, Acc &) const {
    compute(e, __builtin_nontemporal_load(reinterpret_cast<const u4 *>(x) + vi), vi);
  }
  // V vectors per thread: all loads issued before any compute
  __device__ void vec_block(const Enc &e, int64_t vb, int nv, Acc &) const {
    const u4 *xv = reinterpret_cast<const u4 *>(x) + vb;
    u4 v[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) v[k] = __builtin_nontemporal_load(xv + i);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) compute(e, v[k], vb + i);
    }
  }
};

template <int OP, typename T, typename R, bool ENC>
struct BwdW {
  using El = Elem<T, R>;
  using Enc = typename El::Enc;
  using Acc = Sum2;
  static constexpr bool kReduce = ENC;
  static constexpr bool kFold = ENC;
  static constexpr int E = Io<T>::E;
  static constexpr int V = kVecQdq;
  const T *x, *g;
  T *dx;
  const float *scale, *offset;
  Params p;
  MinMaxSrc mm;
  FusedFold ff;  // how the encoding gradients complete (ENC)

  __device__ Enc enc(int64_t c) const { return El::enc(scale, offset, mm, c, p); }
  __device__ static Acc zero() { return Sum2{0.0, 0.0}; }
  __device__ void elem(const Enc &e, int64_t i, Acc &acc) const {
    Io<T>::st(dx, i,
              bwd_elem<OP, T, R>(Io<T>::ld(x, i), Io<T>::ld(g, i), e, p, acc.a, acc.b));
  }
  __device__ void compute(const Enc &e, const u4 &xv, const u4 &gv, int64_t vi,
                          Acc &acc) const {
    typename Io<T>::V a[E], b[E];
    Io<T>::unpack(xv, a);
    Io<T>::unpack(gv, b);
#pragma unroll
    for (int k = 0; k < E; ++k) a[k] = bwd_elem<OP, T, R>(a[k], b[k], e, p, acc.a, acc.b);
    __builtin_nontemporal_store(Io<T>::pack(a), reinterpret_cast<u4 *>(dx) + vi);
  }
  __device__ void vec1(const Enc &e, int64_t vi, Acc &acc) const {
    const u4 xv = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(x) + vi);
    const u4 gv = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(g) + vi);
    compute(e, xv, gv, vi, acc);
  }
  __device__ void vec_block(const Enc &e, int64_t vb, int nv, Acc &acc) const {
    const u4 *xv = reinterpret_cast<const u4 *>(x) + vb;
    const u4 *gv = reinterpret_cast<const u4 *>(g) + vb;
    u4 xr[V], gr[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) {
        xr[k] = __builtin_nontemporal_load(xv + i);
        gr[k] = __builtin_nontemporal_load(gv + i);
      }
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) compute(e, xr[k], gr[k], vb + i, acc);
    }
  }
};

// SKIP_NAN: NaN never replaces a running value, as the reference's CPU statistics
// (math_functions.cpp:356-375: val = min(val, x) from +-max) — a block of NaN only keeps
// +inf / -inf.  Otherwise NaN propagates (torch.aminmax).
template <typename T, bool SKIP_NAN = false>
struct MinMaxW {
  struct Enc {};
  using Acc = MinMax;
  static constexpr bool kReduce = true;
  static constexpr bool kFold = false;
  static constexpr int E = Io<T>::E;
  static constexpr int V = kVecMinMax;
  const T *x;

  __device__ Enc enc(int64_t) const { return Enc{}; }
  __device__ static Acc zero() { return MinMax{INFINITY, -INFINITY}; }
  __device__ static void take(Acc &acc, float v) {
    if constexpr (SKIP_NAN) {
      acc.mn = v < acc.mn ? v : acc.mn;
      acc.mx = acc.mx < v ? v : acc.mx;
    } else {
      acc.mn = nan_min(acc.mn, v);
      acc.mx = nan_max(acc.mx, v);
    }
  }
  // fp64 values are rounded to fp32 first: rounding is monotone, so the fp32 min / max equal
  // the rounded fp64 min / max (the statistics are fp32)
  __device__ void elem(const Enc &, int64_t i, Acc &acc) const {
    take(acc, static_cast<float>(Io<T>::ld(x, i)));
  }
  __device__ static void take_vec(const u4 &v, Acc &acc) {
    typename Io<T>::V a[E];
    Io<T>::unpack(v, a);
#pragma unroll
    for (int k = 0; k < E; ++k) take(acc, static_cast<float>(a[k]));
  }
  __device__ void vec1(const Enc &, int64_t vi, Acc &acc) const {
    take_vec(__builtin_nontemporal_load(reinterpret_cast<const u4 *>(x) + vi), acc);
  }
  __device__ void vec_block(const Enc &, int64_t vb, int nv, Acc &acc) const {
    const u4 *xv = reinterpret_cast<const u4 *>(x) + vb;
    u4 v[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) v[k] = __builtin_nontemporal_load(xv + i);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int i = k * kThreads + threadIdx.x;
      if (i < nv) take_vec(v[k], acc);
    }
  }
};

// ---------------------------------------------------------------------------------
// Decompositions.
// ---------------------------------------------------------------------------------
struct Geo {
  int64_t inner, C1, midC1, C0;
};
// encoding of run q = ((o * C0 + c0) * mid + m) * C1 + c1
__device__ __forceinline__ int64_t enc_of_run(const Geo &g, int64_t q) {
  return ((q / g.midC1) % g.C0) * g.C1 + q % g.C1;
}

struct ColGeo {
  int64_t mid, K, inner, C1, C0;  // band rows, band columns (C1 * inner)
  int64_t col_tiles, chunks, rows_per_chunk;
  int kt_shift;                    // log2 of the threads per row (the rest walk rows)
};

// runs: block b handles chunks sp, sp + splits, ... (`passes` of them, sp = b % splits) of
// run b / splits, so that the blocks in flight read adjacent memory; one partial per block,
// or (kFold, direct) the block's encoding gradients.
template <class W>
__global__ __launch_bounds__(kThreads) void k_runs(W w, Geo geo, int64_t splits, int passes,
                                                   int vec,
                                                   typename W::Acc *__restrict__ partial) {
  constexpr int64_t kChunk = int64_t(kThreads) * W::V * W::E;
  const int64_t b = blockIdx.x;
  const int64_t run = b / splits, sp = b % splits;
  const int64_t c = enc_of_run(geo, run);
  const auto e = w.enc(c);
  const int64_t first = sp * kChunk, step = kChunk * splits;
  const int64_t rb = run * geo.inner;
  typename W::Acc acc = W::zero();
  for (int q = 0; q < passes; ++q) {
    const int64_t beg = first + q * step;
    if (beg >= geo.inner) break;
    const int64_t end = min(geo.inner, beg + kChunk);
    if (vec) {
      w.vec_block(e, (rb + beg) / W::E, static_cast<int>((end - beg) / W::E), acc);
    } else {
      const int n = static_cast<int>(end - beg);
      for (int i = threadIdx.x; i < n; i += kThreads) w.elem(e, rb + beg + i, acc);
    }
  }
  if constexpr (W::kReduce) {
    block_reduce(acc);
    if constexpr (W::kFold) {
      if (w.ff.direct) {
        if (threadIdx.x == 0) w.ff.put(acc, c);
        return;
      }
    }
    if (threadIdx.x == 0) partial[b] = acc;
  }
}

// segs: a segment of 2^tpr_shift lanes per run, kThreads >> tpr_shift runs per pass,
// `iters` passes per block; one partial per run.
template <class W>
__global__ __launch_bounds__(kThreads) void k_segs(W w, Geo geo, int64_t runs, int tpr_shift,
                                                   int iters, int vec,
                                                   typename W::Acc *__restrict__ partial) {
  const int tpr = 1 << tpr_shift;
  const int seg = threadIdx.x >> tpr_shift, lane = threadIdx.x & (tpr - 1);
  const int64_t per_pass = kThreads >> tpr_shift;
  const int64_t n = vec ? geo.inner / W::E : geo.inner;
  for (int it = 0; it < iters; ++it) {
    const int64_t q = (static_cast<int64_t>(blockIdx.x) * iters + it) * per_pass + seg;
    typename W::Acc acc = W::zero();
    if (q < runs) {
      const auto e = w.enc(enc_of_run(geo, q));
      if (vec) {
        const int64_t vb = q * n;
        for (int64_t v = lane; v < n; v += tpr) w.vec1(e, vb + v, acc);
      } else {
        const int64_t base = q * geo.inner;
        for (int64_t i = lane; i < n; i += tpr) w.elem(e, base + i, acc);
      }
    }
    if constexpr (W::kReduce) {
      for (int off = tpr >> 1; off > 0; off >>= 1) acc_add(acc, acc_shfl(acc, off));
      if (lane == 0 && q < runs) partial[q] = acc;
    }
  }
}

// cols: block b owns columns [tile * Kt, +Kt) of the rows of chunk h of band `band`;
// kThreads / Kt rows are walked in parallel and combined through LDS.
template <class W>
__global__ __launch_bounds__(kThreads) void k_cols(W w, ColGeo cg,
                                                   typename W::Acc *__restrict__ partial) {
  const int kt = 1 << cg.kt_shift;
  const int lane = threadIdx.x & (kt - 1), prow = threadIdx.x >> cg.kt_shift;
  const int P = kThreads >> cg.kt_shift;
  const int64_t tile = blockIdx.x % cg.col_tiles, rest = blockIdx.x / cg.col_tiles;
  const int64_t h = rest % cg.chunks, band = rest / cg.chunks;
  const int64_t j = tile * kt + lane;
  typename W::Acc acc = W::zero();
  if (j < cg.K) {
    const auto e = w.enc((band % cg.C0) * cg.C1 + j / cg.inner);
    const int64_t rb = band * cg.mid;
    const int64_t r1 = rb + min(cg.mid, (h + 1) * cg.rows_per_chunk);
    for (int64_t r = rb + h * cg.rows_per_chunk + prow; r < r1; r += P)
      w.elem(e, r * cg.K + j, acc);
  }
  if constexpr (W::kReduce) {
    if (P > 1) {
      __shared__ typename W::Acc red[kThreads];
      red[threadIdx.x] = acc;
      __syncthreads();
      if (prow == 0)
        for (int q = 1; q < P; ++q) acc_add(acc, red[q * kt + lane]);
    }
    if (prow == 0 && j < cg.K) partial[(band * cg.chunks + h) * cg.K + j] = acc;
  }
}

// ---------------------------------------------------------------------------------
// Host-side plan (shared by the entry points and the per-type launchers).
// ---------------------------------------------------------------------------------
enum Kind { KIND_RUNS = 0, KIND_SEGS = 1, KIND_COLS = 2 };

struct FoldMap {
  int64_t n0, n1, n2;  // loop counts
  int64_t s0, s1, s2;  // loop strides
  int64_t C1, sc0, sc1;  // encoding c = c0 * C1 + c1 adds c0 * sc0 + c1 * sc1
};

struct Plan {
  int kind = KIND_RUNS;
  int64_t outer = 0, C0 = 1, mid = 1, C1 = 1, inner = 0;  // normalized layout
  int64_t n = 0;                                           // elements
  int64_t runs = 0, splits = 0;                            // runs / segs
  int passes = 1;                                          // runs: chunks per block
  bool direct = false;  // runs: one block per encoding (its gradients need no fold)
  Geo geo{};
  ColGeo cg{};
  int64_t col_blocks = 0;
  int64_t partial_slots = 0;
  FoldMap fold{};
  int esize = 4;
};

struct Call {
  const Plan *plan;
  int op;
  int internal;            // RXMET_QDQ_F32 / F16 / BF16 / F64
  const void *x, *g;
  void *out;               // y / q / dx
  const float *scale, *offset;
  Params p;
  void *partial;           // Sum2 / MinMax partials, or null
  hipStream_t stream;
  MinMaxSrc mm;            // mm.mn != null: encodings derived from min / max in the kernels
  FusedFold ff;            // backward with encoding gradients: how they complete
};

template <class W>
static int launch_decomp(const Plan &pl, const W &w, bool aligned, void *partial,
                         hipStream_t s) {
  using Acc = typename W::Acc;
  Acc *part = static_cast<Acc *>(partial);
  const bool vec = aligned && pl.inner % W::E == 0;
  if (pl.kind == KIND_RUNS) {
    hipLaunchKernelGGL(k_runs<W>, dim3(static_cast<unsigned>(pl.runs * pl.splits)),
                       dim3(kThreads), 0, s, w, pl.geo, pl.splits, pl.passes, int(vec), part);
  } else if (pl.kind == KIND_SEGS) {
    const int64_t nv = vec ? pl.inner / W::E : pl.inner;
    int shift = 0;
    while (shift < 6 && (int64_t(1) << shift) < nv) ++shift;
    const int64_t per_thread = (nv + (int64_t(1) << shift) - 1) >> shift;
    const int64_t per_pass = kThreads >> shift;
    int iters = per_thread >= 8 ? 1 : static_cast<int>(8 / per_thread);
    while (iters > 1 && (pl.runs + per_pass * iters - 1) / (per_pass * iters) < 2048) iters >>= 1;
    const int64_t blocks = (pl.runs + per_pass * iters - 1) / (per_pass * iters);
    hipLaunchKernelGGL(k_segs<W>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, w,
                       pl.geo, pl.runs, shift, iters, int(vec), part);
  } else {
    hipLaunchKernelGGL(k_cols<W>, dim3(static_cast<unsigned>(pl.col_blocks)), dim3(kThreads), 0,
                       s, w, pl.cg, part);
  }
  return 0;
}

static inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <int OP, typename T, typename R>
static int run_forward(const Call &c) {
  FwdW<OP, T, R> w{static_cast<const T *>(c.x), static_cast<T *>(c.out), c.scale, c.offset, c.p,
                   c.mm};
  return launch_decomp(*c.plan, w, aligned16(c.x) && aligned16(c.out), nullptr, c.stream);
}

template <int OP, typename T, typename R>
static int run_backward(const Call &c) {
  const bool al = aligned16(c.x) && aligned16(c.g) && aligned16(c.out);
  if (c.partial) {
    BwdW<OP, T, R, true> w{static_cast<const T *>(c.x), static_cast<const T *>(c.g),
                           static_cast<T *>(c.out), c.scale, c.offset, c.p, c.mm, c.ff};
    return launch_decomp(*c.plan, w, al, c.partial, c.stream);
  }
  BwdW<OP, T, R, false> w{static_cast<const T *>(c.x), static_cast<const T *>(c.g),
                          static_cast<T *>(c.out), c.scale, c.offset, c.p, c.mm};
  return launch_decomp(*c.plan, w, al, nullptr, c.stream);
}

template <typename T, bool SKIP_NAN>
static int run_minmax(const Call &c) {
  MinMaxW<T, SKIP_NAN> w{static_cast<const T *>(c.x)};
  return launch_decomp(*c.plan, w, aligned16(c.x), c.partial, c.stream);
}

enum What { WHAT_FORWARD = 0, WHAT_BACKWARD = 1, WHAT_MINMAX = 2, WHAT_MINMAX_SKIP_NAN = 3 };

// The internal types each io type pairs with: R = T, fp32 or fp64 (fp32 io: fp32, fp64).
template <typename T>
static int run_typed(const Call &c, int what) {
  if (what == WHAT_MINMAX) return run_minmax<T, false>(c);
  if (what == WHAT_MINMAX_SKIP_NAN) return run_minmax<T, true>(c);
  if (c.op == OP_NATIVE || c.op == OP_FP16) {  // fp32 arithmetic, forward only
    if (what != WHAT_FORWARD) return -22;
    return c.op == OP_NATIVE ? run_forward<OP_NATIVE, T, float>(c)
                             : run_forward<OP_FP16, T, float>(c);
  }
  auto go = [&](auto rtag) -> int {
    using R = decltype(rtag);
    auto fw = what == WHAT_FORWARD;
    switch (c.op) {
      case OP_QDQ_LEARN:
        return fw ? run_forward<OP_QDQ_LEARN, T, R>(c) : run_backward<OP_QDQ_LEARN, T, R>(c);
      case OP_Q:
        return fw ? run_forward<OP_Q, T, R>(c) : run_backward<OP_Q, T, R>(c);
      default:
        return -22;
    }
  };
  if (c.op == OP_QDQ_FROZEN)  // torch's fake_quantize kernels: fp32 math on any io type
    return what == WHAT_FORWARD ? run_forward<OP_QDQ_FROZEN, T, float>(c)
                                : run_backward<OP_QDQ_FROZEN, T, float>(c);
  if (c.op == OP_DQ)  // DequantizeFunc runs in the tensor's own type
    return what == WHAT_FORWARD ? run_forward<OP_DQ, T, T>(c) : run_backward<OP_DQ, T, T>(c);
  if constexpr (std::is_same<T, double>::value) {
    if (c.internal != RXMET_QDQ_F64) return -22;  // an fp64 tensor computes in fp64
    return go(double{});
  }
  switch (c.internal) {
    case RXMET_QDQ_F64:
      return go(double{});
    case RXMET_QDQ_F32:
      return go(float{});
    default:
      if constexpr (!std::is_same<T, float>::value) return go(T{});
      return -22;
  }
}

// Per-io-type entry points, one translation unit each.
int run_f32(const Call &c, int what);
int run_f16(const Call &c, int what);
int run_bf16(const Call &c, int what);
int run_f64(const Call &c, int what);

// Where a TF-scheme quantizer's statistics update lands (ONNX Runtime op): the running
// min / max (replaced after a reset), and with enc set the TfEncodings derived from them.
struct StatsSink {
  float *st_min, *st_max;
  int reset, enc;
  int bw, sym, strict, unsigned_sym;
  rxmet_tf_encoding *enc64;
  TfEnc32 *enc32;
};

// Shared with the ONNX Runtime op core (qc_quantize.hip), defined in qdq.hip:
// per-encoding min / max of the layout with NaN skipped (the reference's CPU statistics), and
// the OP_NATIVE / OP_FP16 forward (f32 or f16 tensors).
int minmax_stats(const void *x, int32_t io, const rxmet_qdq_layout &l, const StatsSink &sink,
                 void *workspace, hipStream_t s);
int forward_tf(int op, const void *x, void *y, int32_t io, const rxmet_qdq_layout &l,
               const TfEnc32 *enc, hipStream_t s);

}  // namespace qdq
}  // namespace rxmet
