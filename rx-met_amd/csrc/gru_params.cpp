// gru_params.cpp — host-side quantisation parameters of the QuantGRU path.
//
// * rxmet_gru_make_params: min/max ranges -> per-operator grids, following
//   calculateGRUQuantitativeParameters (operators/quant-gru/src/gru_host.cc:13-124):
//   calibrateContinuousScaleFromRange (include/pot_sqnr_calibrator.h:372-447), then either
//   the 16-bit-mantissa affine encoding or a power of two (include/scale_encoding.h:250-321,
//   include/pot_scale_encode.h:72-103); biases use the headroom rule of calibrateBias
//   (include/gru_calibration_helpers.h:31-61); gate outputs get ensureMinRange(0.5)
//   (include/calibration_utils.h:27-44).
// * rxmet_gru_make_luts: the 16-segment piecewise-linear sigmoid/tanh tables
//   (src/quantize_lut.cc:53-365), rebuilt from the stored scales as the reference binding
//   does on every call (pytorch/lib/gru_interface_binding.cc:1313).
// * make_step_params / make_channel_factors: the kernels' parameter block, i.e. the
//   reference's setRescaleParam (src/gru_forward_gpu_quant_fp.cu:454-645);
//   make_int_step_params / make_int_channel_rescales: the int32 carrier's
//   (src/gru_forward_gpu_quant.cu:662-752, fillLinearParams / fillGateParams).
//
// All arithmetic is fp32 in the reference's evaluation order (the library is built with
// -ffp-contract=off); libm calls are the same glibc functions the reference uses.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "gru_internal.h"
#include "rxmet_common.h"

namespace rxmet {
namespace gru {
namespace {

struct Grid {
  int32_t bits;
  bool uns;
  Grid(int32_t b, int32_t u) : bits(b), uns(b >= 32 ? false : u != 0) {}
  int32_t qmin() const { return bits >= 32 ? INT32_MIN : (uns ? 0 : -(1 << (bits - 1))); }
  int32_t qmax() const {
    if (bits >= 32) return INT32_MAX;
    return uns ? static_cast<int32_t>((1u << bits) - 1u) : (1 << (bits - 1)) - 1;
  }
  int64_t steps() const { return static_cast<int64_t>(qmax()) - qmin(); }
};

// 16-bit mantissa encoding: scale ~= M * 2^-shift, M in [2^15, 2^16).
struct MShift {
  uint32_t m;
  int shift;
  static MShift encode(float scale) {
    if (!(scale > 0.0f)) throw std::runtime_error("scale must be > 0");
    int e = 0;
    const double frac = std::frexp(static_cast<double>(scale), &e);
    uint32_t m = static_cast<uint32_t>(std::llround(frac * 65536.0));
    if (m == 65536u) {
      m = 32768u;
      ++e;
    }
    m = std::max(m, 32768u);
    const int shift = 16 - e;
    if (shift < -128 || shift > 127) throw std::runtime_error("scale encoding shift out of range");
    return MShift{m, shift};
  }
  float decode() const { return static_cast<float>(m) * std::ldexp(1.0f, -shift); }
};

int8_t pow2_exponent(float scale) {
  if (!(scale > 0.0f)) return 0;
  return static_cast<int8_t>(std::lround(-std::log2(static_cast<double>(scale))));
}

float smallest_scale(int64_t steps) {
  return std::min(1.19209290e-07f, 0.01f / static_cast<float>(steps));
}

struct Continuous {
  float scale, lo, hi;
};

Continuous continuous_scale(float lo, float hi, const Grid &g, bool symmetric) {
  const int64_t n = g.steps();
  if (n <= 0) throw std::runtime_error("grid has no steps");
  const float nf = static_cast<float>(n);
  const float floor_s = smallest_scale(n);
  const float lo0 = std::min(lo, 0.0f);
  const float hi0 = std::max(hi, 0.0f);
  const float step = ((hi0 - lo0) / nf < floor_s) ? floor_s : 0.0f;
  float a = lo0, b = hi0;
  if (symmetric && g.uns) {
    b = hi0 + nf * step;
    a = 0.0f;
  } else if (symmetric) {
    b = hi0 + std::floor(nf / 2.0f) * step;
    a = lo0 - std::ceil(nf / 2.0f) * step;
  } else {
    b = hi0 + nf * step;
  }
  Continuous c{};
  if (symmetric && g.uns) {
    c.scale = std::max(std::max(b, floor_s) / static_cast<float>(g.qmax()), floor_s);
    c.lo = 0.0f;
    c.hi = c.scale * static_cast<float>(g.qmax());
  } else if (symmetric) {
    const int64_t pos = n / 2, neg = (n + 1) / 2;
    const int64_t pos_div = pos + (n == 3 ? 1 : 0);
    const float from_hi = pos_div > 0 ? b / static_cast<float>(pos_div) : 0.0f;
    const float from_lo = neg > 0 ? -a / static_cast<float>(neg) : 0.0f;
    c.scale = std::max(std::max(from_hi, from_lo), floor_s);
    c.lo = -static_cast<float>(neg) * c.scale;
    c.hi = static_cast<float>(pos) * c.scale;
  } else {
    const float span = std::max(b - a, floor_s * nf);
    c.scale = std::max(span / nf, floor_s);
    c.lo = a;
    c.hi = a + c.scale * nf;
  }
  return c;
}

bool close_to_pow2(float v, float rel) {
  if (!(v > 0.0f)) return false;
  const float p = std::pow(2.0f, std::round(std::log2(v)));
  return std::abs(v - p) / p < rel;
}

rxmet_grid encode_grid(const Continuous &c, const Grid &g, bool symmetric,
                       const rxmet_gru_config &cfg) {
  rxmet_grid out{};
  out.bits = g.bits;
  out.is_unsigned = g.uns ? 1 : 0;
  const float qmin_f = static_cast<float>(g.qmin());
  if (cfg.use_pot2) {
    if (!(c.scale > 0.0f)) throw std::runtime_error("scale must be > 0");
    const float e = -std::log2(c.scale);
    float pick;
    switch (cfg.pot_method) {
      case RXMET_POT_ROUND: pick = std::round(e); break;
      case RXMET_POT_FLOOR: pick = std::floor(e); break;
      default:
        pick = close_to_pow2(std::abs(c.hi - c.lo), cfg.pot_tolerance) ? std::round(e)
                                                                         : std::floor(e);
    }
    if (pick < -128.0f || pick > 127.0f) throw std::runtime_error("power-of-two shift out of range");
    const int8_t shift = static_cast<int8_t>(pick);
    const float p2 = std::pow(2.0f, -static_cast<float>(shift));
    int32_t zp = 0;
    if (!symmetric) {
      if (cfg.pot_method == RXMET_POT_FLOOR) {
        const float aligned = std::floor(c.lo / p2) * p2;
        zp = static_cast<int32_t>(std::rint(qmin_f - aligned / p2));
      } else {
        zp = static_cast<int32_t>(std::rint(qmin_f - c.lo / p2));
      }
    }
    out.scale = p2;
    out.zero_point = zp;
    return out;
  }
  const float eff = MShift::encode(c.scale).decode();
  out.scale = c.scale;
  out.zero_point = symmetric ? 0 : static_cast<int32_t>(std::rint(qmin_f - c.lo / eff));
  return out;
}

rxmet_grid grid_from_range(float lo, float hi, const rxmet_bitspec &spec,
                           const rxmet_gru_config &cfg) {
  const Grid g(spec.bits, spec.is_unsigned);
  return encode_grid(continuous_scale(lo, hi, g, spec.symmetric != 0), g, spec.symmetric != 0, cfg);
}

int group_size(int granularity, int H) {
  return granularity == RXMET_PER_TENSOR ? 3 * H : (granularity == RXMET_PER_GATE ? H : 1);
}

// ------------------------------------------------------------------------------------
// Piecewise-linear activation tables
// ------------------------------------------------------------------------------------

std::vector<float> breakpoints(float x_lo, float x_hi) {
  constexpr int kSamples = 1000;
  std::vector<float> xs(kSamples), weight(kSamples - 1), cum(kSamples - 1);
  for (int i = 0; i < kSamples; ++i)
    xs[i] = x_lo + (x_hi - x_lo) * static_cast<float>(i) / (kSamples - 1);
  float total = 0.0f;
  for (int i = 0; i < kSamples - 1; ++i) {
    const float y0 = 1.0f / (1.0f + std::exp(-xs[i]));
    const float y1 = 1.0f / (1.0f + std::exp(-xs[i + 1]));
    const float slope = std::abs(y1 - y0) / (xs[i + 1] - xs[i] + 1e-9f);
    const float d = std::abs(xs[i]);
    weight[i] = d < 2.0f ? 5.0f * (1.0f - d / 2.0f) + 1.0f : 1.0f + slope * 0.5f;
  }
  for (int i = 0; i < kSamples - 1; ++i) total += weight[i];
  for (int i = 0; i < kSamples - 1; ++i) weight[i] /= total;
  cum[0] = weight[0];
  for (int i = 1; i < kSamples - 1; ++i) cum[i] = cum[i - 1] + weight[i];
  std::vector<float> pts{x_lo};
  for (int s = 1; s < kSegments; ++s) {
    const float target = static_cast<float>(s) / kSegments;
    int idx = static_cast<int>(std::lower_bound(cum.begin(), cum.end(), target) - cum.begin());
    idx = std::min(std::max(idx, 0), kSamples - 2);
    pts.push_back(xs[idx]);
  }
  pts.push_back(x_hi);
  std::sort(pts.begin(), pts.end());
  pts.erase(std::unique(pts.begin(), pts.end(),
                        [](float a, float b) { return std::abs(a - b) < 1e-9f; }),
            pts.end());
  while (static_cast<int>(pts.size()) < kSegments + 1) {
    size_t at = 0;
    float widest = 0.0f;
    for (size_t i = 0; i + 1 < pts.size(); ++i)
      if (pts[i + 1] - pts[i] > widest) {
        widest = pts[i + 1] - pts[i];
        at = i;
      }
    pts.insert(pts.begin() + at + 1, (pts[at] + pts[at + 1]) / 2.0f);
  }
  return pts;
}

// Least-squares line through 100 samples of f on [a, b].
template <class F>
void least_squares(float a, float b, F f, float *slope, float *icpt) {
  constexpr int n = 100;
  float sx = 0.0f, sy = 0.0f, sxy = 0.0f, sxx = 0.0f;
  for (int j = 0; j < n; ++j) {
    const float x = a + (b - a) * static_cast<float>(j) / (n - 1);
    const float y = f(x);
    sx += x;
    sy += y;
    sxy += x * y;
    sxx += x * x;
  }
  const float den = n * sxx - sx * sx;
  if (std::abs(den) < 1e-9f) {
    *slope = 0.0f;
    *icpt = sy / n;
    return;
  }
  *slope = (n * sxy - sx * sy) / den;
  *icpt = (sy - *slope * sx) / n;
}

void build_lut(bool is_tanh, const rxmet_grid &in, const rxmet_grid &out, rxmet_pwl_lut *lut) {
  const Grid gi(in.bits, in.is_unsigned), go(out.bits, out.is_unsigned);
  const float sx = in.scale, sy = out.scale;
  const float limit = is_tanh ? 4.0f : 8.0f;
  const float x_lo = std::max(static_cast<float>(gi.qmin() - in.zero_point) * sx, -limit);
  const float x_hi = std::min(static_cast<float>(gi.qmax() - in.zero_point) * sx, limit);
  const std::vector<float> pts = breakpoints(x_lo, x_hi);
  lut->zp_x = in.zero_point;
  const int32_t out_max = go.qmax();
  for (int s = 0; s < kSegments; ++s) {
    float slope, icpt;
    if (is_tanh)
      least_squares(pts[s], pts[s + 1], [](float x) { return std::tanh(x); }, &slope, &icpt);
    else
      least_squares(pts[s], pts[s + 1], [](float x) { return 1.0f / (1.0f + std::exp(-x)); },
                    &slope, &icpt);
    const float m = slope * (sx / sy);
    int32_t q_b = 0, n = 0;
    if (!(std::abs(m) < 1e-12f)) {
      n = static_cast<int8_t>(std::floor(std::log2(static_cast<double>(out_max) / std::abs(m))));
      int64_t q = static_cast<int64_t>(std::rint(static_cast<double>(m) * std::ldexp(1.0, n)));
      q = std::min<int64_t>(std::max<int64_t>(q, -out_max), out_max);
      q_b = static_cast<int32_t>(q);
    }
    lut->seg[s].q_b = q_b;
    lut->seg[s].n = n;
    lut->seg[s].c = static_cast<int32_t>(std::rint(icpt / sy + static_cast<float>(out.zero_point)));
    const int32_t th =
        static_cast<int32_t>(std::rint(pts[s + 1] / sx + static_cast<float>(in.zero_point)));
    lut->seg[s].threshold = std::min(std::max(th, gi.qmin()), gi.qmax());
  }
}

}  // namespace

Bounds bounds_of(int32_t bits, int32_t is_unsigned) {
  const Grid g(bits, is_unsigned);
  Bounds b{static_cast<float>(g.qmin()), static_cast<float>(g.qmax())};
  if (static_cast<double>(b.lo) < static_cast<double>(g.qmin())) b.lo = std::nextafter(b.lo, INFINITY);
  if (static_cast<double>(b.hi) > static_cast<double>(g.qmax())) b.hi = std::nextafter(b.hi, -INFINITY);
  return b;
}

float effective_scale(float scale, bool use_pot2) {
  if (use_pot2) return std::ldexp(1.0f, -static_cast<int>(pow2_exponent(scale)));
  return MShift::encode(scale).decode();
}

static void lut_to_carrier(const rxmet_pwl_lut &l, Lut *o) {
  for (int i = 0; i < kSegments; ++i) {
    o->thr[i] = static_cast<float>(l.seg[i].threshold);
    o->qb[i] = static_cast<float>(l.seg[i].q_b);
    o->n[i] = l.seg[i].n;
    o->c[i] = static_cast<float>(l.seg[i].c);
  }
  o->zp_x = static_cast<float>(l.zp_x);
}

void make_step_params(const rxmet_gru_qparams &p, int H, StepParams *s) {
  const rxmet_grid *g = p.g;
  const bool pot = p.use_pot2 != 0;
  auto zp = [&](int i) { return static_cast<float>(g[i].zero_point); };
  auto sc = [&](int i) { return g[i].scale; };
  s->H = H;
  s->zp_x = zp(RXMET_GRU_X);
  s->zp_h = zp(RXMET_GRU_H);
  s->zp_wx = zp(RXMET_GRU_WX);
  s->zp_rh = zp(RXMET_GRU_RH);
  s->zp_zin = zp(RXMET_GRU_Z_IN);
  s->zp_zout = zp(RXMET_GRU_Z_OUT);
  s->zp_rin = zp(RXMET_GRU_R_IN);
  s->zp_rout = zp(RXMET_GRU_R_OUT);
  s->zp_nin = zp(RXMET_GRU_N_IN);
  s->zp_nout = zp(RXMET_GRU_N_OUT);
  s->ih_to_zin = sc(RXMET_GRU_WX) / sc(RXMET_GRU_Z_IN);
  s->hh_to_zin = sc(RXMET_GRU_RH) / sc(RXMET_GRU_Z_IN);
  s->ih_to_rin = sc(RXMET_GRU_WX) / sc(RXMET_GRU_R_IN);
  s->hh_to_rin = sc(RXMET_GRU_RH) / sc(RXMET_GRU_R_IN);
  s->ih_to_nin = sc(RXMET_GRU_WX) / sc(RXMET_GRU_N_IN);
  s->rmul_to_nin = (sc(RXMET_GRU_R_OUT) * sc(RXMET_GRU_RH)) / sc(RXMET_GRU_N_IN);
  s->quant_one = std::rint(1.0f / sc(RXMET_GRU_Z_OUT)) + zp(RXMET_GRU_Z_OUT);
  s->old_to_h = (sc(RXMET_GRU_Z_OUT) * sc(RXMET_GRU_H)) / sc(RXMET_GRU_H);
  s->nout_to_h = sc(RXMET_GRU_N_OUT) / sc(RXMET_GRU_H);
  auto bnd = [&](int i) { return bounds_of(g[i].bits, g[i].is_unsigned); };
  s->x = bnd(RXMET_GRU_X);
  s->h = bnd(RXMET_GRU_H);
  s->wx = bnd(RXMET_GRU_WX);
  s->rh = bnd(RXMET_GRU_RH);
  s->zin = bnd(RXMET_GRU_Z_IN);
  s->zout = bnd(RXMET_GRU_Z_OUT);
  s->rin = bnd(RXMET_GRU_R_IN);
  s->rout = bnd(RXMET_GRU_R_OUT);
  s->nin = bnd(RXMET_GRU_N_IN);
  s->nout = bnd(RXMET_GRU_N_OUT);
  rxmet_pwl_lut luts[3];
  build_lut(false, g[RXMET_GRU_Z_IN], g[RXMET_GRU_Z_OUT], &luts[0]);
  build_lut(false, g[RXMET_GRU_R_IN], g[RXMET_GRU_R_OUT], &luts[1]);
  build_lut(true, g[RXMET_GRU_N_IN], g[RXMET_GRU_N_OUT], &luts[2]);
  for (int i = 0; i < 3; ++i) lut_to_carrier(luts[i], &s->lut[i]);
  s->eff_x = effective_scale(sc(RXMET_GRU_X), pot);
  s->eff_h = effective_scale(sc(RXMET_GRU_H), pot);
  s->eff_zout = effective_scale(sc(RXMET_GRU_Z_OUT), pot);
  s->eff_rout = effective_scale(sc(RXMET_GRU_R_OUT), pot);
  s->eff_nout = effective_scale(sc(RXMET_GRU_N_OUT), pot);
  s->eff_rh = effective_scale(sc(RXMET_GRU_RH), pot);
}

// ---- int32 carrier ----
// makeRescale / makeRescaleProduct / makeRescaleToProduct (include/scale_encoding.h:133-188):
// power-of-two mode takes differences of the grids' shifts, affine mode encodes the fp32 ratio
// of the stored scales as a 16-bit mantissa and a shift.
static IRescale checked(IRescale r) {
  if (r.shift < -32 || r.shift > 62) throw std::runtime_error("integer rescale shift out of range");
  return r;
}
static IRescale rescale_of(bool pot, float ratio, int pot_shift) {
  if (pot) return checked(IRescale{1, static_cast<int8_t>(pot_shift)});
  const MShift m = MShift::encode(ratio);
  return checked(IRescale{static_cast<int32_t>(m.m), m.shift});
}
static IRescale rs_single(bool pot, float src, float dst) {
  return rescale_of(pot, src / dst, pow2_exponent(src) - pow2_exponent(dst));
}
static IRescale rs_product(bool pot, float a, float b, float dst) {
  return rescale_of(pot, (a * b) / dst, pow2_exponent(a) + pow2_exponent(b) - pow2_exponent(dst));
}
static IRescale rs_to_product(bool pot, float src, float a, float b) {
  return rescale_of(pot, src / (a * b), pow2_exponent(src) - (pow2_exponent(a) + pow2_exponent(b)));
}

IGrid igrid_of(int32_t bits, int32_t is_unsigned) {
  const Grid g(bits, is_unsigned);
  return IGrid{g.qmin(), g.qmax()};
}

void make_int_step_params(const rxmet_gru_qparams &p, int H, IntStepParams *s) {
  const rxmet_grid *g = p.g;
  const bool pot = p.use_pot2 != 0;
  auto sc = [&](int i) { return g[i].scale; };
  s->H = H;
  s->zp_x = g[RXMET_GRU_X].zero_point;
  s->zp_h = g[RXMET_GRU_H].zero_point;
  s->zp_wx = g[RXMET_GRU_WX].zero_point;
  s->zp_rh = g[RXMET_GRU_RH].zero_point;
  s->zp_zin = g[RXMET_GRU_Z_IN].zero_point;
  s->zp_zout = g[RXMET_GRU_Z_OUT].zero_point;
  s->zp_rin = g[RXMET_GRU_R_IN].zero_point;
  s->zp_rout = g[RXMET_GRU_R_OUT].zero_point;
  s->zp_nin = g[RXMET_GRU_N_IN].zero_point;
  s->zp_nout = g[RXMET_GRU_N_OUT].zero_point;
  s->ih_zin = rs_single(pot, sc(RXMET_GRU_WX), sc(RXMET_GRU_Z_IN));
  s->hh_zin = rs_single(pot, sc(RXMET_GRU_RH), sc(RXMET_GRU_Z_IN));
  s->ih_rin = rs_single(pot, sc(RXMET_GRU_WX), sc(RXMET_GRU_R_IN));
  s->hh_rin = rs_single(pot, sc(RXMET_GRU_RH), sc(RXMET_GRU_R_IN));
  s->ih_nin = rs_single(pot, sc(RXMET_GRU_WX), sc(RXMET_GRU_N_IN));
  s->rmul_nin = rs_product(pot, sc(RXMET_GRU_R_OUT), sc(RXMET_GRU_RH), sc(RXMET_GRU_N_IN));
  s->nout_h = rs_single(pot, sc(RXMET_GRU_N_OUT), sc(RXMET_GRU_H));
  s->old_h = rs_product(pot, sc(RXMET_GRU_Z_OUT), sc(RXMET_GRU_H), sc(RXMET_GRU_H));
  // the constant 1 on the update-gate output grid: round_to_int(1 / S) + zp
  s->quant_one = static_cast<int32_t>(static_cast<uint32_t>(static_cast<int32_t>(
                                          std::rint(1.0f / sc(RXMET_GRU_Z_OUT)))) +
                                      static_cast<uint32_t>(s->zp_zout));
  auto ig = [&](int i) { return igrid_of(g[i].bits, g[i].is_unsigned); };
  s->x = ig(RXMET_GRU_X);
  s->h = ig(RXMET_GRU_H);
  s->wx = ig(RXMET_GRU_WX);
  s->rh = ig(RXMET_GRU_RH);
  s->zin = ig(RXMET_GRU_Z_IN);
  s->zout = ig(RXMET_GRU_Z_OUT);
  s->rin = ig(RXMET_GRU_R_IN);
  s->rout = ig(RXMET_GRU_R_OUT);
  s->nin = ig(RXMET_GRU_N_IN);
  s->nout = ig(RXMET_GRU_N_OUT);
  rxmet_pwl_lut luts[3];
  build_lut(false, g[RXMET_GRU_Z_IN], g[RXMET_GRU_Z_OUT], &luts[0]);
  build_lut(false, g[RXMET_GRU_R_IN], g[RXMET_GRU_R_OUT], &luts[1]);
  build_lut(true, g[RXMET_GRU_N_IN], g[RXMET_GRU_N_OUT], &luts[2]);
  for (int i = 0; i < 3; ++i) {
    for (int k = 0; k < kSegments; ++k) {
      s->lut[i].thr[k] = luts[i].seg[k].threshold;
      s->lut[i].qb[k] = luts[i].seg[k].q_b;
      s->lut[i].n[k] = luts[i].seg[k].n;
      s->lut[i].c[k] = luts[i].seg[k].c;
    }
    s->lut[i].zp_x = luts[i].zp_x;
  }
  s->eff_x = effective_scale(sc(RXMET_GRU_X), pot);
  s->eff_h = effective_scale(sc(RXMET_GRU_H), pot);
  s->eff_zout = effective_scale(sc(RXMET_GRU_Z_OUT), pot);
  s->eff_rout = effective_scale(sc(RXMET_GRU_R_OUT), pot);
  s->eff_nout = effective_scale(sc(RXMET_GRU_N_OUT), pot);
  s->eff_rh = effective_scale(sc(RXMET_GRU_RH), pot);
}

void make_int_channel_rescales(const rxmet_gru_qparams &p, int H, IRescale *rs) {
  const bool pot = p.use_pot2 != 0;
  const int C = 3 * H;
  const float sx = p.g[RXMET_GRU_X].scale, sh = p.g[RXMET_GRU_H].scale;
  const float swx = p.g[RXMET_GRU_WX].scale, srh = p.g[RXMET_GRU_RH].scale;
  for (int c = 0; c < C; ++c) {
    const float sW = p.chan_scale[RXMET_GRU_W][c], sR = p.chan_scale[RXMET_GRU_R][c];
    rs[c] = rs_product(pot, sW, sx, swx);
    rs[C + c] = rs_to_product(pot, p.chan_scale[RXMET_GRU_BW][c], sW, sx);
    rs[2 * C + c] = rs_product(pot, sR, sh, srh);
    rs[3 * C + c] = rs_to_product(pot, p.chan_scale[RXMET_GRU_BR][c], sR, sh);
  }
}

void make_channel_factors(const rxmet_gru_qparams &p, int H, float *igx, float *ibx, float *igh,
                          float *ibh, float *eff_w, float *eff_r, float *eff_bw, float *eff_br) {
  const bool pot = p.use_pot2 != 0;
  const float sx = p.g[RXMET_GRU_X].scale, sh = p.g[RXMET_GRU_H].scale;
  const float swx = p.g[RXMET_GRU_WX].scale, srh = p.g[RXMET_GRU_RH].scale;
  for (int c = 0; c < 3 * H; ++c) {
    const float gemm_x = p.chan_scale[RXMET_GRU_W][c] * sx;
    igx[c] = gemm_x / swx;
    ibx[c] = p.chan_scale[RXMET_GRU_BW][c] / gemm_x;
    const float gemm_h = p.chan_scale[RXMET_GRU_R][c] * sh;
    igh[c] = gemm_h / srh;
    ibh[c] = p.chan_scale[RXMET_GRU_BR][c] / gemm_h;
    eff_w[c] = effective_scale(p.chan_scale[RXMET_GRU_W][c], pot);
    eff_r[c] = effective_scale(p.chan_scale[RXMET_GRU_R][c], pot);
    eff_bw[c] = effective_scale(p.chan_scale[RXMET_GRU_BW][c], pot);
    eff_br[c] = effective_scale(p.chan_scale[RXMET_GRU_BR][c], pot);
  }
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int rxmet_gru_make_params(const rxmet_gru_ranges *r, const rxmet_gru_config *cfg,
                          rxmet_gru_qparams *out) {
  clear_error();
  RXMET_CHECK_ARG(r && cfg && out, "null argument");
  RXMET_CHECK_ARG(r->hidden > 0, "hidden size must be positive");
  for (int k = 0; k < RXMET_GRU_NCHAN; ++k) {
    RXMET_CHECK_ARG(cfg->chan[k].symmetric,
                    "W/R/bw/br must remain symmetric (zero point 0): asymmetric weight or bias "
                    "quantisation is not supported");
    RXMET_CHECK_ARG(r->chan_min[k] && r->chan_max[k] && out->chan_scale[k],
                    "per-channel range/scale arrays must be provided");
  }
  try {
    const int H = r->hidden, C = 3 * H;
    out->hidden = H;
    out->use_pot2 = cfg->use_pot2;
    for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
      float lo = r->min[i], hi = r->max[i];
      if (i == RXMET_GRU_Z_OUT || i == RXMET_GRU_R_OUT || i == RXMET_GRU_N_OUT) {
        // gate outputs span at least 0.5 around their centre
        if (hi - lo < 0.5f) {
          const float mid = (lo + hi) / 2.0f;
          lo = mid - 0.5f / 2.0f;
          hi = mid + 0.5f / 2.0f;
        }
      }
      out->g[i] = grid_from_range(lo, hi, cfg->op[i], *cfg);
    }
    for (int k = 0; k < RXMET_GRU_NCHAN; ++k) {
      const rxmet_bitspec &spec = cfg->chan[k];
      const Grid g(spec.bits, spec.is_unsigned);
      out->chan_bits[k] = g.bits;
      out->chan_unsigned[k] = g.uns ? 1 : 0;
      const int group = group_size(spec.granularity, H);
      for (int g0 = 0; g0 < C; g0 += group) {
        float s;
        if (k < 2) {  // weights: scale from the group's min/max
          float lo = r->chan_min[k][g0], hi = r->chan_max[k][g0];
          if (group > 1) {
            lo = *std::min_element(r->chan_min[k] + g0, r->chan_min[k] + g0 + group);
            hi = *std::max_element(r->chan_max[k] + g0, r->chan_max[k] + g0 + group);
          }
          s = grid_from_range(lo, hi, spec, *cfg).scale;
        } else {  // biases: symmetric headroom over the largest magnitude
          double extent = 0.0;
          for (int c = g0; c < g0 + group; ++c) {
            const float lo = r->chan_min[k][c], hi = r->chan_max[k][c];
            RXMET_CHECK_ARG(std::isfinite(lo) && std::isfinite(hi) && lo <= hi,
                            "bias calibration requires finite observations");
            extent = std::max(extent, std::max(std::abs(static_cast<double>(lo)),
                                               std::abs(static_cast<double>(hi))));
          }
          double sd = std::max(2.0 * extent, 0.01) / g.qmax();
          if (cfg->use_pot2) sd = std::exp2(std::ceil(std::log2(sd)));
          RXMET_CHECK_ARG(std::isfinite(sd) && sd <= FLT_MAX, "bias scale exceeds float32 range");
          s = static_cast<float>(sd);
        }
        std::fill(out->chan_scale[k] + g0, out->chan_scale[k] + g0 + group, s);
      }
    }
  } catch (const std::exception &e) {
    set_error(e.what());
    return -22;
  }
  return 0;
}

int rxmet_gru_make_luts(const rxmet_gru_qparams *p, rxmet_pwl_lut out[3]) {
  clear_error();
  RXMET_CHECK_ARG(p && out, "null argument");
  try {
    build_lut(false, p->g[RXMET_GRU_Z_IN], p->g[RXMET_GRU_Z_OUT], &out[0]);
    build_lut(false, p->g[RXMET_GRU_R_IN], p->g[RXMET_GRU_R_OUT], &out[1]);
    build_lut(true, p->g[RXMET_GRU_N_IN], p->g[RXMET_GRU_N_OUT], &out[2]);
  } catch (const std::exception &e) {
    set_error(e.what());
    return -22;
  }
  return 0;
}

float rxmet_gru_effective_scale(float scale, int32_t use_pot2) {
  try {
    return effective_scale(scale, use_pot2 != 0);
  } catch (const std::exception &) {
    return NAN;
  }
}

}  // extern "C"
