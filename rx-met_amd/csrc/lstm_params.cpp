// lstm_params.cpp — QuantLSTM quantisation parameters on the host: MinMax finalisation
// from device statistics and the execution encodings the kernels consume.
//
// Semantics follow the reference (operators/quant-lstm/): integer grids
// (include/quantization/bit_width.h:23-58), calibrateMinMax and the minimum-scale
// fallback (src/quantization/scale_encoding.cc:30-103), POT2 CoverRange (:150-185), bias
// headroom and per-granularity expansion (src/lstm/quant_params.cc:24-50, 248-291),
// M+shift with round-to-nearest-even (scale_encoding.cc:105-128), POT2 rescales
// (:134-148), Q31 cell ratios with the mantissa/exponent fallback and fp32 product scales
// (src/lstm/lstm_execution_params.cc:54-77, 236-328).
#include <cfloat>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>

#include "lstm_internal.h"
#include "rxmet_common.h"

namespace rxmet {
namespace lstm {
namespace {

constexpr int kNops = RXMET_LSTM_NOPS;

bool is_param(int op) { return op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH; }
bool is_bias(int op) { return op == RXMET_LSTM_B_IH || op == RXMET_LSTM_B_HH; }

int check_type(const rxmet_lstm_op_config &t, int op) {
  if (t.bits < 1 || t.bits > 32) return -1;
  if (t.is_unsigned && t.bits == 32) return -1;
  if (!t.is_unsigned && t.is_symmetric && t.bits == 1) return -1;
  if (is_param(op) && (t.is_unsigned || !t.is_symmetric)) return -2;
  if (!is_param(op) && t.granularity != RXMET_LSTM_PER_TENSOR) return -3;
  if (t.granularity < 0 || t.granularity > 2) return -3;
  return 0;
}

void int_range(const rxmet_lstm_op_config &t, int32_t *lo, int32_t *hi) {
  if (t.is_unsigned) {
    *lo = 0;
    *hi = static_cast<int32_t>((uint64_t{1} << t.bits) - 1u);
  } else {
    const auto m = static_cast<int32_t>((uint64_t{1} << (t.bits - 1)) - 1u);
    *lo = -m - 1;
    *hi = m;
  }
}

int32_t zero_point(float lower, float scale, int32_t lo, int32_t hi) {
  const double cand = static_cast<double>(lo) - static_cast<double>(lower) / scale;
  if (cand <= lo) return lo;
  if (cand >= hi) return hi;
  double r = std::nearbyint(cand);
  return static_cast<int32_t>(r < lo ? lo : (r > hi ? hi : r));
}

struct Calibrated {
  float scale;
  int32_t zp;
  float adj_lo, adj_hi;
};

// MinMax -> (scale, zero point); POT2 CoverRange; bias headroom.
bool calibrate(float rmin, float rmax, const rxmet_lstm_op_config &t, bool pot2, bool bias,
               Calibrated *out) {
  if (!std::isfinite(rmin) || !std::isfinite(rmax) || rmin > rmax) return false;
  int32_t lo, hi;
  int_range(t, &lo, &hi);
  const double steps = static_cast<double>(hi) - lo;
  const float min_scale = static_cast<float>(std::fmin(std::ldexp(1.0, -23), 0.01 / steps));
  double cand;
  if (t.is_symmetric && !t.is_unsigned) {
    cand = std::fmax(std::fabs(static_cast<double>(rmin)), std::fabs(static_cast<double>(rmax))) / hi;
  } else if (t.is_symmetric) {
    cand = static_cast<double>(std::fmax(rmax, 0.0f)) / hi;
  } else {
    cand = (static_cast<double>(std::fmax(rmax, 0.0f)) - std::fmin(rmin, 0.0f)) / steps;
  }
  const float scale = cand < static_cast<double>(min_scale) ? min_scale : static_cast<float>(cand);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return false;
  Calibrated c;
  c.scale = scale;
  if (t.is_symmetric && !t.is_unsigned) {
    c.adj_hi = static_cast<float>(hi) * scale;
    c.adj_lo = -c.adj_hi;
  } else if (t.is_symmetric) {
    c.adj_lo = 0.0f;
    c.adj_hi = static_cast<float>(hi) * scale;
  } else {
    c.adj_lo = std::fmin(rmin, 0.0f);
    c.adj_hi = c.adj_lo + static_cast<float>(steps) * scale;
  }
  c.zp = t.is_symmetric ? 0 : zero_point(c.adj_lo, scale, lo, hi);
  if (pot2) {
    const double range = std::fabs(static_cast<double>(c.adj_hi) - c.adj_lo);
    if (!std::isfinite(range) || range <= 0.0) return false;
    const double near_pow = std::ldexp(1.0, static_cast<int>(std::nearbyint(std::log2(range))));
    const bool near = std::fabs(range - near_pow) / near_pow < 0.02;
    const double ev = -std::log2(static_cast<double>(c.scale));
    const double e = near ? std::nearbyint(ev) : std::floor(ev);
    if (!std::isfinite(e) || e < -128 || e > 127) return false;
    c.scale = static_cast<float>(std::ldexp(1.0, -static_cast<int>(e)));
    c.zp = t.is_symmetric ? 0 : zero_point(c.adj_lo, c.scale, lo, hi);
  }
  if (bias) {
    const double ext = std::fmax(std::fabs(static_cast<double>(rmin)), std::fabs(static_cast<double>(rmax)));
    double s = std::fmax(2.0 * ext, 0.01) / hi;
    if (pot2) s = std::exp2(std::ceil(std::log2(s)));
    if (!std::isfinite(s) || s > FLT_MAX) return false;
    c.scale = static_cast<float>(s);
  }
  *out = c;
  return true;
}

bool mshift(double ratio, Rescale *r) {
  if (!std::isfinite(ratio) || ratio <= 0.0) return false;
  int e = 0;
  const double m = std::frexp(ratio, &e);
  auto mult = static_cast<int64_t>(std::nearbyint(m * 65536.0));
  if (mult == 65536) {
    mult = 32768;
    ++e;
  }
  const int shift = 16 - e;
  if (mult < 32768 || mult > 65535 || shift < -128 || shift > 127) return false;
  r->mult = static_cast<float>(mult);
  r->shift = shift;
  return true;
}

bool pot2_rescale(float src, float dst, Rescale *r) {
  int es = 0, ed = 0;
  if (std::frexp(src, &es) != 0.5f || std::frexp(dst, &ed) != 0.5f) return false;
  const int shift = ed - es;
  if (shift < -128 || shift > 127) return false;
  r->mult = 1.0f;
  r->shift = shift;
  return true;
}

bool encode(bool pot2, float src, float dst, Rescale *r) {
  return pot2 ? pot2_rescale(src, dst, r) : mshift(static_cast<double>(src) / dst, r);
}

float product_scale(float a, float b) { return static_cast<float>(static_cast<double>(a) * b); }

void cell_ratio(double ratio, float *r, int64_t *q31, double *mant, int32_t *ex, int32_t *fp) {
  const double s = std::ldexp(ratio, 31);
  *mant = 0.0;
  *ex = 0;
  *fp = 0;
  *r = 0.0f;
  *q31 = 0;
  if (std::isfinite(s) && s > 0.5 && s < 9.2233720368547758e18) {
    *q31 = static_cast<int64_t>(std::nearbyint(s));
    *r = std::ldexp(static_cast<float>(*q31), -31);  // fl((float)multiplier) * 2^-31
    return;
  }
  int e = 0;
  *mant = std::frexp(ratio, &e);
  *ex = e;
  *fp = 1;
}

// The activation's input and output grids: k < 4 gate k, k == 4 tanh of the cell.
void act_grids(const StepParams &sp, int k, const Grid **in, const Grid **out, bool *is_tanh) {
  *in = k < 4 ? &sp.gin[k] : &sp.c;
  *out = k < 4 ? &sp.gout[k] : &sp.tanh_c;
  *is_tanh = k == 2 || k == 4;
}

// realSigmoid / realTanh of the reference (quantized_fp_math.cuh:21-30) on the host: the C
// library's expf and tanhf in fp32.
float sigmoid_libm(float x) {
  if (x >= 0.0f) {
    const float e = ::expf(-x);
    return 1.0f / (1.0f + e);
  }
  const float e = ::expf(x);
  return e / (1.0f + e);
}

// The kernels' form: exp and tanh in double, rounded once to fp32, same op order around exp.
float sigmoid_dbl(float x) {
  if (x >= 0.0f) {
    const float e = static_cast<float>(std::exp(-static_cast<double>(x)));
    return 1.0f / (1.0f + e);
  }
  const float e = static_cast<float>(std::exp(static_cast<double>(x)));
  return e / (1.0f + e);
}

struct ActCacheEntry {
  std::vector<double> key;
  ActExceptions ex;
};

}  // namespace

uint32_t act_entry(const StepParams &sp, int k, int32_t q, bool reference) {
  const Grid *in, *out;
  bool is_tanh;
  act_grids(sp, k, &in, &out, &is_tanh);
  // realActivationQuantizedCore (quantized_fp_math.cuh:32-63): dequantise in double,
  // activate in fp32, RNE of the double quotient plus the zero point, clamp to the grid.
  const float x = static_cast<float>((static_cast<double>(q) - in->dzp) * in->dscale);
  const float a = is_tanh ? (reference ? ::tanhf(x) : static_cast<float>(std::tanh(static_cast<double>(x))))
                          : (reference ? sigmoid_libm(x) : sigmoid_dbl(x));
  const double t = std::nearbyint(static_cast<double>(a) / out->dscale) + out->dzp;
  const uint32_t m = (t < out->dlo || t > out->dhi) ? 1u : 0u;
  const double v = t <= out->dflo ? out->flo : (t >= out->dfhi ? out->fhi : t);
  return (static_cast<uint32_t>(static_cast<int64_t>(v) - out->lo) << 1) | m;
}

ActExceptions act_exceptions(const StepParams &sp) {
  std::vector<double> key;
  for (int k = 0; k < 5; ++k) {
    const Grid *in, *out;
    bool is_tanh;
    act_grids(sp, k, &in, &out, &is_tanh);
    for (const Grid *g : {in, out}) {
      key.push_back(g->lo);
      key.push_back(g->hi);
      key.push_back(g->scale);
      key.push_back(g->zp);
    }
  }
  static std::mutex mu;
  static std::vector<ActCacheEntry> cache;  // most recent last; a handful of parameter sets
  std::lock_guard<std::mutex> lock(mu);
  for (size_t i = 0; i < cache.size(); ++i)
    if (cache[i].key == key) return cache[i].ex;
  ActCacheEntry e;
  e.key = key;
  for (int k = 0; k < 5; ++k) {
    const Grid *in, *out;
    bool is_tanh;
    act_grids(sp, k, &in, &out, &is_tanh);
    e.ex.off[k] = static_cast<int32_t>(e.ex.key.size());
    const int64_t ncodes = static_cast<int64_t>(in->hi) - in->lo + 1;
    if (ncodes <= kActExcMaxCodes)
      for (int64_t q = in->lo; q <= in->hi; ++q) {
        const uint32_t r = act_entry(sp, k, static_cast<int32_t>(q), true);
        if (r != act_entry(sp, k, static_cast<int32_t>(q), false)) {
          e.ex.key.push_back(static_cast<int32_t>(q));
          e.ex.val.push_back(r);
        }
      }
    e.ex.n[k] = static_cast<int32_t>(e.ex.key.size()) - e.ex.off[k];
  }
  if (cache.size() >= 8) cache.erase(cache.begin());
  cache.push_back(std::move(e));
  return cache.back().ex;
}

Grid grid_of(const rxmet_lstm_op_config &t, float scale, int32_t zp) {
  Grid g;
  int_range(t, &g.lo, &g.hi);
  const float el = static_cast<float>(g.lo), eh = static_cast<float>(g.hi);
  g.flo = static_cast<double>(el) < g.lo ? std::nextafter(el, INFINITY) : el;
  g.fhi = static_cast<double>(eh) > g.hi ? std::nextafter(eh, -INFINITY) : eh;
  g.scale = scale;
  g.zp = zp;
  g.dlo = g.lo;
  g.dhi = g.hi;
  g.dflo = g.flo;
  g.dfhi = g.fhi;
  g.dscale = scale;
  g.dzp = zp;
  return g;
}

int derive(const rxmet_lstm_params &p, StepParams *sp, ChannelParams *cp) {
  const int H = p.hidden, C = 4 * H;
  const rxmet_lstm_op_config *op = p.config.op;
  for (int i = 0; i < kNops; ++i)
    RXMET_CHECK_ARG(check_type(op[i], i) == 0, "invalid QuantLSTM operator configuration");
  for (int i = 0; i < kNops; ++i)
    if (!is_param(i))
      RXMET_CHECK_ARG(std::isfinite(p.scale[i]) && p.scale[i] > 0.0f,
                      "QuantLSTM standard scales must be finite and positive");
  const bool pot2 = p.config.scale_mode == RXMET_LSTM_POT2;
  sp->exc_key = nullptr;
  sp->exc_val = nullptr;
  for (int k = 0; k < 5; ++k) sp->exc_off[k] = sp->exc_n[k] = 0;
  auto G = [&](int i) { return grid_of(op[i], p.scale[i], p.zero_point[i]); };
  sp->x = G(RXMET_LSTM_INPUT);
  sp->h = G(RXMET_LSTM_OUTPUT);
  sp->c = G(RXMET_LSTM_CELL_STATE);
  sp->ih_lin = G(RXMET_LSTM_IH_LINEAR);
  sp->hh_lin = G(RXMET_LSTM_HH_LINEAR);
  sp->tanh_c = G(RXMET_LSTM_CELL_TANH);
  for (int g = 0; g < 4; ++g) {
    sp->gin[g] = G(RXMET_LSTM_I_GATE_IN + g);
    sp->gout[g] = G(RXMET_LSTM_I_GATE_OUT + g);
    RXMET_CHECK_ARG(encode(pot2, p.scale[RXMET_LSTM_IH_LINEAR], sp->gin[g].scale,
                           &sp->ih_to_gate[g]) &&
                        encode(pot2, p.scale[RXMET_LSTM_HH_LINEAR], sp->gin[g].scale,
                               &sp->hh_to_gate[g]),
                    "linear -> gate-input rescale is not encodable");
  }
  const float sc = p.scale[RXMET_LSTM_CELL_STATE];
  cell_ratio(static_cast<double>(p.scale[RXMET_LSTM_F_GATE_OUT]) * sc / sc, &sp->cell_ratio[0],
             &sp->cell_q31[0], &sp->cell_mant[0], &sp->cell_exp[0], &sp->cell_fp[0]);
  cell_ratio(static_cast<double>(p.scale[RXMET_LSTM_I_GATE_OUT]) * p.scale[RXMET_LSTM_G_GATE_OUT] / sc,
             &sp->cell_ratio[1], &sp->cell_q31[1], &sp->cell_mant[1], &sp->cell_exp[1],
             &sp->cell_fp[1]);
  RXMET_CHECK_ARG(encode(pot2, product_scale(p.scale[RXMET_LSTM_O_GATE_OUT], p.scale[RXMET_LSTM_CELL_TANH]),
                         p.scale[RXMET_LSTM_OUTPUT], &sp->hidden),
                  "hidden rescale is not encodable");
  if (!cp) return 0;
  cp->w_ih_scale.assign(p.chan_scale[0], p.chan_scale[0] + C);
  cp->w_hh_scale.assign(p.chan_scale[1], p.chan_scale[1] + C);
  cp->b_ih_scale.assign(C, 0.0f);
  cp->b_hh_scale.assign(C, 0.0f);
  if (p.bias_enabled) {
    cp->b_ih_scale.assign(p.chan_scale[2], p.chan_scale[2] + C);
    cp->b_hh_scale.assign(p.chan_scale[3], p.chan_scale[3] + C);
  }
  cp->ih_acc_to_lin.resize(C);
  cp->hh_acc_to_lin.resize(C);
  cp->ih_bias_to_acc.assign(C, Rescale{0.0f, 0});
  cp->hh_bias_to_acc.assign(C, Rescale{0.0f, 0});
  for (int c = 0; c < C; ++c) {
    const float ai = product_scale(sp->x.scale, cp->w_ih_scale[c]);
    const float ah = product_scale(sp->h.scale, cp->w_hh_scale[c]);
    RXMET_CHECK_ARG(cp->w_ih_scale[c] > 0.0f && cp->w_hh_scale[c] > 0.0f,
                    "weight scales must be positive");
    RXMET_CHECK_ARG(encode(pot2, ai, sp->ih_lin.scale, &cp->ih_acc_to_lin[c]) &&
                        encode(pot2, ah, sp->hh_lin.scale, &cp->hh_acc_to_lin[c]),
                    "accumulator -> linear rescale is not encodable");
    if (p.bias_enabled) {
      RXMET_CHECK_ARG(cp->b_ih_scale[c] > 0.0f && cp->b_hh_scale[c] > 0.0f,
                      "bias scales must be positive");
      RXMET_CHECK_ARG(encode(pot2, cp->b_ih_scale[c], ai, &cp->ih_bias_to_acc[c]) &&
                          encode(pot2, cp->b_hh_scale[c], ah, &cp->hh_bias_to_acc[c]),
                      "bias -> accumulator rescale is not encodable");
    }
  }
  return 0;
}

}  // namespace lstm
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::lstm;

extern "C" {

int64_t rxmet_lstm_stats_size(int32_t hidden) {
  return 2 * RXMET_LSTM_NOPS + 8 * 4 * static_cast<int64_t>(hidden) + 1;
}

int rxmet_lstm_finalize_params(const float *stats, const rxmet_lstm_config *config, int32_t H,
                               int32_t bias, rxmet_lstm_params *p) {
  clear_error();
  RXMET_CHECK_ARG(stats && config && p && H > 0, "invalid arguments");
  for (int i = 0; i < kNops; ++i)
    RXMET_CHECK_ARG(check_type(config->op[i], i) == 0,
                    "invalid QuantLSTM configuration: weights/biases must be signed symmetric, "
                    "activations per-tensor, bit widths 1..32 (no UINT32, no signed symmetric INT1)");
  RXMET_CHECK_ARG(stats[rxmet_lstm_stats_size(H) - 1] == 0.0f,
                  "calibration values must be finite FP32 (non-finite samples were observed)");
  const int C = 4 * H;
  const bool pot2 = config->scale_mode == RXMET_LSTM_POT2;
  p->hidden = H;
  p->bias_enabled = bias ? 1 : 0;
  p->config = *config;
  for (int i = 0; i < kNops; ++i) {
    const auto &t = config->op[i];
    p->scale[i] = 0.0f;
    p->zero_point[i] = 0;
    if (!is_param(i)) {
      Calibrated c;
      RXMET_CHECK_ARG(calibrate(stats[i], stats[kNops + i], t, pot2, false, &c),
                      std::string("calibration range of operator ") + std::to_string(i) +
                          " is empty or not encodable");
      p->scale[i] = c.scale;
      p->zero_point[i] = c.zp;
      continue;
    }
    if (is_bias(i) && !bias) continue;
    RXMET_CHECK_ARG(p->chan_scale[i - RXMET_LSTM_W_IH] != nullptr, "chan_scale array missing");
    const float *mn = stats + 2 * kNops + static_cast<size_t>(i - RXMET_LSTM_W_IH) * 2 * C;
    const float *mx = mn + C;
    const int groups = t.granularity == RXMET_LSTM_PER_TENSOR ? 1
                       : t.granularity == RXMET_LSTM_PER_GATE ? 4 : C;
    const int span = C / groups;
    for (int g = 0; g < groups; ++g) {
      float lo = INFINITY, hi = -INFINITY;
      for (int c = g * span; c < (g + 1) * span; ++c) {
        lo = std::fmin(lo, mn[c]);
        hi = std::fmax(hi, mx[c]);
      }
      Calibrated cg;
      RXMET_CHECK_ARG(calibrate(lo, hi, t, pot2, is_bias(i), &cg),
                      "parameter calibration range is empty or not encodable");
      for (int c = g * span; c < (g + 1) * span; ++c) p->chan_scale[i - RXMET_LSTM_W_IH][c] = cg.scale;
    }
  }
  return 0;
}

int rxmet_lstm_derive_exec(const rxmet_lstm_params *p, int32_t input_size,
                           rxmet_lstm_rescale *acc_to_linear, rxmet_lstm_rescale *bias_to_acc,
                           rxmet_lstm_rescale *linear_to_gate, rxmet_lstm_q31 *cell,
                           rxmet_lstm_rescale *hidden_rescale) {
  clear_error();
  RXMET_CHECK_ARG(p && input_size > 0, "invalid arguments");
  StepParams sp;
  ChannelParams cp;
  if (int rc = derive(*p, &sp, &cp)) return rc;
  const bool pot2 = p->config.scale_mode == RXMET_LSTM_POT2;
  auto put = [&](const Rescale &r, rxmet_lstm_rescale *o) {
    o->is_mshift = pot2 ? 0 : 1;
    o->multiplier = pot2 ? 0 : static_cast<int32_t>(r.mult);
    o->shift = r.shift;
  };
  const int C = 4 * p->hidden;
  for (int c = 0; c < C; ++c) {
    if (acc_to_linear) {
      put(cp.ih_acc_to_lin[c], &acc_to_linear[c]);
      put(cp.hh_acc_to_lin[c], &acc_to_linear[C + c]);
    }
    if (bias_to_acc && p->bias_enabled) {
      put(cp.ih_bias_to_acc[c], &bias_to_acc[c]);
      put(cp.hh_bias_to_acc[c], &bias_to_acc[C + c]);
    }
  }
  for (int g = 0; g < 4 && linear_to_gate; ++g) {
    put(sp.ih_to_gate[g], &linear_to_gate[g]);
    put(sp.hh_to_gate[g], &linear_to_gate[4 + g]);
  }
  for (int k = 0; k < 2 && cell; ++k) {
    cell[k].uses_fp = sp.cell_fp[k];
    cell[k].mantissa = sp.cell_mant[k];
    cell[k].exponent = sp.cell_exp[k];
    cell[k].multiplier = sp.cell_q31[k];
  }
  if (hidden_rescale) put(sp.hidden, hidden_rescale);
  return 0;
}

int32_t rxmet_lstm_activation_table(const rxmet_lstm_params *p, int32_t k, int32_t reference,
                                    uint32_t *entries, int32_t capacity) {
  clear_error();
  RXMET_CHECK_ARG(p && entries && k >= 0 && k < 5, "invalid arguments");
  StepParams sp;
  if (int rc = derive(*p, &sp, nullptr)) return rc;
  const Grid &in = k < 4 ? sp.gin[k] : sp.c;
  const int64_t n = static_cast<int64_t>(in.hi) - in.lo + 1;
  RXMET_CHECK_ARG(n <= kActExcMaxCodes && n <= capacity,
                  "input grid wider than 65536 codes or capacity too small");
  for (int64_t i = 0; i < n; ++i)
    entries[i] = act_entry(sp, k, static_cast<int32_t>(in.lo + i), reference != 0);
  return static_cast<int32_t>(n);
}

int32_t rxmet_lstm_activation_exceptions(const rxmet_lstm_params *p, int32_t *keys,
                                         uint32_t *entries, int32_t capacity, int32_t *off,
                                         int32_t *n) {
  clear_error();
  RXMET_CHECK_ARG(p && off && n && capacity >= 0 && (capacity == 0 || (keys && entries)),
                  "invalid arguments");
  StepParams sp;
  if (int rc = derive(*p, &sp, nullptr)) return rc;
  const ActExceptions ex = act_exceptions(sp);
  for (int k = 0; k < 5; ++k) {
    off[k] = ex.off[k];
    n[k] = ex.n[k];
  }
  const size_t m = ex.key.size() < static_cast<size_t>(capacity) ? ex.key.size()
                                                                 : static_cast<size_t>(capacity);
  for (size_t i = 0; i < m; ++i) {
    keys[i] = ex.key[i];
    entries[i] = ex.val[i];
  }
  return static_cast<int32_t>(ex.key.size());
}

}  // extern "C"
