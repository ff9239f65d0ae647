/*
 * lstm_oracle.c — CPU restatement of the reference QuantLSTM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker; the product (rx-met_amd/) never calls it.
 *
 * Follows (operators/quant-lstm/ in the reference):
 *   - integer grids (include/quantization/bit_width.h:23-58) and the float-carrier
 *     endpoints / clamps (include/quantization/float_carrier_ops.h:16-44);
 *   - MinMax calibration, minimum scale, zero point (src/quantization/scale_encoding.cc:
 *     12-103), POT2 CoverRange (:150-185), bias headroom and per-granularity expansion
 *     (src/lstm/quant_params.cc:24-50, 248-291);
 *   - execution encodings: M+shift with RNE (scale_encoding.cc:105-128), POT2 rescale
 *     (:134-148), Q31 cell ratios with the frexp fallback (src/lstm/lstm_execution_params.cc:
 *     61-77, 277-287), product scales in fp32 (:54-60);
 *   - the FP32 q-carrier forward (src/lstm/forward_quantized_fp_cpu.cc:20-197) with the
 *     real activation boundary (src/lstm/cuda/quantized_fp_math.cuh:21-71), cell and hidden
 *     fusion (include/lstm/quantized_cell_fp.h:78-150) and the clamp masks of the CUDA
 *     path (src/lstm/forward_quantized_fp_cuda.cu:533-548, 731-858);
 *   - the float forward used for calibration (src/lstm/forward_float_cpu.cc:57-153) and
 *     the observed operators (src/lstm/calibration.cc:154-240);
 *   - the STE backward (lstm_interface_binding.cc:384-480 dequantisation,
 *     src/lstm/backward_float_cuda.cu:50-104 pointwise with masks, :286-327 GEMMs and
 *     masks) with GEMM sums accumulated in double.
 *
 * Modes: ACT_LIBM evaluates sigmoid/tanh with the C library's expf/tanhf in the
 * reference's float op order and accumulates each linear's centred integer products in
 * float in index order (the reference CPU semantics, pinned against the reference compiled
 * into oracle/_ref); ACT_CR evaluates exp and tanh in double and rounds once to float
 * (correctly rounded apart from double-rounding ties), keeping the same float op order
 * around them, and sums each linear's products exactly (one rounding to float at the end);
 * ACT_LIBM_EXACT takes ACT_LIBM's activations with ACT_CR's exact sums, which is what the GPU
 * kernels compute.  The two sums agree while every partial sum stays below 2^24 (all 8-bit h
 * configurations); past that the reference's own result depends on its GEMM's summation
 * order.
 *
 * Pinning (tests/test_lstm_oracle.py): the reference's golden vectors
 * (the JSON files in tests/golden/lstm, copied data from the reference tests/golden/spec) for
 * primitives, one cell step and a 3-step recurrence; parameters, execution encodings,
 * q-carrier forward and float forward against oracle/_ref; the float forward against
 * torch.nn.LSTM; the backward against torch autograd through an STE surrogate.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/rxmet_lstm.h"

enum { ACT_LIBM = 0, ACT_CR = 1, ACT_LIBM_EXACT = 2 };

/* ------------------------------------------------------------------------------ */
/* Grids and rounding                                                              */
/* ------------------------------------------------------------------------------ */

static void grid_range(const rxmet_lstm_op_config *t, int32_t *lo, int32_t *hi) {
  if (t->is_unsigned) {
    *lo = 0;
    *hi = (int32_t)((1ull << t->bits) - 1ull);
  } else {
    const int32_t m = (int32_t)((1ull << (t->bits - 1)) - 1ull);
    *lo = -m - 1;
    *hi = m;
  }
}

static double rne(double v) { return rint(v); }  /* default rounding mode: ties to even */
static float rnef(float v) { return rintf(v); }

static float carrier_min(int32_t m) {
  const float e = (float)m;
  return (double)e < (double)m ? nextafterf(e, INFINITY) : e;
}
static float carrier_max(int32_t m) {
  const float e = (float)m;
  return (double)e > (double)m ? nextafterf(e, -INFINITY) : e;
}
static float clamp_carrier(double v, int32_t lo, int32_t hi) {
  const float l = carrier_min(lo), h = carrier_max(hi);
  return v <= (double)l ? l : (v >= (double)h ? h : (float)v);
}
static float center(float v, int32_t zp) { return (float)((double)v - zp); }

/* Sum of w[k] * (x[k] - zx) over k: in float in index order, as linearValue
 * (forward_quantized_fp_cpu.cc:20-45) does, for ACT_LIBM; exactly in 64-bit integers and
 * rounded once to float for ACT_CR and ACT_LIBM_EXACT (the codes are integers, so every
 * product is exact). */
static float linear_sum(const float *w, const float *x, int32_t zx, int K, int mode) {
  if (mode != ACT_LIBM) {
    int64_t s = 0;
    for (int k = 0; k < K; ++k) s += (int64_t)w[k] * ((int64_t)x[k] - zx);
    return (float)s;
  }
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) acc += center(w[k], 0) * center(x[k], zx);
  return acc;
}

/* ------------------------------------------------------------------------------ */
/* Calibration (scale_encoding.cc, quant_params.cc)                                */
/* ------------------------------------------------------------------------------ */

static float minimum_scale(int32_t lo, int32_t hi) {
  const double steps = (double)hi - lo;
  const double a = ldexp(1.0, -23), b = 0.01 / steps;
  return (float)(a < b ? a : b);
}

static int32_t zero_point_of(float lower, float scale, int32_t lo, int32_t hi) {
  const double cand = (double)lo - (double)lower / scale;
  if (cand <= (double)lo) return lo;
  if (cand >= (double)hi) return hi;
  double r = rne(cand);
  if (r < lo) r = lo;
  if (r > hi) r = hi;
  return (int32_t)r;
}

typedef struct {
  float scale;
  int32_t zp;
  float adj_min, adj_max;
} calib_t;

static int calibrate_minmax(float rmin, float rmax, const rxmet_lstm_op_config *t, calib_t *out) {
  if (!isfinite(rmin) || !isfinite(rmax) || rmin > rmax) return -1;
  int32_t lo, hi;
  grid_range(t, &lo, &hi);
  const double steps = (double)hi - lo;
  const float ms = minimum_scale(lo, hi);
  double cand;
  float amin = rmin, amax = rmax;
  if (t->is_symmetric && !t->is_unsigned) {
    const double a = fabs((double)rmin) > fabs((double)rmax) ? fabs((double)rmin) : fabs((double)rmax);
    cand = a / hi;
  } else if (t->is_symmetric) {
    amin = 0.0f;
    amax = rmax > 0.0f ? rmax : 0.0f;
    cand = (double)amax / hi;
  } else {
    amin = rmin < 0.0f ? rmin : 0.0f;
    amax = rmax > 0.0f ? rmax : 0.0f;
    cand = ((double)amax - amin) / steps;
  }
  const int fb = cand < (double)ms;
  const float scale = fb ? ms : (float)cand;
  if (!(scale > 0.0f) || !isfinite(scale)) return -1;
  if (t->is_symmetric && !t->is_unsigned) {
    const float e = (float)hi * scale;
    amin = -e;
    amax = e;
  } else if (t->is_symmetric) {
    amin = 0.0f;
    amax = (float)hi * scale;
  } else {
    amin = rmin < 0.0f ? rmin : 0.0f;
    amax = amin + (float)steps * scale;
  }
  out->scale = scale;
  out->zp = t->is_symmetric ? 0 : zero_point_of(amin, scale, lo, hi);
  out->adj_min = amin;
  out->adj_max = amax;
  return 0;
}

static int pot2_cover_range(calib_t *c, const rxmet_lstm_op_config *t) {
  int32_t lo, hi;
  grid_range(t, &lo, &hi);
  const double range = fabs((double)c->adj_max - (double)c->adj_min);
  if (!isfinite(range) || range <= 0.0) return -1;
  const double l2 = log2(range);
  const int nexp = (int)rne(l2);
  const double npow = ldexp(1.0, nexp);
  const int near = fabs(range - npow) / npow < 0.02;
  const double ev = -log2((double)c->scale);
  const double sel = near ? rne(ev) : floor(ev);
  if (!isfinite(sel) || sel < -128 || sel > 127) return -1;
  const int e = (int)sel;
  c->scale = (float)ldexp(1.0, -e);
  c->zp = t->is_symmetric ? 0 : zero_point_of(c->adj_min, c->scale, lo, hi);
  return 0;
}

static int calibrate_group(float rmin, float rmax, const rxmet_lstm_op_config *t, int pot2,
                           int bias, calib_t *out) {
  if (calibrate_minmax(rmin, rmax, t, out)) return -1;
  if (pot2 && pot2_cover_range(out, t)) return -1;
  if (bias) {
    int32_t lo, hi;
    grid_range(t, &lo, &hi);
    const double ext = fabs((double)rmin) > fabs((double)rmax) ? fabs((double)rmin) : fabs((double)rmax);
    double s = (2.0 * ext > 0.01 ? 2.0 * ext : 0.01) / hi;
    if (pot2) s = exp2(ceil(log2(s)));
    if (!isfinite(s) || s > FLT_MAX) return -1;
    out->scale = (float)s;
    out->adj_min = lo * out->scale;
    out->adj_max = hi * out->scale;
  }
  return 0;
}

static int is_param(int op) { return op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH; }
static int is_bias(int op) { return op == RXMET_LSTM_B_IH || op == RXMET_LSTM_B_HH; }

int64_t olstm_stats_size(int32_t H) { return 2 * RXMET_LSTM_NOPS + 8 * 4 * (int64_t)H + 1; }

int olstm_finalize_params(const float *stats, const rxmet_lstm_config *cfg, int32_t H, int32_t bias,
                          rxmet_lstm_params *p) {
  const int C = 4 * H;
  p->hidden = H;
  p->bias_enabled = bias;
  p->config = *cfg;
  if (stats[olstm_stats_size(H) - 1] != 0.0f) return -2;  /* non-finite samples */
  const int pot2 = cfg->scale_mode == RXMET_LSTM_POT2;
  for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
    const rxmet_lstm_op_config *t = &cfg->op[op];
    if (!is_param(op)) {
      calib_t c;
      if (calibrate_group(stats[op], stats[RXMET_LSTM_NOPS + op], t, pot2, 0, &c)) return -1;
      p->scale[op] = c.scale;
      p->zero_point[op] = c.zp;
      continue;
    }
    const int k = op - RXMET_LSTM_W_IH;
    p->scale[op] = 0.0f;
    p->zero_point[op] = 0;
    if (is_bias(op) && !bias) continue;
    const float *mn = stats + 2 * RXMET_LSTM_NOPS + (size_t)k * 2 * C, *mx = mn + C;
    const int groups = t->granularity == RXMET_LSTM_PER_TENSOR ? 1
                       : t->granularity == RXMET_LSTM_PER_GATE ? 4 : C;
    const int span = C / groups;
    for (int g = 0; g < groups; ++g) {
      float lo = INFINITY, hi = -INFINITY;
      for (int c = g * span; c < (g + 1) * span; ++c) {
        lo = mn[c] < lo ? mn[c] : lo;
        hi = mx[c] > hi ? mx[c] : hi;
      }
      calib_t cg;
      if (calibrate_group(lo, hi, t, pot2, is_bias(op), &cg)) return -1;
      for (int c = g * span; c < (g + 1) * span; ++c) p->chan_scale[k][c] = cg.scale;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Execution encodings (lstm_execution_params.cc)                                   */
/* ------------------------------------------------------------------------------ */

static int encode_mshift(double ratio, rxmet_lstm_rescale *r) {
  if (!isfinite(ratio) || ratio <= 0.0) return -1;
  int e = 0;
  const double m = frexp(ratio, &e);
  int64_t mult = (int64_t)rne(m * 65536.0);
  if (mult == 65536) {
    mult = 32768;
    ++e;
  }
  const int shift = 16 - e;
  if (mult < 32768 || mult > 65535 || shift < -128 || shift > 127) return -1;
  r->is_mshift = 1;
  r->multiplier = (int32_t)mult;
  r->shift = shift;
  return 0;
}

static int encode_pot2(float src, float dst, rxmet_lstm_rescale *r) {
  int es = 0, ed = 0;
  if (frexpf(src, &es) != 0.5f || frexpf(dst, &ed) != 0.5f) return -1;
  const int shift = ed - es;
  if (shift < -128 || shift > 127) return -1;
  r->is_mshift = 0;
  r->multiplier = 0;
  r->shift = shift;
  return 0;
}

static int encode(int pot2, float src, float dst, rxmet_lstm_rescale *r) {
  return pot2 ? encode_pot2(src, dst, r) : encode_mshift((double)src / dst, r);
}

static float product_scale(float a, float b) { return (float)((double)a * b); }

static void encode_cell(double ratio, rxmet_lstm_q31 *q) {
  const double s = ldexp(ratio, 31);
  memset(q, 0, sizeof(*q));
  if (isfinite(s) && s > 0.5 && s < 9.2233720368547758e18) {
    q->multiplier = (int64_t)rne(s);
    return;
  }
  int e = 0;
  q->mantissa = frexp(ratio, &e);
  q->exponent = e;
  q->uses_fp = 1;
}

static float chan_scale(const rxmet_lstm_params *p, int op, int c) {
  return p->chan_scale[op - RXMET_LSTM_W_IH][c];
}

int olstm_derive_exec(const rxmet_lstm_params *p, int32_t I, rxmet_lstm_rescale *acc_to_lin,
                      rxmet_lstm_rescale *bias_to_acc, rxmet_lstm_rescale *lin_to_gate,
                      rxmet_lstm_q31 *cell, rxmet_lstm_rescale *hid) {
  (void)I;
  const int H = p->hidden, C = 4 * H;
  const int pot2 = p->config.scale_mode == RXMET_LSTM_POT2;
  const int in_ops[2] = {RXMET_LSTM_INPUT, RXMET_LSTM_OUTPUT};
  const int w_ops[2] = {RXMET_LSTM_W_IH, RXMET_LSTM_W_HH};
  const int b_ops[2] = {RXMET_LSTM_B_IH, RXMET_LSTM_B_HH};
  const int out_ops[2] = {RXMET_LSTM_IH_LINEAR, RXMET_LSTM_HH_LINEAR};
  for (int l = 0; l < 2; ++l)
    for (int c = 0; c < C; ++c) {
      const float acc = product_scale(p->scale[in_ops[l]], chan_scale(p, w_ops[l], c));
      if (encode(pot2, acc, p->scale[out_ops[l]], &acc_to_lin[l * C + c])) return -1;
      if (p->bias_enabled) {
        if (encode(pot2, chan_scale(p, b_ops[l], c), acc, &bias_to_acc[l * C + c])) return -1;
      } else {
        memset(&bias_to_acc[l * C + c], 0, sizeof(rxmet_lstm_rescale));
      }
    }
  for (int g = 0; g < 4; ++g) {
    if (encode(pot2, p->scale[RXMET_LSTM_IH_LINEAR], p->scale[RXMET_LSTM_I_GATE_IN + g], &lin_to_gate[g]))
      return -1;
    if (encode(pot2, p->scale[RXMET_LSTM_HH_LINEAR], p->scale[RXMET_LSTM_I_GATE_IN + g], &lin_to_gate[4 + g]))
      return -1;
  }
  const float sc = p->scale[RXMET_LSTM_CELL_STATE];
  encode_cell((double)p->scale[RXMET_LSTM_F_GATE_OUT] * sc / sc, &cell[0]);
  encode_cell((double)p->scale[RXMET_LSTM_I_GATE_OUT] * p->scale[RXMET_LSTM_G_GATE_OUT] / sc, &cell[1]);
  if (encode(pot2, product_scale(p->scale[RXMET_LSTM_O_GATE_OUT], p->scale[RXMET_LSTM_CELL_TANH]),
             p->scale[RXMET_LSTM_OUTPUT], hid))
    return -1;
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Primitive arithmetic of the carrier                                              */
/* ------------------------------------------------------------------------------ */

static float apply_rescale(float v, const rxmet_lstm_rescale *r) {
  return r->is_mshift ? rnef(ldexpf(v * (float)r->multiplier, -r->shift)) : rnef(ldexpf(v, -r->shift));
}

static float act_sigmoid(float x, int mode) {
  if (x >= 0.0f) {
    const float e = mode == ACT_CR ? (float)exp(-(double)x) : expf(-x);
    return 1.0f / (1.0f + e);
  }
  const float e = mode == ACT_CR ? (float)exp((double)x) : expf(x);
  return e / (1.0f + e);
}
static float act_tanh(float x, int mode) { return mode == ACT_CR ? (float)tanh((double)x) : tanhf(x); }

/* realActivationQuantizedCore + realActivationCore (quantized_fp_math.cuh:32-71). */
static float real_activation(float q, float s_in, int32_t zp_in, float s_out, int32_t zp_out,
                             const rxmet_lstm_op_config *out_t, int is_tanh, int mode,
                             uint8_t *clamped) {
  int32_t lo, hi;
  grid_range(out_t, &lo, &hi);
  const float x = (float)(((double)q - (double)zp_in) * (double)s_in);
  const float a = is_tanh ? act_tanh(x, mode) : act_sigmoid(x, mode);
  const double t = rne((double)a / (double)s_out) + (double)zp_out;
  double v = t;
  uint8_t c = 0;
  if (t <= (double)lo) {
    c = t < (double)lo;
    v = lo;
  } else if (t >= (double)hi) {
    c = t > (double)hi;
    v = hi;
  }
  if (clamped) *clamped = c;
  return clamp_carrier(v, lo, hi);
}

/* quantizeMasterDevice (forward_quantized_fp_cuda.cu:533-548). */
static float quantize_master(float v, float s, int32_t zp, const rxmet_lstm_op_config *t,
                             uint8_t *clamped) {
  int32_t lo, hi;
  grid_range(t, &lo, &hi);
  const double r = rne((double)v / (double)s) + (double)zp;
  if (clamped) *clamped = r < (double)lo || r > (double)hi;
  return clamp_carrier(r, lo, hi);
}

static float clamp_point(double v, const rxmet_lstm_op_config *t, uint8_t *clamped) {
  int32_t lo, hi;
  grid_range(t, &lo, &hi);
  if (clamped) *clamped = v < (double)lo || v > (double)hi;
  return clamp_carrier(v, lo, hi);
}

static float dequant(float q, float s, int32_t zp) {
  return (float)(((double)q - zp) * (double)s);
}

int olstm_real_activation(float q, float s_in, int32_t zp_in, float s_out, int32_t zp_out,
                          const rxmet_lstm_op_config *out_t, int is_tanh, int mode, float *out,
                          uint8_t *clamped) {
  *out = real_activation(q, s_in, zp_in, s_out, zp_out, out_t, is_tanh, mode, clamped);
  return 0;
}

/* real_activation of every code lo..hi of an input grid (a whole activation table). */
int olstm_real_activation_table(float s_in, int32_t zp_in, int32_t lo, int32_t hi, float s_out,
                                int32_t zp_out, const rxmet_lstm_op_config *out_t, int is_tanh,
                                int mode, float *out, uint8_t *clamped) {
  for (int64_t q = lo; q <= hi; ++q)
    out[q - lo] = real_activation((float)q, s_in, zp_in, s_out, zp_out, out_t, is_tanh, mode,
                                  &clamped[q - lo]);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Quantised FP32-carrier forward                                                   */
/* ------------------------------------------------------------------------------ */

/* Host mirror of rxmet_lstm_saved. */
typedef rxmet_lstm_saved olstm_saved;

int olstm_forward_quant(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                        const float *b_ih, const float *b_hh, const float *x, const float *h0,
                        const float *c0, const rxmet_lstm_params *p, int mode, float *output,
                        float *h_n, float *c_n, const olstm_saved *sv,
                        float *ih_linear, float *hh_linear, float *gate_in /* optional traces */) {
  const int C = 4 * H;
  const rxmet_lstm_op_config *cfg = p->config.op;
  rxmet_lstm_rescale *acc_to_lin = malloc(sizeof(rxmet_lstm_rescale) * 2 * C);
  rxmet_lstm_rescale *bias_to_acc = malloc(sizeof(rxmet_lstm_rescale) * 2 * C);
  rxmet_lstm_rescale lin_to_gate[8], hid;
  rxmet_lstm_q31 cell[2];
  if (olstm_derive_exec(p, I, acc_to_lin, bias_to_acc, lin_to_gate, cell, &hid)) {
    free(acc_to_lin);
    free(bias_to_acc);
    return -1;
  }
  /* masters */
  const size_t nx = (size_t)T * B * I;
  float *xq = malloc(sizeof(float) * nx), *wiq = malloc(sizeof(float) * (size_t)C * I);
  float *whq = malloc(sizeof(float) * (size_t)C * H);
  float *biq = malloc(sizeof(float) * C), *bhq = malloc(sizeof(float) * C);
  float *hs = malloc(sizeof(float) * (size_t)B * H), *cs = malloc(sizeof(float) * (size_t)B * H);
  uint8_t m;
  for (size_t i = 0; i < nx; ++i) {
    xq[i] = quantize_master(x[i], p->scale[RXMET_LSTM_INPUT], p->zero_point[RXMET_LSTM_INPUT],
                            &cfg[RXMET_LSTM_INPUT], &m);
    if (sv) { sv->x_q[i] = xq[i]; sv->x_m[i] = m; }
  }
  for (int c = 0; c < C; ++c) {
    for (int k = 0; k < I; ++k) {
      const size_t i = (size_t)c * I + k;
      wiq[i] = quantize_master(W_ih[i], chan_scale(p, RXMET_LSTM_W_IH, c), 0, &cfg[RXMET_LSTM_W_IH], &m);
      if (sv) { sv->w_ih_q[i] = wiq[i]; sv->w_ih_m[i] = m; }
    }
    for (int k = 0; k < H; ++k) {
      const size_t i = (size_t)c * H + k;
      whq[i] = quantize_master(W_hh[i], chan_scale(p, RXMET_LSTM_W_HH, c), 0, &cfg[RXMET_LSTM_W_HH], &m);
      if (sv) { sv->w_hh_q[i] = whq[i]; sv->w_hh_m[i] = m; }
    }
    if (p->bias_enabled) {
      biq[c] = quantize_master(b_ih[c], chan_scale(p, RXMET_LSTM_B_IH, c), 0, &cfg[RXMET_LSTM_B_IH], &m);
      if (sv) { sv->b_ih_q[c] = biq[c]; sv->b_ih_m[c] = m; }
      bhq[c] = quantize_master(b_hh[c], chan_scale(p, RXMET_LSTM_B_HH, c), 0, &cfg[RXMET_LSTM_B_HH], &m);
      if (sv) { sv->b_hh_q[c] = bhq[c]; sv->b_hh_m[c] = m; }
    }
  }
  for (int i = 0; i < B * H; ++i) {
    uint8_t mh = 0, mc = 0;
    hs[i] = quantize_master(h0 ? h0[i] : 0.0f, p->scale[RXMET_LSTM_OUTPUT],
                            p->zero_point[RXMET_LSTM_OUTPUT], &cfg[RXMET_LSTM_OUTPUT], h0 ? &mh : NULL);
    cs[i] = quantize_master(c0 ? c0[i] : 0.0f, p->scale[RXMET_LSTM_CELL_STATE],
                            p->zero_point[RXMET_LSTM_CELL_STATE], &cfg[RXMET_LSTM_CELL_STATE],
                            c0 ? &mc : NULL);
    if (sv) { sv->h0_q[i] = hs[i]; sv->h0_m[i] = mh; sv->c0_q[i] = cs[i]; sv->c0_m[i] = mc; }
  }

  const int32_t zx = p->zero_point[RXMET_LSTM_INPUT], zh = p->zero_point[RXMET_LSTM_OUTPUT];
  const int32_t zil = p->zero_point[RXMET_LSTM_IH_LINEAR], zhl = p->zero_point[RXMET_LSTM_HH_LINEAR];
  const int32_t zc = p->zero_point[RXMET_LSTM_CELL_STATE], zt = p->zero_point[RXMET_LSTM_CELL_TANH];
  float *gout = malloc(sizeof(float) * C);
  float *hn = malloc(sizeof(float) * (size_t)B * H);
  for (int t = 0; t < T; ++t) {
    for (int b = 0; b < B; ++b) {
      const float *xr = xq + ((size_t)t * B + b) * I;
      const float *hr = hs + (size_t)b * H;
      for (int c = 0; c < C; ++c) {
        const int g = c / H;
        /* linearValue (forward_quantized_fp_cpu.cc:20-45) */
        float acc = linear_sum(wiq + (size_t)c * I, xr, zx, I, mode);
        if (p->bias_enabled) acc += apply_rescale(center(biq[c], 0), &bias_to_acc[c]);
        uint8_t m_il, m_hl, m_gi, m_go;
        const float lin_ih =
            clamp_point((double)apply_rescale(acc, &acc_to_lin[c]) + zil, &cfg[RXMET_LSTM_IH_LINEAR], &m_il);
        acc = linear_sum(whq + (size_t)c * H, hr, zh, H, mode);
        if (p->bias_enabled) acc += apply_rescale(center(bhq[c], 0), &bias_to_acc[C + c]);
        const float lin_hh = clamp_point((double)apply_rescale(acc, &acc_to_lin[C + c]) + zhl,
                                         &cfg[RXMET_LSTM_HH_LINEAR], &m_hl);
        const float lhs = apply_rescale(center(lin_ih, zil), &lin_to_gate[g]);
        const float rhs = apply_rescale(center(lin_hh, zhl), &lin_to_gate[4 + g]);
        const int gin_op = RXMET_LSTM_I_GATE_IN + g, gout_op = RXMET_LSTM_I_GATE_OUT + g;
        const float gi = clamp_point((double)(lhs + rhs) + p->zero_point[gin_op], &cfg[gin_op], &m_gi);
        gout[c] = real_activation(gi, p->scale[gin_op], p->zero_point[gin_op], p->scale[gout_op],
                                  p->zero_point[gout_op], &cfg[gout_op], g == 2, mode, &m_go);
        const size_t ci = ((size_t)t * B + b) * C + c;
        if (ih_linear) ih_linear[ci] = lin_ih;
        if (hh_linear) hh_linear[ci] = lin_hh;
        if (gate_in) gate_in[ci] = gi;
        if (sv) {
          sv->gate_out[ci] = gout[c];
          sv->ih_linear_m[ci] = m_il;
          sv->hh_linear_m[ci] = m_hl;
          sv->gate_in_m[ci] = m_gi;
          sv->gate_out_m[ci] = m_go;
        }
      }
      for (int j = 0; j < H; ++j) {
        const size_t si = (size_t)b * H + j;
        /* computeQuantizedCellFpCore (quantized_cell_fp.h:95-127) */
        const float pf = center(gout[H + j], p->zero_point[RXMET_LSTM_F_GATE_OUT]) * center(cs[si], zc);
        const float pi = center(gout[j], p->zero_point[RXMET_LSTM_I_GATE_OUT]) *
                         center(gout[2 * H + j], p->zero_point[RXMET_LSTM_G_GATE_OUT]);
        float sf, s_i;
        if (cell[0].uses_fp) sf = (float)ldexp((double)pf * cell[0].mantissa, cell[0].exponent);
        else sf = pf * ldexpf((float)cell[0].multiplier, -31);
        if (cell[1].uses_fp) s_i = (float)ldexp((double)pi * cell[1].mantissa, cell[1].exponent);
        else s_i = pi * ldexpf((float)cell[1].multiplier, -31);
        const float sum = sf + s_i;
        uint8_t m_c, m_t, m_h;
        const float cnew = clamp_point((double)rnef(sum) + zc, &cfg[RXMET_LSTM_CELL_STATE], &m_c);
        cs[si] = cnew;
        const float ct = real_activation(cnew, p->scale[RXMET_LSTM_CELL_STATE], zc,
                                         p->scale[RXMET_LSTM_CELL_TANH], zt,
                                         &cfg[RXMET_LSTM_CELL_TANH], 1, mode, &m_t);
        /* computeQuantizedHiddenFpCore (quantized_cell_fp.h:131-144) */
        const float raw = center(gout[3 * H + j], p->zero_point[RXMET_LSTM_O_GATE_OUT]) * center(ct, zt);
        const float hv = clamp_point((double)apply_rescale(raw, &hid) + zh, &cfg[RXMET_LSTM_OUTPUT], &m_h);
        hn[si] = hv;
        const size_t oi = ((size_t)t * B + b) * H + j;
        output[oi] = dequant(hv, p->scale[RXMET_LSTM_OUTPUT], zh);
        if (sv) {
          sv->cell[oi] = cnew;
          sv->cell_tanh[oi] = ct;
          sv->hidden[oi] = hv;
          sv->cell_m[oi] = m_c;
          sv->cell_tanh_m[oi] = m_t;
          sv->hidden_m[oi] = m_h;
        }
      }
    }
    memcpy(hs, hn, sizeof(float) * (size_t)B * H);
  }
  for (int i = 0; i < B * H; ++i) {
    h_n[i] = dequant(hs[i], p->scale[RXMET_LSTM_OUTPUT], zh);
    c_n[i] = dequant(cs[i], p->scale[RXMET_LSTM_CELL_STATE], zc);
  }
  free(acc_to_lin); free(bias_to_acc); free(xq); free(wiq); free(whq); free(biq); free(bhq);
  free(hs); free(cs); free(gout); free(hn);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Float forward + MinMax statistics (forward_float_cpu.cc, calibration.cc)         */
/* ------------------------------------------------------------------------------ */

static void obs(float *mn, float *mx, float *bad, float v) {
  if (!isfinite(v)) { *bad += 1.0f; return; }
  if (v < *mn) *mn = v;
  if (v > *mx) *mx = v;
}

int olstm_forward_float(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                        const float *b_ih, const float *b_hh, const float *x, const float *h0,
                        const float *c0, int mode, float *output, float *h_n, float *c_n,
                        float *stats /* may be null */) {
  const int C = 4 * H;
  float *lin_i = malloc(sizeof(float) * C), *lin_h = malloc(sizeof(float) * C);
  float *gates = malloc(sizeof(float) * C);
  float *mn = stats, *mx = stats ? stats + RXMET_LSTM_NOPS : NULL;
  float *bad = stats ? stats + olstm_stats_size(H) - 1 : NULL;
  for (int i = 0; i < B * H; ++i) {
    h_n[i] = h0 ? h0[i] : 0.0f;
    c_n[i] = c0 ? c0[i] : 0.0f;
    if (stats) {
      obs(&mn[RXMET_LSTM_OUTPUT], &mx[RXMET_LSTM_OUTPUT], bad, h_n[i]);
      obs(&mn[RXMET_LSTM_CELL_STATE], &mx[RXMET_LSTM_CELL_STATE], bad, c_n[i]);
    }
  }
  if (stats) {
    for (size_t i = 0; i < (size_t)T * B * I; ++i) obs(&mn[RXMET_LSTM_INPUT], &mx[RXMET_LSTM_INPUT], bad, x[i]);
    const float *src[4] = {W_ih, W_hh, b_ih, b_hh};
    const int width[4] = {I, H, 1, 1};
    for (int k = 0; k < 4; ++k) {
      if (!src[k]) continue;
      float *cmn = stats + 2 * RXMET_LSTM_NOPS + (size_t)k * 2 * C, *cmx = cmn + C;
      for (int c = 0; c < C; ++c)
        for (int e = 0; e < width[k]; ++e) obs(&cmn[c], &cmx[c], bad, src[k][(size_t)c * width[k] + e]);
    }
  }
  for (int t = 0; t < T; ++t)
    for (int b = 0; b < B; ++b) {
      const float *xr = x + ((size_t)t * B + b) * I;
      float *hr = h_n + (size_t)b * H, *cr = c_n + (size_t)b * H;
      for (int c = 0; c < C; ++c) {
        float li = b_ih ? b_ih[c] : 0.0f, lh = b_hh ? b_hh[c] : 0.0f;
        for (int k = 0; k < I; ++k) li += W_ih[(size_t)c * I + k] * xr[k];
        for (int k = 0; k < H; ++k) lh += W_hh[(size_t)c * H + k] * hr[k];
        lin_i[c] = li;
        lin_h[c] = lh;
        gates[c] = li + lh;
        if (stats) {
          obs(&mn[RXMET_LSTM_IH_LINEAR], &mx[RXMET_LSTM_IH_LINEAR], bad, li);
          obs(&mn[RXMET_LSTM_HH_LINEAR], &mx[RXMET_LSTM_HH_LINEAR], bad, lh);
          obs(&mn[RXMET_LSTM_I_GATE_IN + c / H], &mx[RXMET_LSTM_I_GATE_IN + c / H], bad, gates[c]);
        }
      }
      for (int j = 0; j < H; ++j) {
        const float ig = act_sigmoid(gates[j], mode), fg = act_sigmoid(gates[H + j], mode);
        const float gg = act_tanh(gates[2 * H + j], mode), og = act_sigmoid(gates[3 * H + j], mode);
        const float cn = fg * cr[j] + ig * gg;
        const float ct = act_tanh(cn, mode);
        const float hv = og * ct;
        cr[j] = cn;
        hr[j] = hv;
        output[((size_t)t * B + b) * H + j] = hv;
        if (stats) {
          obs(&mn[RXMET_LSTM_I_GATE_OUT], &mx[RXMET_LSTM_I_GATE_OUT], bad, ig);
          obs(&mn[RXMET_LSTM_F_GATE_OUT], &mx[RXMET_LSTM_F_GATE_OUT], bad, fg);
          obs(&mn[RXMET_LSTM_G_GATE_OUT], &mx[RXMET_LSTM_G_GATE_OUT], bad, gg);
          obs(&mn[RXMET_LSTM_O_GATE_OUT], &mx[RXMET_LSTM_O_GATE_OUT], bad, og);
          obs(&mn[RXMET_LSTM_CELL_STATE], &mx[RXMET_LSTM_CELL_STATE], bad, cn);
          obs(&mn[RXMET_LSTM_CELL_TANH], &mx[RXMET_LSTM_CELL_TANH], bad, ct);
          obs(&mn[RXMET_LSTM_OUTPUT], &mx[RXMET_LSTM_OUTPUT], bad, hv);
        }
      }
    }
  free(lin_i); free(lin_h); free(gates);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* STE backward (backward_float_cuda.cu semantics, double GEMM sums)                */
/* ------------------------------------------------------------------------------ */

static float keep(const uint8_t *m, size_t i) { return (m == NULL || m[i] == 0) ? 1.0f : 0.0f; }

int olstm_backward_quant(int T, int B, int I, int H, const rxmet_lstm_params *p,
                         const olstm_saved *sv, const float *grad_output, const float *grad_h_n,
                         const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                         float *db_ih, float *db_hh, float *dh0, float *dc0) {
  const int C = 4 * H;
  const size_t SB = (size_t)B * H, nx = (size_t)T * B * I;
  /* dequantise masters and checkpoints (dequantizeQCarrierKernel, double) */
  float *xd = malloc(sizeof(float) * nx), *wi = malloc(sizeof(float) * (size_t)C * I);
  float *wh = malloc(sizeof(float) * (size_t)C * H);
  float *h0d = malloc(sizeof(float) * SB), *c0d = malloc(sizeof(float) * SB);
  float *gd = malloc(sizeof(float) * (size_t)T * B * C), *cd = malloc(sizeof(float) * (size_t)T * SB);
  float *td = malloc(sizeof(float) * (size_t)T * SB), *hd = malloc(sizeof(float) * (size_t)T * SB);
  for (size_t i = 0; i < nx; ++i) xd[i] = dequant(sv->x_q[i], p->scale[RXMET_LSTM_INPUT], p->zero_point[RXMET_LSTM_INPUT]);
  for (int c = 0; c < C; ++c) {
    for (int k = 0; k < I; ++k) wi[(size_t)c * I + k] = dequant(sv->w_ih_q[(size_t)c * I + k], chan_scale(p, RXMET_LSTM_W_IH, c), 0);
    for (int k = 0; k < H; ++k) wh[(size_t)c * H + k] = dequant(sv->w_hh_q[(size_t)c * H + k], chan_scale(p, RXMET_LSTM_W_HH, c), 0);
  }
  for (size_t i = 0; i < SB; ++i) {
    h0d[i] = dequant(sv->h0_q[i], p->scale[RXMET_LSTM_OUTPUT], p->zero_point[RXMET_LSTM_OUTPUT]);
    c0d[i] = dequant(sv->c0_q[i], p->scale[RXMET_LSTM_CELL_STATE], p->zero_point[RXMET_LSTM_CELL_STATE]);
  }
  for (size_t r = 0; r < (size_t)T * B; ++r)
    for (int c = 0; c < C; ++c) {
      const int op = RXMET_LSTM_I_GATE_OUT + c / H;
      gd[r * C + c] = dequant(sv->gate_out[r * C + c], p->scale[op], p->zero_point[op]);
    }
  for (size_t i = 0; i < (size_t)T * SB; ++i) {
    cd[i] = dequant(sv->cell[i], p->scale[RXMET_LSTM_CELL_STATE], p->zero_point[RXMET_LSTM_CELL_STATE]);
    td[i] = dequant(sv->cell_tanh[i], p->scale[RXMET_LSTM_CELL_TANH], p->zero_point[RXMET_LSTM_CELL_TANH]);
    hd[i] = dequant(sv->hidden[i], p->scale[RXMET_LSTM_OUTPUT], p->zero_point[RXMET_LSTM_OUTPUT]);
  }
  float *gh = malloc(sizeof(float) * SB), *gc = malloc(sizeof(float) * SB);
  float *dli = malloc(sizeof(float) * (size_t)T * B * C), *dlh = malloc(sizeof(float) * (size_t)T * B * C);
  for (size_t i = 0; i < SB; ++i) {
    gh[i] = grad_h_n ? grad_h_n[i] : 0.0f;
    gc[i] = grad_c_n ? grad_c_n[i] : 0.0f;
  }
  for (int t = T - 1; t >= 0; --t) {
    const size_t so = (size_t)t * SB, go = (size_t)t * B * C;
    const float *pc = t == 0 ? c0d : cd + so - SB;
    for (int b = 0; b < B; ++b)
      for (int j = 0; j < H; ++j) {
        const size_t e = (size_t)b * H + j, gb = (size_t)b * C + j;
        const float ig = gd[go + gb], fg = gd[go + gb + H], gg = gd[go + gb + 2 * H], og = gd[go + gb + 3 * H];
        const float ct = td[so + e];
        const float dh = (gh[e] + grad_output[so + e]) * keep(sv->hidden_m, so + e);
        const float d_o = dh * ct;
        const float dct = dh * og * keep(sv->cell_tanh_m, so + e);
        const float dc = gc[e] + dct * (1.0f - ct * ct);
        const float mdc = dc * keep(sv->cell_m, so + e);
        const float dfg = mdc * pc[e];
        const float dig = mdc * gg, dgg = mdc * ig;
        const float go_[4] = {dig * keep(sv->gate_out_m, go + gb), dfg * keep(sv->gate_out_m, go + gb + H),
                              dgg * keep(sv->gate_out_m, go + gb + 2 * H), d_o * keep(sv->gate_out_m, go + gb + 3 * H)};
        const float gi_[4] = {go_[0] * ig * (1.0f - ig), go_[1] * fg * (1.0f - fg), go_[2] * (1.0f - gg * gg),
                              go_[3] * og * (1.0f - og)};
        for (int g = 0; g < 4; ++g) {
          const size_t gi = go + gb + (size_t)g * H;
          const float gr = gi_[g] * keep(sv->gate_in_m, gi);
          dli[gi] = gr * keep(sv->ih_linear_m, gi);
          dlh[gi] = gr * keep(sv->hh_linear_m, gi);
        }
        gc[e] = mdc * fg;
      }
    for (int b = 0; b < B; ++b)
      for (int k = 0; k < H; ++k) {
        double s = 0.0;
        for (int c = 0; c < C; ++c) s += (double)dlh[go + (size_t)b * C + c] * wh[(size_t)c * H + k];
        gh[(size_t)b * H + k] = (float)s;
      }
  }
  for (size_t r = 0; r < (size_t)T * B; ++r)
    for (int k = 0; k < I; ++k) {
      double s = 0.0;
      for (int c = 0; c < C; ++c) s += (double)dli[r * C + c] * wi[(size_t)c * I + k];
      dx[r * I + k] = (float)s * keep(sv->x_m, r * I + k);
    }
  for (int c = 0; c < C; ++c) {
    for (int k = 0; k < I; ++k) {
      double s = 0.0;
      for (size_t r = 0; r < (size_t)T * B; ++r) s += (double)dli[r * C + c] * xd[r * I + k];
      dW_ih[(size_t)c * I + k] = (float)s * keep(sv->w_ih_m, (size_t)c * I + k);
    }
    for (int k = 0; k < H; ++k) {
      double s = 0.0;
      for (int t = 0; t < T; ++t)
        for (int b = 0; b < B; ++b) {
          const float hp = t == 0 ? h0d[(size_t)b * H + k] : hd[((size_t)(t - 1) * B + b) * H + k];
          s += (double)dlh[((size_t)t * B + b) * C + c] * hp;
        }
      dW_hh[(size_t)c * H + k] = (float)s * keep(sv->w_hh_m, (size_t)c * H + k);
    }
    if (db_ih) {
      double si = 0.0, sh = 0.0;
      for (size_t r = 0; r < (size_t)T * B; ++r) { si += dli[r * C + c]; sh += dlh[r * C + c]; }
      db_ih[c] = (float)si * keep(sv->b_ih_m, c);
      db_hh[c] = (float)sh * keep(sv->b_hh_m, c);
    }
  }
  for (size_t i = 0; i < SB; ++i) {
    dh0[i] = gh[i] * keep(sv->h0_m, i);
    dc0[i] = gc[i] * keep(sv->c0_m, i);
  }
  free(xd); free(wi); free(wh); free(h0d); free(c0d); free(gd); free(cd); free(td); free(hd);
  free(gh); free(gc); free(dli); free(dlh);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Primitive entry points (pinned by the reference's primitive golden vectors)       */
/* ------------------------------------------------------------------------------ */

double olstm_prim_rne(double v) { return rne(v); }

void olstm_prim_range(const rxmet_lstm_op_config *t, int32_t *lo, int32_t *hi) {
  grid_range(t, lo, hi);
}

float olstm_prim_quantize(float v, float s, int32_t zp, const rxmet_lstm_op_config *t) {
  return quantize_master(v, s, zp, t, NULL);
}

float olstm_prim_dequantize(float q, float s, int32_t zp) { return dequant(q, s, zp); }

int olstm_prim_mshift(double ratio, rxmet_lstm_rescale *r) { return encode_mshift(ratio, r); }

float olstm_prim_apply(float v, const rxmet_lstm_rescale *r) { return apply_rescale(v, r); }

int olstm_prim_calibrate(float mn, float mx, const rxmet_lstm_op_config *t, int pot2, int bias,
                         float *scale, int32_t *zp) {
  calib_t c;
  if (calibrate_group(mn, mx, t, pot2, bias, &c)) return -1;
  *scale = c.scale;
  *zp = c.zp;
  return 0;
}
