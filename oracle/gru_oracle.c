/*
 * gru_oracle.c — CPU oracle of the QuantGRU FP32-carrier QAT path. TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this code
 * (through oracle/gru_oracle.py), and only as the checker or the CPU baseline; the
 * product library never links it.
 *
 * Plain C restatement, single thread, fp32 arithmetic in the reference's operation
 * order (built with -ffp-contract=off), of:
 *   - grid helpers and scale encoding: QuantBitWidth (quantize_bitwidth_config.h:7-54),
 *     encodeMShift/decodeMShift/pot2Shift (scale_encoding.h:87-125), scaleToPowerOfTwo
 *     (pot_scale_encode.h:72-103), get_minimum_scale (histogram_collector.h:34-38);
 *   - calculateGRUQuantitativeParameters (src/gru_host.cc:13-124) with
 *     calibrateContinuousScaleFromRange (pot_sqnr_calibrator.h:372-447),
 *     encodeScaleResult (scale_encoding.h:250-321), calibrateBias and
 *     ensureMinRange (gru_calibration_helpers.h:31-61, calibration_utils.h:27-44);
 *   - the 16-segment PWL LUT generator (src/quantize_lut.cc:53-365);
 *   - the float calibration forward (src/gru_forward_cpu.cc:58-151);
 *   - the FP32-carrier quantised forward: boundary quantisation
 *     (src/quantize_ops.cu:109-142, gru_interface.cc:213-290,636-716), rescale parameters
 *     (src/gru_forward_gpu_quant_fp.cu:454-645) and PointwiseOperationsFP (:90-393,
 *     604-801); GEMMs of integer codes are summed exactly (int64) and rounded once to
 *     fp32, which equals any fp32 summation whenever partial sums stay below 2^24;
 *   - the STE backward (src/gru_backward_gpu_quant.cu:93-266, 379-493) on dequantised
 *     values, GEMM sums accumulated in fp64.
 *
 * Pinning (tests/test_gru_oracle.py): parameters, LUTs and calibration statistics are
 * compared with the reference's own C++ compiled from /root/reference into oracle/_ref;
 * the forward with an equivalent dequantised-domain fake-quant formulation, the float
 * limit against torch.nn.GRU and train/eval invariants; the backward against torch
 * autograd through the reference's surrogate construction (tests/recurrent/
 * test_gru_autograd.py:21-48).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/rxmet_gru.h"

/* Summation of the two GEMMs of codes in the FP32-carrier forward.  ORACLE_SUM_EXACT (the
 * default, what the HIP kernels compute): exact int64 sums rounded once to fp32.
 * ORACLE_SUM_SEQ_F32: fp32 products added in K order, a model of the reference's cuBLAS
 * SGEMM (ComputeLinearX / ComputeLinearH, gru_forward_gpu_quant_fp.cu:1111-1155), whose own
 * summation order is not reproducible here.  The two agree while every partial sum stays
 * below 2^24; the mode exists to measure how far they drift apart beyond that. */
enum { ORACLE_SUM_EXACT = 0, ORACLE_SUM_SEQ_F32 = 1 };
static int g_sum_mode = ORACLE_SUM_EXACT;
void oracle_gru_set_sum_mode(int mode) { g_sum_mode = mode; }

/* ------------------------------------------------------------------------------ */
/* Grids                                                                           */
/* ------------------------------------------------------------------------------ */

static int32_t g_qmin(int32_t bits, int32_t uns) {
  if (bits >= 32) return INT32_MIN;
  return uns ? 0 : -(1 << (bits - 1));
}
static int32_t g_qmax(int32_t bits, int32_t uns) {
  if (bits >= 32) return INT32_MAX;
  return uns ? (int32_t)((1u << bits) - 1u) : (1 << (bits - 1)) - 1;
}
static int32_t eff_uns(int32_t bits, int32_t uns) { return bits >= 32 ? 0 : uns; }

/* clamp_f (quantize_ops_helper.h:332-354), GPU semantics (fmaxf/fminf: NaN -> hi). */
static float clampq(float v, int32_t bits, int32_t uns, uint8_t *keep) {
  uns = eff_uns(bits, uns);
  const int32_t qlo = g_qmin(bits, uns), qhi = g_qmax(bits, uns);
  float lo = (float)qlo, hi = (float)qhi;
  if ((double)lo < (double)qlo) lo = nextafterf(lo, INFINITY);
  if ((double)hi > (double)qhi) hi = nextafterf(hi, -INFINITY);
  if (keep) *keep = (v < lo || v > hi) ? 0 : 1;
  return fmaxf(lo, fminf(v, hi));
}

/* ------------------------------------------------------------------------------ */
/* Scale encoding                                                                  */
/* ------------------------------------------------------------------------------ */

typedef struct { uint16_t m; int8_t shift; } fixed_scale;

static fixed_scale encode_mshift(float scale) {
  int e = 0;
  double mant = frexp((double)scale, &e);
  uint32_t m = (uint32_t)llround(mant * 65536.0);
  if (m == 65536u) { m = 32768u; e += 1; }
  if (m < 32768u) m = 32768u;
  fixed_scale f = {(uint16_t)m, (int8_t)(16 - e)};
  return f;
}
static float decode_mshift(fixed_scale f) {
  return (float)f.m * ldexpf(1.0f, -(int)f.shift);
}
static int8_t pot2_shift(float scale) {
  if (!(scale > 0.0f)) return 0;
  return (int8_t)lround(-log2((double)scale));
}

float oracle_effective_scale(float scale, int32_t use_pot2) {
  if (use_pot2) {
    fixed_scale f = {1, pot2_shift(scale)};
    return decode_mshift(f);
  }
  return decode_mshift(encode_mshift(scale));
}

static float min_scale(int64_t num_steps) {
  const float eps = 1.19209290e-07f;
  const float r = 0.01f / (float)num_steps;
  return eps < r ? eps : r;
}

typedef struct { float scale, min, max; } cont_scale;

/* std::min / std::max with their exact NaN behaviour. */
static float smin(float a, float b) { return (b < a) ? b : a; }
static float smax(float a, float b) { return (a < b) ? b : a; }

static cont_scale continuous_from_range(float mn, float mx, int32_t bits, int32_t uns, int32_t sym) {
  uns = eff_uns(bits, uns);
  const int32_t qmin = g_qmin(bits, uns), qmax = g_qmax(bits, uns);
  const int64_t n = (int64_t)qmax - (int64_t)qmin;
  const float ms = min_scale(n);
  const float mn_z = smin(mn, 0.0f);
  const float mx_z = smax(mx, 0.0f);
  const float diff = (mx_z - mn_z) / (float)n;
  const float adj = (diff < ms) ? ms : 0.0f;
  float umin = mn_z, umax = mx_z;
  if (sym) {
    if (uns) {
      umax = mx_z + (float)n * adj;
      umin = 0.0f;
    } else {
      umax = mx_z + floorf((float)n / 2.0f) * adj;
      umin = mn_z - ceilf((float)n / 2.0f) * adj;
    }
  } else {
    umax = mx_z + (float)n * adj;
  }
  cont_scale c;
  if (sym) {
    if (uns) {
      const float dmax = smax(umax, ms);
      c.scale = smax(dmax / (float)qmax, ms);
      c.min = 0.0f;
      c.max = c.scale * (float)qmax;
    } else {
      const int64_t npos = n / 2, nneg = (n + 1) / 2;
      const int add = (n == 3) ? 1 : 0;
      const float dfm = (npos + add > 0) ? umax / (float)(npos + add) : 0.0f;
      const float dfn = (nneg > 0) ? -umin / (float)nneg : 0.0f;
      c.scale = smax(smax(dfm, dfn), ms);
      c.min = -(float)nneg * c.scale;
      c.max = (float)npos * c.scale;
    }
  } else {
    const float range = smax(umax - umin, ms * (float)n);
    c.scale = smax(range / (float)n, ms);
    c.min = umin;
    c.max = umin + c.scale * (float)n;
  }
  return c;
}

static int near_pow2(float v, float tol) {
  if (!(v > 0.0f)) return 0;
  const float l = log2f(v);
  const float nearest = powf(2.0f, roundf(l));
  return fabsf(v - nearest) / nearest < tol;
}

/* encodeScaleResult -> (stored scale, zero point). Returns 0, or -1 on bad shift. */
static int encode_grid(cont_scale c, int32_t bits, int32_t uns, int32_t sym, int32_t use_pot2,
                       int32_t method, float tol, float *stored, int32_t *zp) {
  uns = eff_uns(bits, uns);
  const int32_t qmin = g_qmin(bits, uns);
  if (use_pot2) {
    if (!(c.scale > 0.0f)) return -1;
    const float n = -log2f(c.scale);
    float nc;
    if (method == RXMET_POT_ROUND) nc = roundf(n);
    else if (method == RXMET_POT_FLOOR) nc = floorf(n);
    else nc = near_pow2(fabsf(c.max - c.min), tol) ? roundf(n) : floorf(n);
    if (nc < -128.0f || nc > 127.0f) return -1;
    const int8_t no = (int8_t)nc;
    const float po2 = powf(2.0f, -(float)no);
    if (sym) *zp = 0;
    else if (method == RXMET_POT_FLOOR) {
      const float aligned = floorf(c.min / po2) * po2;
      *zp = (int32_t)rintf((float)qmin - aligned / po2);
    } else {
      *zp = (int32_t)rintf((float)qmin - c.min / po2);
    }
    *stored = po2;
    return 0;
  }
  const float eff = decode_mshift(encode_mshift(c.scale));
  *zp = sym ? 0 : (int32_t)rintf((float)qmin - c.min / eff);
  *stored = c.scale;
  return 0;
}

static int calib_scalar(const rxmet_gru_config *cfg, const rxmet_bitspec *b, float mn, float mx,
                        rxmet_grid *out) {
  cont_scale c = continuous_from_range(mn, mx, b->bits, b->is_unsigned, b->symmetric);
  out->bits = b->bits;
  out->is_unsigned = eff_uns(b->bits, b->is_unsigned);
  return encode_grid(c, b->bits, b->is_unsigned, b->symmetric, cfg->use_pot2, cfg->pot_method,
                     cfg->pot_tolerance, &out->scale, &out->zero_point);
}

static void ensure_min_range(float *mn, float *mx, float thr) {
  const float range = *mx - *mn;
  if (range < thr) {
    const float center = (*mn + *mx) / 2.0f;
    *mn = center - thr / 2.0f;
    *mx = center + thr / 2.0f;
  }
}

int oracle_gru_make_params(const rxmet_gru_ranges *r, const rxmet_gru_config *cfg,
                           rxmet_gru_qparams *out) {
  for (int k = 0; k < RXMET_GRU_NCHAN; ++k)
    if (!cfg->chan[k].symmetric) return -2;
  const int H = r->hidden, C = 3 * H;
  out->hidden = H;
  out->use_pot2 = cfg->use_pot2;
  for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
    float mn = r->min[i], mx = r->max[i];
    if (i == RXMET_GRU_Z_OUT || i == RXMET_GRU_R_OUT || i == RXMET_GRU_N_OUT)
      ensure_min_range(&mn, &mx, 0.5f);
    if (calib_scalar(cfg, &cfg->op[i], mn, mx, &out->g[i])) return -3;
  }
  /* weights W, R: per tensor / gate / channel over channel ranges */
  for (int k = 0; k < 2; ++k) {
    const rxmet_bitspec *b = &cfg->chan[k];
    out->chan_bits[k] = b->bits;
    out->chan_unsigned[k] = eff_uns(b->bits, b->is_unsigned);
    const int group = b->granularity == RXMET_PER_TENSOR ? C : (b->granularity == RXMET_PER_GATE ? H : 1);
    for (int g0 = 0; g0 < C; g0 += group) {
      float mn = FLT_MAX, mx = -FLT_MAX;
      if (group == 1) {
        mn = r->chan_min[k][g0];
        mx = r->chan_max[k][g0];
      } else {
        for (int c = g0; c < g0 + group; ++c) {
          mn = r->chan_min[k][c] < mn ? r->chan_min[k][c] : mn;
          mx = r->chan_max[k][c] > mx ? r->chan_max[k][c] : mx;
        }
      }
      rxmet_grid gr;
      if (calib_scalar(cfg, b, mn, mx, &gr)) return -3;
      for (int c = g0; c < g0 + group; ++c) out->chan_scale[k][c] = gr.scale;
    }
  }
  /* biases: headroom rule */
  for (int k = 2; k < 4; ++k) {
    const rxmet_bitspec *b = &cfg->chan[k];
    out->chan_bits[k] = b->bits;
    out->chan_unsigned[k] = eff_uns(b->bits, b->is_unsigned);
    const int group = b->granularity == RXMET_PER_TENSOR ? C : (b->granularity == RXMET_PER_GATE ? H : 1);
    const int32_t qmax = g_qmax(b->bits, eff_uns(b->bits, b->is_unsigned));
    for (int g0 = 0; g0 < C; g0 += group) {
      double ext = 0.0;
      for (int c = g0; c < g0 + group; ++c) {
        const float lo = r->chan_min[k][c], hi = r->chan_max[k][c];
        if (!isfinite(lo) || !isfinite(hi) || lo > hi) return -4;
        const double a = fabs((double)lo), bb = fabs((double)hi);
        const double m = a > bb ? a : bb;
        ext = ext > m ? ext : m;
      }
      double s = (2.0 * ext > 0.01 ? 2.0 * ext : 0.01) / qmax;
      if (cfg->use_pot2) s = exp2(ceil(log2(s)));
      if (!isfinite(s) || s > FLT_MAX) return -5;
      for (int c = g0; c < g0 + group; ++c) out->chan_scale[k][c] = (float)s;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* PWL LUT                                                                         */
/* ------------------------------------------------------------------------------ */

static int cmpf(const void *a, const void *b) {
  const float x = *(const float *)a, y = *(const float *)b;
  return (x > y) - (x < y);
}

/* Returns the number of points (17 on success) in pts. */
static int segment_points(float x_min, float x_max, float *pts) {
  enum { NS = 1000, NSEG = 16 };
  static float xs[NS], w[NS - 1], cw[NS - 1];
  for (int i = 0; i < NS; ++i) xs[i] = x_min + (x_max - x_min) * (float)i / (float)(NS - 1);
  for (int i = 0; i < NS - 1; ++i) {
    const float x = xs[i], xn = xs[i + 1];
    const float y = 1.0f / (1.0f + expf(-x));
    const float yn = 1.0f / (1.0f + expf(-xn));
    const float slope = fabsf(yn - y) / (xn - x + 1e-9f);
    const float d = fabsf(x);
    w[i] = d < 2.0f ? 5.0f * (1.0f - d / 2.0f) + 1.0f : 1.0f + slope * 0.5f;
  }
  float sw = 0.0f;
  for (int i = 0; i < NS - 1; ++i) sw += w[i];
  for (int i = 0; i < NS - 1; ++i) w[i] /= sw;
  cw[0] = w[0];
  for (int i = 1; i < NS - 1; ++i) cw[i] = cw[i - 1] + w[i];
  float tmp[64];
  int np = 0;
  tmp[np++] = x_min;
  for (int i = 1; i < NSEG; ++i) {
    const float target = (float)i / (float)NSEG;
    int idx = 0;
    while (idx < NS - 1 && cw[idx] < target) ++idx; /* lower_bound */
    if (idx >= NS - 1) idx = NS - 2;
    tmp[np++] = xs[idx];
  }
  tmp[np++] = x_max;
  qsort(tmp, np, sizeof(float), cmpf);
  int u = 0;
  for (int i = 0; i < np; ++i) {
    if (u > 0 && fabsf(tmp[u - 1] - tmp[i]) < 1e-9f) continue;
    tmp[u++] = tmp[i];
  }
  np = u;
  while (np < NSEG + 1) {
    float gmax = 0.0f;
    int gi = 0;
    for (int i = 0; i < np - 1; ++i) {
      const float gap = tmp[i + 1] - tmp[i];
      if (gap > gmax) { gmax = gap; gi = i; }
    }
    const float mid = (tmp[gi] + tmp[gi + 1]) / 2.0f;
    memmove(&tmp[gi + 2], &tmp[gi + 1], sizeof(float) * (np - gi - 1));
    tmp[gi + 1] = mid;
    ++np;
  }
  memcpy(pts, tmp, sizeof(float) * np);
  return np;
}

static void fit_line(const float *x, const float *y, int n, float *b, float *c) {
  float sx = 0.0f, sy = 0.0f, sxy = 0.0f, sx2 = 0.0f;
  for (int i = 0; i < n; ++i) {
    sx += x[i];
    sy += y[i];
    sxy += x[i] * y[i];
    sx2 += x[i] * x[i];
  }
  const float den = (float)n * sx2 - sx * sx;
  if (fabsf(den) < 1e-9f) {
    *b = 0.0f;
    *c = sy / (float)n;
    return;
  }
  *b = ((float)n * sxy - sx * sy) / den;
  *c = (sy - *b * sx) / (float)n;
}

static void quant_multiplier(float v, int32_t out_bits, int32_t out_uns, int32_t *q, int32_t *n) {
  if (fabsf(v) < 1e-12f) { *q = 0; *n = 0; return; }
  const int32_t mq = g_qmax(out_bits, eff_uns(out_bits, out_uns));
  const int8_t nn = (int8_t)floor(log2((double)mq / (double)fabsf(v)));
  int64_t qq = (int64_t)rint((double)v * ldexp(1.0, nn));
  if (qq > mq) qq = mq;
  if (qq < -mq) qq = -mq;
  *q = (int32_t)qq;
  *n = nn;
}

static void make_lut(int is_tanh, float sx, int32_t zpx, float sy, int32_t zpy, int32_t in_bits,
                     int32_t in_uns, int32_t out_bits, int32_t out_uns, rxmet_pwl_lut *lut) {
  in_uns = eff_uns(in_bits, in_uns);
  const int32_t qmin = g_qmin(in_bits, in_uns), qmax = g_qmax(in_bits, in_uns);
  float x_min = (float)(qmin - zpx) * sx;
  float x_max = (float)(qmax - zpx) * sx;
  const float range = is_tanh ? 4.0f : 8.0f;
  x_min = x_min > -range ? x_min : -range;
  x_max = x_max < range ? x_max : range;
  float pts[64];
  segment_points(x_min, x_max, pts);
  lut->zp_x = zpx;
  for (int i = 0; i < 16; ++i) {
    const float xa = pts[i], xb = pts[i + 1];
    float xv[100], yv[100];
    for (int j = 0; j < 100; ++j) {
      xv[j] = xa + (xb - xa) * (float)j / (float)99;
      yv[j] = is_tanh ? tanhf(xv[j]) : 1.0f / (1.0f + expf(-xv[j]));
    }
    float b, c;
    fit_line(xv, yv, 100, &b, &c);
    const float m = b * (sx / sy);
    int32_t qb, n;
    quant_multiplier(m, out_bits, out_uns, &qb, &n);
    lut->seg[i].q_b = qb;
    lut->seg[i].n = n;
    lut->seg[i].c = (int32_t)rintf(c / sy + (float)zpy);
    int32_t th = (int32_t)rintf(xb / sx + (float)zpx);
    th = th < qmin ? qmin : (th > qmax ? qmax : th);
    lut->seg[i].threshold = th;
  }
}

int oracle_gru_make_luts(const rxmet_gru_qparams *p, rxmet_pwl_lut out[3]) {
  const rxmet_grid *g = p->g;
  make_lut(0, g[RXMET_GRU_Z_IN].scale, g[RXMET_GRU_Z_IN].zero_point, g[RXMET_GRU_Z_OUT].scale,
           g[RXMET_GRU_Z_OUT].zero_point, g[RXMET_GRU_Z_IN].bits, g[RXMET_GRU_Z_IN].is_unsigned,
           g[RXMET_GRU_Z_OUT].bits, g[RXMET_GRU_Z_OUT].is_unsigned, &out[0]);
  make_lut(0, g[RXMET_GRU_R_IN].scale, g[RXMET_GRU_R_IN].zero_point, g[RXMET_GRU_R_OUT].scale,
           g[RXMET_GRU_R_OUT].zero_point, g[RXMET_GRU_R_IN].bits, g[RXMET_GRU_R_IN].is_unsigned,
           g[RXMET_GRU_R_OUT].bits, g[RXMET_GRU_R_OUT].is_unsigned, &out[1]);
  make_lut(1, g[RXMET_GRU_N_IN].scale, g[RXMET_GRU_N_IN].zero_point, g[RXMET_GRU_N_OUT].scale,
           g[RXMET_GRU_N_OUT].zero_point, g[RXMET_GRU_N_IN].bits, g[RXMET_GRU_N_IN].is_unsigned,
           g[RXMET_GRU_N_OUT].bits, g[RXMET_GRU_N_OUT].is_unsigned, &out[2]);
  return 0;
}

static float pwl(float q, const rxmet_pwl_lut *lut, int32_t out_bits, int32_t out_uns,
                 uint8_t *keep) {
  int s = 15;
  for (int i = 0; i < 16; ++i)
    if (q < (float)lut->seg[i].threshold) { s = i; break; }
  const float prod = (float)lut->seg[s].q_b * (q - (float)lut->zp_x);
  const float v = rintf(ldexpf(prod, -lut->seg[s].n)) + (float)lut->seg[s].c;
  return clampq(v, out_bits, out_uns, keep);
}

/* Exported for tests: one PWL evaluation. */
float oracle_pwl_eval(float q, const rxmet_pwl_lut *lut, int32_t out_bits, int32_t out_uns) {
  return pwl(q, lut, out_bits, out_uns, NULL);
}

/* ------------------------------------------------------------------------------ */
/* Float calibration forward                                                       */
/* ------------------------------------------------------------------------------ */

static void observe(const float *d, size_t n, float *mn, float *mx) {
  float lo = FLT_MAX, hi = -FLT_MAX;
  for (size_t i = 0; i < n; ++i)
    if (isfinite(d[i])) {
      lo = d[i] < lo ? d[i] : lo;
      hi = d[i] > hi ? d[i] : hi;
    }
  if (lo > hi) lo = hi = 0.0f;
  *mn = lo < *mn ? lo : *mn;
  *mx = hi > *mx ? hi : *mx;
}

/* stats layout: min[13], max[13], then per k in (W,R,bw,br): min[3H], max[3H]. */
int oracle_gru_forward_calibrate(int T, int B, int I, int H, const float *W, const float *R,
                                 const float *bw, const float *br, const float *x,
                                 const float *h0, float *h, float *v, float *stats) {
  const int C = 3 * H;
  const size_t NH = (size_t)B * H, cnt = (size_t)T * NH;
  float *wx = malloc(sizeof(float) * cnt * 3), *rh = malloc(sizeof(float) * cnt * 3);
  float *zp = malloc(sizeof(float) * cnt), *rp = malloc(sizeof(float) * cnt);
  float *np_ = malloc(sizeof(float) * cnt), *zv = malloc(sizeof(float) * cnt);
  float *rv = malloc(sizeof(float) * cnt), *nv = malloc(sizeof(float) * cnt);
  float *rhm = malloc(sizeof(float) * cnt), *newc = malloc(sizeof(float) * cnt);
  float *oldc = malloc(sizeof(float) * cnt);
  if (h0) memcpy(h, h0, sizeof(float) * NH);
  else memset(h, 0, sizeof(float) * NH);
  for (int t = 0; t < T; ++t)
    for (int b = 0; b < B; ++b) {
      const size_t lin = ((size_t)t * B + b) * C;
      for (int c = 0; c < C; ++c) {
        float si = 0.0f, sh = 0.0f;
        for (int k = 0; k < I; ++k) si += x[((size_t)t * B + b) * I + k] * W[(size_t)k * C + c];
        for (int k = 0; k < H; ++k) sh += h[(size_t)t * NH + (size_t)b * H + k] * R[(size_t)k * C + c];
        wx[lin + c] = si + bw[c];
        rh[lin + c] = sh + br[c];
      }
      for (int c = 0; c < H; ++c) {
        const size_t idx = (size_t)t * NH + (size_t)b * H + c;
        zp[idx] = wx[lin + c] + rh[lin + c];
        rp[idx] = wx[lin + H + c] + rh[lin + H + c];
        /* inline_ops.h:8-11: sigmoid<float> calls the double exp (unqualified exp on a
           float resolves to ::exp(double)), so the quotient is formed in double */
        const float z = (float)(1.0 / (1.0 + exp(-(double)zp[idx])));
        const float r = (float)(1.0 / (1.0 + exp(-(double)rp[idx])));
        const float rec = rh[lin + 2 * H + c];
        rhm[idx] = r * rec;
        np_[idx] = wx[lin + 2 * H + c] + rhm[idx];
        const float n = tanhf(np_[idx]);
        zv[idx] = z;
        rv[idx] = r;
        nv[idx] = n;
        oldc[idx] = z * h[idx];
        newc[idx] = (1.0f - z) * n;
        h[idx + NH] = oldc[idx] + newc[idx];
        if (v) {
          const size_t base = ((size_t)t * B + b) * H * 4 + c;
          v[base] = z;
          v[base + H] = r;
          v[base + 2 * H] = n;
          v[base + 3 * H] = rec;
        }
      }
    }
  float *mn = stats, *mx = stats + RXMET_GRU_NGRIDS;
  observe(x, (size_t)T * B * I, &mn[RXMET_GRU_X], &mx[RXMET_GRU_X]);
  observe(h + NH, cnt, &mn[RXMET_GRU_H], &mx[RXMET_GRU_H]);
  observe(wx, cnt * 3, &mn[RXMET_GRU_WX], &mx[RXMET_GRU_WX]);
  observe(rh, cnt * 3, &mn[RXMET_GRU_RH], &mx[RXMET_GRU_RH]);
  observe(zp, cnt, &mn[RXMET_GRU_Z_IN], &mx[RXMET_GRU_Z_IN]);
  observe(rp, cnt, &mn[RXMET_GRU_R_IN], &mx[RXMET_GRU_R_IN]);
  observe(np_, cnt, &mn[RXMET_GRU_N_IN], &mx[RXMET_GRU_N_IN]);
  observe(zv, cnt, &mn[RXMET_GRU_Z_OUT], &mx[RXMET_GRU_Z_OUT]);
  observe(rv, cnt, &mn[RXMET_GRU_R_OUT], &mx[RXMET_GRU_R_OUT]);
  observe(nv, cnt, &mn[RXMET_GRU_N_OUT], &mx[RXMET_GRU_N_OUT]);
  observe(rhm, cnt, &mn[RXMET_GRU_MUL_RH], &mx[RXMET_GRU_MUL_RH]);
  observe(newc, cnt, &mn[RXMET_GRU_MUL_NEW], &mx[RXMET_GRU_MUL_NEW]);
  observe(oldc, cnt, &mn[RXMET_GRU_MUL_OLD], &mx[RXMET_GRU_MUL_OLD]);
  float *chan = stats + 2 * RXMET_GRU_NGRIDS;
  const float *src[4] = {W, R, bw, br};
  const int rows[4] = {I, H, 1, 1};
  for (int k = 0; k < 4; ++k) {
    float *cmin = chan + (size_t)k * 2 * C, *cmax = cmin + C;
    float col[4096];
    for (int c = 0; c < C; ++c) {
      for (int rr = 0; rr < rows[k]; ++rr) col[rr] = src[k][(size_t)rr * C + c];
      observe(col, rows[k], &cmin[c], &cmax[c]);
    }
  }
  free(wx); free(rh); free(zp); free(rp); free(np_); free(zv); free(rv); free(nv);
  free(rhm); free(newc); free(oldc);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Quantised forward (FP32 carrier)                                                */
/* ------------------------------------------------------------------------------ */

typedef struct {
  float zp_wx, zp_rh, zp_h, zp_x;
  float zp_zin, zp_zout, zp_rin, zp_rout, zp_nin, zp_nout;
  float ih_to_zin, hh_to_zin, ih_to_rin, hh_to_rin, ih_to_nin, rmul_to_nin;
  float quant_one, old_to_h, nout_to_h;
} gate_rescale;

static void make_rescale(const rxmet_gru_qparams *p, gate_rescale *g) {
  const rxmet_grid *q = p->g;
  g->zp_wx = (float)q[RXMET_GRU_WX].zero_point;
  g->zp_rh = (float)q[RXMET_GRU_RH].zero_point;
  g->zp_h = (float)q[RXMET_GRU_H].zero_point;
  g->zp_x = (float)q[RXMET_GRU_X].zero_point;
  g->zp_zin = (float)q[RXMET_GRU_Z_IN].zero_point;
  g->zp_zout = (float)q[RXMET_GRU_Z_OUT].zero_point;
  g->zp_rin = (float)q[RXMET_GRU_R_IN].zero_point;
  g->zp_rout = (float)q[RXMET_GRU_R_OUT].zero_point;
  g->zp_nin = (float)q[RXMET_GRU_N_IN].zero_point;
  g->zp_nout = (float)q[RXMET_GRU_N_OUT].zero_point;
  g->ih_to_zin = q[RXMET_GRU_WX].scale / q[RXMET_GRU_Z_IN].scale;
  g->hh_to_zin = q[RXMET_GRU_RH].scale / q[RXMET_GRU_Z_IN].scale;
  g->ih_to_rin = q[RXMET_GRU_WX].scale / q[RXMET_GRU_R_IN].scale;
  g->hh_to_rin = q[RXMET_GRU_RH].scale / q[RXMET_GRU_R_IN].scale;
  g->ih_to_nin = q[RXMET_GRU_WX].scale / q[RXMET_GRU_N_IN].scale;
  g->rmul_to_nin = (q[RXMET_GRU_R_OUT].scale * q[RXMET_GRU_RH].scale) / q[RXMET_GRU_N_IN].scale;
  g->quant_one = rintf(1.0f / q[RXMET_GRU_Z_OUT].scale) + (float)q[RXMET_GRU_Z_OUT].zero_point;
  g->old_to_h = (q[RXMET_GRU_Z_OUT].scale * q[RXMET_GRU_H].scale) / q[RXMET_GRU_H].scale;
  g->nout_to_h = q[RXMET_GRU_N_OUT].scale / q[RXMET_GRU_H].scale;
}

static float quant_elem(float v, float eff, float zp, int32_t bits, int32_t uns, uint8_t *keep) {
  return clampq(rintf(v / eff) + zp, bits, uns, keep);
}

int oracle_gru_forward_quant(int is_training, int T, int B, int I, int H, const float *W,
                             const float *R, const float *bw, const float *br, const float *x,
                             const float *h0, const rxmet_gru_qparams *p, float *h, float *v,
                             float *W_q, float *R_q, float *bw_q, float *br_q, float *x_q,
                             uint8_t *x_mask, uint8_t *h0_mask, uint8_t *W_mask, uint8_t *R_mask,
                             uint8_t *bw_mask, uint8_t *br_mask, uint8_t *ih_mask,
                             uint8_t *hh_mask, uint8_t *gin_mask, uint8_t *gout_mask,
                             uint8_t *h_mask) {
  const int C = 3 * H;
  const size_t NH = (size_t)B * H;
  const int pot = p->use_pot2;
  const rxmet_grid *q = p->g;
  uint8_t k;
#define KEEP(ptr, idx) (is_training && (ptr) ? &(ptr)[idx] : &k)
  /* boundary quantisation */
  const float *wsrc[4] = {W, R, bw, br};
  float *wdst[4] = {W_q, R_q, bw_q, br_q};
  uint8_t *wmask[4] = {W_mask, R_mask, bw_mask, br_mask};
  const int wrows[4] = {I, H, 1, 1};
  for (int kk = 0; kk < 4; ++kk)
    for (int r = 0; r < wrows[kk]; ++r)
      for (int c = 0; c < C; ++c) {
        const size_t idx = (size_t)r * C + c;
        const float eff = oracle_effective_scale(p->chan_scale[kk][c], pot);
        wdst[kk][idx] = quant_elem(wsrc[kk][idx], eff, 0.0f, p->chan_bits[kk],
                                   p->chan_unsigned[kk], KEEP(wmask[kk], idx));
      }
  const float eff_x = oracle_effective_scale(q[RXMET_GRU_X].scale, pot);
  const float eff_h = oracle_effective_scale(q[RXMET_GRU_H].scale, pot);
  for (size_t i = 0; i < (size_t)T * B * I; ++i)
    x_q[i] = quant_elem(x[i], eff_x, (float)q[RXMET_GRU_X].zero_point, q[RXMET_GRU_X].bits,
                        q[RXMET_GRU_X].is_unsigned, KEEP(x_mask, i));
  for (size_t i = 0; i < NH; ++i)
    h[i] = h0 ? quant_elem(h0[i], eff_h, (float)q[RXMET_GRU_H].zero_point, q[RXMET_GRU_H].bits,
                           q[RXMET_GRU_H].is_unsigned, KEEP(h0_mask, i))
              : (float)q[RXMET_GRU_H].zero_point;
  /* rescale parameters */
  gate_rescale g;
  make_rescale(p, &g);
  float *igx = malloc(sizeof(float) * C), *ibx = malloc(sizeof(float) * C);
  float *igh = malloc(sizeof(float) * C), *ibh = malloc(sizeof(float) * C);
  float *wsum = malloc(sizeof(float) * C), *rsum = malloc(sizeof(float) * C);
  for (int c = 0; c < C; ++c) {
    const float swx = p->chan_scale[RXMET_GRU_W][c] * q[RXMET_GRU_X].scale;
    igx[c] = swx / q[RXMET_GRU_WX].scale;
    ibx[c] = p->chan_scale[RXMET_GRU_BW][c] / swx;
    const float srh = p->chan_scale[RXMET_GRU_R][c] * q[RXMET_GRU_H].scale;
    igh[c] = srh / q[RXMET_GRU_RH].scale;
    ibh[c] = p->chan_scale[RXMET_GRU_BR][c] / srh;
    float s = 0.0f;
    for (int r = 0; r < I; ++r) s += W_q[(size_t)r * C + c];
    wsum[c] = g.zp_x != 0.0f ? s * g.zp_x : 0.0f;
    s = 0.0f;
    for (int r = 0; r < H; ++r) s += R_q[(size_t)r * C + c];
    rsum[c] = g.zp_h != 0.0f ? s * g.zp_h : 0.0f;
  }
  rxmet_pwl_lut lut[3];
  oracle_gru_make_luts(p, lut);
  const rxmet_grid *gwx = &q[RXMET_GRU_WX], *grh = &q[RXMET_GRU_RH];
  float gih[3], ghh[3], wxv[3], rhv[3];
  for (int t = 0; t < T; ++t)
    for (int b = 0; b < B; ++b) {
      const float *hp = h + (size_t)t * NH + (size_t)b * H;
      const float *xp = x_q + ((size_t)t * B + b) * I;
      for (int j = 0; j < H; ++j) {
        const size_t mi = ((size_t)t * B + b) * C + j;  /* mask index of gate 0 */
        for (int gt = 0; gt < 3; ++gt) {
          const int c = gt * H + j;
          if (g_sum_mode == ORACLE_SUM_SEQ_F32) {
            /* a plain SGEMM model: products rounded to fp32, added in K order */
            float fi = 0.0f, fh = 0.0f;
            for (int r = 0; r < I; ++r) fi += xp[r] * W_q[(size_t)r * C + c];
            for (int r = 0; r < H; ++r) fh += hp[r] * R_q[(size_t)r * C + c];
            gih[gt] = fi;
            ghh[gt] = fh;
          } else {
            int64_t si = 0, sh = 0;
            for (int r = 0; r < I; ++r) si += (int64_t)xp[r] * (int64_t)W_q[(size_t)r * C + c];
            for (int r = 0; r < H; ++r) sh += (int64_t)hp[r] * (int64_t)R_q[(size_t)r * C + c];
            gih[gt] = (float)si;
            ghh[gt] = (float)sh;
          }
          /* biasRescaleInline */
          float val = gih[gt] - wsum[c];
          float bt = rintf(bw_q[c] * ibx[c]);
          float res = rintf((val + bt) * igx[c]) + g.zp_wx;
          wxv[gt] = clampq(res, gwx->bits, gwx->is_unsigned, KEEP(ih_mask, mi + gt * H));
          val = ghh[gt] - rsum[c];
          bt = rintf(br_q[c] * ibh[c]);
          res = rintf((val + bt) * igh[c]) + g.zp_rh;
          rhv[gt] = clampq(res, grh->bits, grh->is_unsigned, KEEP(hh_mask, mi + gt * H));
        }
        /* update gate */
        float in = rintf((wxv[0] - g.zp_wx) * g.ih_to_zin) + rintf((rhv[0] - g.zp_rh) * g.hh_to_zin);
        in += g.zp_zin;
        in = clampq(in, q[RXMET_GRU_Z_IN].bits, q[RXMET_GRU_Z_IN].is_unsigned, KEEP(gin_mask, mi));
        const float z = pwl(in, &lut[0], q[RXMET_GRU_Z_OUT].bits, q[RXMET_GRU_Z_OUT].is_unsigned,
                            KEEP(gout_mask, mi));
        /* reset gate */
        in = rintf((wxv[1] - g.zp_wx) * g.ih_to_rin) + rintf((rhv[1] - g.zp_rh) * g.hh_to_rin);
        in += g.zp_rin;
        in = clampq(in, q[RXMET_GRU_R_IN].bits, q[RXMET_GRU_R_IN].is_unsigned,
                    KEEP(gin_mask, mi + H));
        const float r = pwl(in, &lut[1], q[RXMET_GRU_R_OUT].bits, q[RXMET_GRU_R_OUT].is_unsigned,
                            KEEP(gout_mask, mi + H));
        /* new gate */
        const float rmul = (r - g.zp_rout) * (rhv[2] - g.zp_rh);
        in = rintf((wxv[2] - g.zp_wx) * g.ih_to_nin) + rintf(rmul * g.rmul_to_nin);
        in += g.zp_nin;
        in = clampq(in, q[RXMET_GRU_N_IN].bits, q[RXMET_GRU_N_IN].is_unsigned,
                    KEEP(gin_mask, mi + 2 * H));
        const float n = pwl(in, &lut[2], q[RXMET_GRU_N_OUT].bits, q[RXMET_GRU_N_OUT].is_unsigned,
                            KEEP(gout_mask, mi + 2 * H));
        /* hidden update */
        const float n_h = rintf((n - g.zp_nout) * g.nout_to_h) + g.zp_h;
        const float oldc = (z - g.zp_zout) * (hp[j] - g.zp_h);
        const float newc = (g.quant_one - z) * (n_h - g.zp_h);
        float hn = rintf((oldc + newc) * g.old_to_h) + g.zp_h;
        const size_t hi = (size_t)t * NH + (size_t)b * H + j;
        hn = clampq(hn, q[RXMET_GRU_H].bits, q[RXMET_GRU_H].is_unsigned, KEEP(h_mask, hi));
        h[hi + NH] = hn;
        if (v) {
          const size_t vb = ((size_t)t * B + b) * H * 4 + j;
          v[vb] = z;
          v[vb + H] = r;
          v[vb + 2 * H] = n;
          v[vb + 3 * H] = rhv[2];
        }
      }
    }
  /* dequantise h and v with the effective scales */
  for (size_t i = 0; i < (size_t)(T + 1) * NH; ++i)
    h[i] = (h[i] - (float)q[RXMET_GRU_H].zero_point) * eff_h;
  if (v) {
    const int ids[4] = {RXMET_GRU_Z_OUT, RXMET_GRU_R_OUT, RXMET_GRU_N_OUT, RXMET_GRU_RH};
    float eff[4], zpv[4];
    for (int kk = 0; kk < 4; ++kk) {
      eff[kk] = oracle_effective_scale(q[ids[kk]].scale, pot);
      zpv[kk] = (float)q[ids[kk]].zero_point;
    }
    for (size_t tb = 0; tb < (size_t)T * B; ++tb)
      for (int kk = 0; kk < 4; ++kk)
        for (int j = 0; j < H; ++j) {
          float *e = &v[tb * 4 * H + (size_t)kk * H + j];
          *e = (*e - zpv[kk]) * eff[kk];
        }
  }
  free(igx); free(ibx); free(igh); free(ibh); free(wsum); free(rsum);
#undef KEEP
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Backward                                                                        */
/* ------------------------------------------------------------------------------ */

int oracle_gru_backward_quant(int T, int B, int I, int H, const float *W_q, const float *R_q,
                              const float *bw_q, const float *br_q, const float *x_q,
                              const float *dh_new, const float *h, const float *v,
                              const rxmet_gru_qparams *p, const uint8_t *x_mask,
                              const uint8_t *h0_mask, const uint8_t *W_mask,
                              const uint8_t *R_mask, const uint8_t *bw_mask,
                              const uint8_t *br_mask, const uint8_t *ih_mask,
                              const uint8_t *hh_mask, const uint8_t *gin, const uint8_t *gout,
                              const uint8_t *h_mask, float *dx, float *dW, float *dR, float *dbw,
                              float *dbr, float *dh0) {
  (void)bw_q;
  (void)br_q;
  const int C = 3 * H;
  const size_t NH = (size_t)B * H;
  const int pot = p->use_pot2;
  float *Wd = malloc(sizeof(float) * (size_t)I * C), *Rd = malloc(sizeof(float) * (size_t)H * C);
  for (int r = 0; r < I; ++r)
    for (int c = 0; c < C; ++c)
      Wd[(size_t)r * C + c] = W_q[(size_t)r * C + c] * oracle_effective_scale(p->chan_scale[0][c], pot);
  for (int r = 0; r < H; ++r)
    for (int c = 0; c < C; ++c)
      Rd[(size_t)r * C + c] = R_q[(size_t)r * C + c] * oracle_effective_scale(p->chan_scale[1][c], pot);
  const float eff_x = oracle_effective_scale(p->g[RXMET_GRU_X].scale, pot);
  const float zpx = (float)p->g[RXMET_GRU_X].zero_point;
  float *dp = malloc(sizeof(float) * (size_t)T * B * C), *dq = malloc(sizeof(float) * (size_t)T * B * C);
  float *dh = calloc(NH, sizeof(float));
  double *sbw = calloc(C, sizeof(double)), *sbr = calloc(C, sizeof(double));
  for (int t = T - 1; t >= 0; --t) {
    for (int b = 0; b < B; ++b)
      for (int j = 0; j < H; ++j) {
        const size_t bi = (size_t)b * H + j;
        float dht = dh_new[(size_t)(t + 1) * NH + bi] + dh[bi];
        if (h_mask) dht *= (float)h_mask[(size_t)t * NH + bi];
        const size_t vb = ((size_t)t * B + b) * 4 * H + j;
        const float z = v[vb], r = v[vb + H], gg = v[vb + 2 * H], qg = v[vb + 3 * H];
        dh[bi] = z * dht;
        const float dg = (1.0f - z) * dht;
        const float dz = (h[(size_t)t * NH + bi] - gg) * dht;
        const size_t mi = ((size_t)t * B + b) * C + j;
        float dpg = (1.0f - gg * gg) * dg;
        if (gout) dpg *= (float)gout[mi + 2 * H];
        if (gin) dpg *= (float)gin[mi + 2 * H];
        float dqg = dpg * r;
        const float dr = dpg * qg;
        float dpr = r * (1.0f - r) * dr, dqr = dpr;
        float dpz = z * (1.0f - z) * dz, dqz = dpz;
        if (gout) {
          const float mz = (float)gout[mi], mr = (float)gout[mi + H];
          dpz *= mz; dqz *= mz; dpr *= mr; dqr *= mr;
        }
        if (gin) {
          const float mz = (float)gin[mi], mr = (float)gin[mi + H];
          dpz *= mz; dqz *= mz; dpr *= mr; dqr *= mr;
        }
        if (hh_mask) {
          dqz *= (float)hh_mask[mi]; dqr *= (float)hh_mask[mi + H]; dqg *= (float)hh_mask[mi + 2 * H];
        }
        if (ih_mask) {
          dpz *= (float)ih_mask[mi]; dpr *= (float)ih_mask[mi + H]; dpg *= (float)ih_mask[mi + 2 * H];
        }
        const float dps[3] = {dpz, dpr, dpg}, dqs[3] = {dqz, dqr, dqg};
        for (int gt = 0; gt < 3; ++gt) {
          const int c = gt * H + j;
          dp[mi + gt * H] = dps[gt];
          dq[mi + gt * H] = dqs[gt];
          sbw[c] += (double)(bw_mask ? dps[gt] * (float)bw_mask[c] : dps[gt]);
          sbr[c] += (double)(br_mask ? dqs[gt] * (float)br_mask[c] : dqs[gt]);
        }
      }
    /* dh += R dq_t */
    for (int b = 0; b < B; ++b)
      for (int kk = 0; kk < H; ++kk) {
        double s = 0.0;
        const float *dqr = dq + ((size_t)t * B + b) * C;
        for (int c = 0; c < C; ++c) s += (double)Rd[(size_t)kk * C + c] * (double)dqr[c];
        dh[(size_t)b * H + kk] = (float)((double)dh[(size_t)b * H + kk] + s);
      }
  }
  /* dx = dp W^T (masked), dW = x^T dp, dR = h_prev^T dq */
  for (size_t tb = 0; tb < (size_t)T * B; ++tb)
    for (int i = 0; i < I; ++i) {
      double s = 0.0;
      for (int c = 0; c < C; ++c) s += (double)Wd[(size_t)i * C + c] * (double)dp[tb * C + c];
      float val = (float)s;
      if (x_mask) val *= (float)x_mask[tb * I + i];
      dx[tb * I + i] = val;
    }
  for (int i = 0; i < I; ++i)
    for (int c = 0; c < C; ++c) {
      double s = 0.0;
      for (size_t tb = 0; tb < (size_t)T * B; ++tb)
        s += (double)((x_q[tb * I + i] - zpx) * eff_x) * (double)dp[tb * C + c];
      float val = (float)s;
      if (W_mask) val *= (float)W_mask[(size_t)i * C + c];
      dW[(size_t)i * C + c] = val;
    }
  for (int kk = 0; kk < H; ++kk)
    for (int c = 0; c < C; ++c) {
      double s = 0.0;
      for (size_t tb = 0; tb < (size_t)T * B; ++tb)
        s += (double)h[tb * H + kk] * (double)dq[tb * C + c];
      float val = (float)s;
      if (R_mask) val *= (float)R_mask[(size_t)kk * C + c];
      dR[(size_t)kk * C + c] = val;
    }
  for (int c = 0; c < C; ++c) {
    dbw[c] = (float)sbw[c];
    dbr[c] = (float)sbr[c];
  }
  for (size_t i = 0; i < NH; ++i) dh0[i] = h0_mask ? dh[i] * (float)h0_mask[i] : dh[i];
  free(Wd); free(Rd); free(dp); free(dq); free(dh); free(sbw); free(sbr);
  return 0;
}

/* ------------------------------------------------------------------------------ */
/* Quantised forward, int32 carrier                                                */
/* ------------------------------------------------------------------------------ */
/*
 * quantGRUForwardInt / quantGRUForwardIntIO (src/gru_interface.cc:384-627) over
 * ForwardPassQuant (src/gru_forward_gpu_quant.cu:112-176, 230-373, 526-847), whose
 * arithmetic the reference's CPU carrier repeats (src/gru_forward_cpu_quant.cc:109-343):
 *   - boundary quantisation with the effective scale, the code kept in double before the
 *     saturation (quantize<Training>, quantize_ops_helper.h:356-364,472-476);
 *   - GEMMs of codes summed exactly in int64 with the zero point of the right operand
 *     removed, the bias rescaled into the accumulator scale, then one rescale to the linear
 *     grid (quantizedGemmBiasFused);
 *   - the integer gate templates computeUpdateGate/ResetGate/NewGate/HiddenState
 *     (quantize_ops_helper.h:683-1023) with the 16-segment PWL (:503-549);
 *   - rescales rshift_round(x * M, shift) (M16) or rshift_round(x, shift) (POT2)
 *     (quantize_ops_helper.h:201-247) derived by makeRescale / makeRescaleProduct /
 *     makeRescaleToProduct (scale_encoding.h:133-188).
 * Outputs are int32 codes; h_q [T+1,B,H] holds the initial state in row 0.
 */

typedef struct { int64_t m; int32_t shift; } int_rescale;

/* rshift_round (quantize_ops_helper.h:201-224): round(x / 2^n), half to even, on |x|. */
static int64_t rshift_round64(int64_t x, int n) {
  if (n <= 0) return (int64_t)((uint64_t)x << (-n));
  const int neg = x < 0;
  const uint64_t ax = neg ? (uint64_t)0 - (uint64_t)x : (uint64_t)x;
  const uint64_t half = (uint64_t)1 << (n - 1);
  const uint64_t q = ax >> n, r = ax & (((uint64_t)1 << n) - 1);
  const uint64_t res = r > half ? q + 1 : (r < half ? q : q + (q & 1));
  return neg ? -(int64_t)res : (int64_t)res;
}
static int64_t apply_rescale(int64_t x, int_rescale r) { return rshift_round64(x * r.m, r.shift); }

static int_rescale rescale_of_ratio(float ratio, int pot, int8_t pot_shift) {
  int_rescale r;
  if (pot) {
    r.m = 1;
    r.shift = pot_shift;
  } else {
    const fixed_scale f = encode_mshift(ratio);
    r.m = f.m;
    r.shift = f.shift;
  }
  return r;
}
/* src -> dst */
static int_rescale rs_single(float src, float dst, int pot) {
  return rescale_of_ratio(src / dst, pot, (int8_t)(pot2_shift(src) - pot2_shift(dst)));
}
/* a*b -> dst */
static int_rescale rs_product(float a, float b, float dst, int pot) {
  return rescale_of_ratio((a * b) / dst, pot,
                          (int8_t)(pot2_shift(a) + pot2_shift(b) - pot2_shift(dst)));
}
/* src -> a*b */
static int_rescale rs_to_product(float src, float a, float b, int pot) {
  return rescale_of_ratio(src / (a * b), pot,
                          (int8_t)(pot2_shift(src) - (pot2_shift(a) + pot2_shift(b))));
}

/* clamp_by_bitwidth<Training> on int32 (quantize_ops_helper.h:267-279) */
static int32_t clampi(int32_t v, int32_t bits, int32_t uns, uint8_t *keep) {
  uns = eff_uns(bits, uns);
  const int32_t lo = g_qmin(bits, uns), hi = g_qmax(bits, uns);
  if (keep) *keep = (v < lo || v > hi) ? 0 : 1;
  return v < lo ? lo : (v > hi ? hi : v);
}

/* quantize(float, FixedPointScale, zp, bw): rint in float, zero point added in double,
 * saturated in double before the integer conversion. */
static int32_t quant_int(float v, float eff, int32_t zp, int32_t bits, int32_t uns,
                         uint8_t *keep) {
  uns = eff_uns(bits, uns);
  const double code = (double)rintf(v / eff) + (double)zp;
  const int32_t lo = g_qmin(bits, uns), hi = g_qmax(bits, uns);
  if (keep) *keep = (code < lo || code > hi) ? 0 : 1;
  return code < lo ? lo : (code > hi ? hi : (int32_t)code);
}

/* piecewise_linear_raw (quantize_ops_helper.h:519-535) */
static int32_t pwl_int(int32_t q, const rxmet_pwl_lut *lut) {
  int s = 15;
  for (int i = 0; i < 16; ++i)
    if (q < lut->seg[i].threshold) { s = i; break; }
  const int32_t off = (int32_t)((uint32_t)q - (uint32_t)lut->zp_x);
  const int64_t bx = (int64_t)lut->seg[s].q_b * (int64_t)off;
  const int n = lut->seg[s].n;
  const int32_t term = n >= 0 ? (int32_t)rshift_round64(bx, n)
                              : (int32_t)(int64_t)((uint64_t)bx << (-n));
  return (int32_t)((uint32_t)term + (uint32_t)lut->seg[s].c);
}

static int32_t add32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }

/*
 * x_q_in / h0_q_in non-null: the int-IO form (quantGRUForwardIntIO): codes taken as given,
 * x / h0 ignored.  Otherwise x (and h0 when non-null) are quantised into x_q / h_q[0].
 * v_q [T,B,4H] (z, r, n, weight_hh_linear of n) may be null; masks are written when
 * is_training is set and the pointer is non-null.
 */
int oracle_gru_forward_int(int is_training, int T, int B, int I, int H, const float *W,
                           const float *R, const float *bw, const float *br, const float *x,
                           const int32_t *x_q_in, const float *h0, const int32_t *h0_q_in,
                           const rxmet_gru_qparams *p, int32_t *h_q, int32_t *v_q,
                           int32_t *W_q, int32_t *R_q, int32_t *bw_q, int32_t *br_q,
                           int32_t *x_q, uint8_t *x_mask, uint8_t *h0_mask, uint8_t *W_mask,
                           uint8_t *R_mask, uint8_t *bw_mask, uint8_t *br_mask,
                           uint8_t *ih_mask, uint8_t *hh_mask, uint8_t *gin_mask,
                           uint8_t *gout_mask, uint8_t *h_mask) {
  const int C = 3 * H;
  const size_t NH = (size_t)B * H;
  const int pot = p->use_pot2;
  const rxmet_grid *q = p->g;
  uint8_t k;
#define KEEP(ptr, idx) (is_training && (ptr) ? &(ptr)[idx] : &k)
  /* boundary quantisation: per-channel weights and biases */
  const float *wsrc[4] = {W, R, bw, br};
  int32_t *wdst[4] = {W_q, R_q, bw_q, br_q};
  uint8_t *wmask[4] = {W_mask, R_mask, bw_mask, br_mask};
  const int wrows[4] = {I, H, 1, 1};
  for (int kk = 0; kk < 4; ++kk)
    for (int r = 0; r < wrows[kk]; ++r)
      for (int c = 0; c < C; ++c) {
        const size_t idx = (size_t)r * C + c;
        const float eff = oracle_effective_scale(p->chan_scale[kk][c], pot);
        wdst[kk][idx] = quant_int(wsrc[kk][idx], eff, 0, p->chan_bits[kk], p->chan_unsigned[kk],
                                  KEEP(wmask[kk], idx));
      }
  const rxmet_grid *gx = &q[RXMET_GRU_X], *gh = &q[RXMET_GRU_H];
  const float eff_x = oracle_effective_scale(gx->scale, pot);
  const float eff_h = oracle_effective_scale(gh->scale, pot);
  const size_t nx = (size_t)T * B * I;
  const int32_t *xq = x_q_in;
  if (!xq) {
    for (size_t i = 0; i < nx; ++i)
      x_q[i] = quant_int(x[i], eff_x, gx->zero_point, gx->bits, gx->is_unsigned, KEEP(x_mask, i));
    xq = x_q;
  }
  for (size_t i = 0; i < NH; ++i) {
    if (h0_q_in)
      h_q[i] = h0_q_in[i];
    else if (h0)
      h_q[i] = quant_int(h0[i], eff_h, gh->zero_point, gh->bits, gh->is_unsigned,
                         KEEP(h0_mask, i));
    else
      h_q[i] = gh->zero_point;
  }
  /* rescale parameters (setRescaleParam: fillLinearParams / fillGateParams) */
  int_rescale *rgx = malloc(sizeof(int_rescale) * C), *rbw = malloc(sizeof(int_rescale) * C);
  int_rescale *rgh = malloc(sizeof(int_rescale) * C), *rbr = malloc(sizeof(int_rescale) * C);
  const float sx = gx->scale, sh = gh->scale;
  const float swx = q[RXMET_GRU_WX].scale, srh = q[RXMET_GRU_RH].scale;
  for (int c = 0; c < C; ++c) {
    const float sW = p->chan_scale[RXMET_GRU_W][c], sR = p->chan_scale[RXMET_GRU_R][c];
    rgx[c] = rs_product(sW, sx, swx, pot);
    rbw[c] = rs_to_product(p->chan_scale[RXMET_GRU_BW][c], sW, sx, pot);
    rgh[c] = rs_product(sR, sh, srh, pot);
    rbr[c] = rs_to_product(p->chan_scale[RXMET_GRU_BR][c], sR, sh, pot);
  }
  const int32_t zp_x = gx->zero_point, zp_h = gh->zero_point;
  const int32_t zp_wx = q[RXMET_GRU_WX].zero_point, zp_rh = q[RXMET_GRU_RH].zero_point;
  const int32_t zp_zin = q[RXMET_GRU_Z_IN].zero_point, zp_zout = q[RXMET_GRU_Z_OUT].zero_point;
  const int32_t zp_rin = q[RXMET_GRU_R_IN].zero_point, zp_rout = q[RXMET_GRU_R_OUT].zero_point;
  const int32_t zp_nin = q[RXMET_GRU_N_IN].zero_point, zp_nout = q[RXMET_GRU_N_OUT].zero_point;
  const float szin = q[RXMET_GRU_Z_IN].scale, szout = q[RXMET_GRU_Z_OUT].scale;
  const float srin = q[RXMET_GRU_R_IN].scale, srout = q[RXMET_GRU_R_OUT].scale;
  const float snin = q[RXMET_GRU_N_IN].scale, snout = q[RXMET_GRU_N_OUT].scale;
  const int_rescale ih_zin = rs_single(swx, szin, pot), hh_zin = rs_single(srh, szin, pot);
  const int_rescale ih_rin = rs_single(swx, srin, pot), hh_rin = rs_single(srh, srin, pot);
  const int_rescale ih_nin = rs_single(swx, snin, pot);
  const int_rescale rmul_nin = rs_product(srout, srh, snin, pot);
  const int_rescale nout_h = rs_single(snout, sh, pot);
  const int_rescale old_h = rs_product(szout, sh, sh, pot);
  const int32_t quant_one = add32((int32_t)rintf(1.0f / szout), zp_zout);
  rxmet_pwl_lut lut[3];
  oracle_gru_make_luts(p, lut);
#define GB(id) q[id].bits, q[id].is_unsigned
  /* input projection: W_q (x_q - zp_x) + rescaled bw -> weight_ih_linear */
  int32_t *wx = malloc(sizeof(int32_t) * (size_t)T * B * C);
  for (size_t n = 0; n < (size_t)T * B; ++n)
    for (int c = 0; c < C; ++c) {
      int64_t acc = 0;
      for (int r = 0; r < I; ++r)
        acc += (int64_t)W_q[(size_t)r * C + c] * ((int64_t)xq[n * I + r] - zp_x);
      const int64_t b = apply_rescale((int64_t)bw_q[c], rbw[c]);
      const int32_t res = add32((int32_t)apply_rescale(acc + b, rgx[c]), zp_wx);
      wx[n * C + c] = clampi(res, GB(RXMET_GRU_WX), KEEP(ih_mask, n * C + c));
    }
  int32_t *rh = malloc(sizeof(int32_t) * C);
  for (int t = 0; t < T; ++t)
    for (int b = 0; b < B; ++b) {
      const int32_t *hp = h_q + (size_t)t * NH + (size_t)b * H;
      const size_t n = (size_t)t * B + b;
      /* recurrent projection: R_q (h - zp_h) + rescaled br -> weight_hh_linear */
      for (int c = 0; c < C; ++c) {
        int64_t acc = 0;
        for (int r = 0; r < H; ++r)
          acc += (int64_t)R_q[(size_t)r * C + c] * ((int64_t)hp[r] - zp_h);
        const int64_t bb = apply_rescale((int64_t)br_q[c], rbr[c]);
        const int32_t res = add32((int32_t)apply_rescale(acc + bb, rgh[c]), zp_rh);
        rh[c] = clampi(res, GB(RXMET_GRU_RH), KEEP(hh_mask, n * C + c));
      }
      const int32_t *wxn = wx + n * C;
      for (int j = 0; j < H; ++j) {
        const size_t mi = n * C + j;
        /* update gate */
        int32_t in = add32(add32((int32_t)apply_rescale((int64_t)wxn[j] - zp_wx, ih_zin),
                                 (int32_t)apply_rescale((int64_t)rh[j] - zp_rh, hh_zin)),
                           zp_zin);
        in = clampi(in, GB(RXMET_GRU_Z_IN), KEEP(gin_mask, mi));
        const int32_t z = clampi(pwl_int(in, &lut[0]), GB(RXMET_GRU_Z_OUT), KEEP(gout_mask, mi));
        /* reset gate */
        in = add32(add32((int32_t)apply_rescale((int64_t)wxn[H + j] - zp_wx, ih_rin),
                         (int32_t)apply_rescale((int64_t)rh[H + j] - zp_rh, hh_rin)),
                   zp_rin);
        in = clampi(in, GB(RXMET_GRU_R_IN), KEEP(gin_mask, mi + H));
        const int32_t r = clampi(pwl_int(in, &lut[1]), GB(RXMET_GRU_R_OUT),
                                 KEEP(gout_mask, mi + H));
        /* new gate: r (weight_hh_linear of n) aligned to new_gate_input in one rescale */
        const int64_t rmul = ((int64_t)r - zp_rout) * ((int64_t)rh[2 * H + j] - zp_rh);
        in = add32(add32((int32_t)apply_rescale((int64_t)wxn[2 * H + j] - zp_wx, ih_nin),
                         (int32_t)apply_rescale(rmul, rmul_nin)),
                   zp_nin);
        in = clampi(in, GB(RXMET_GRU_N_IN), KEEP(gin_mask, mi + 2 * H));
        const int32_t nn = clampi(pwl_int(in, &lut[2]), GB(RXMET_GRU_N_OUT),
                                  KEEP(gout_mask, mi + 2 * H));
        /* hidden update: u h_old + (1 - u) n on the scale S_zout S_h, one rescale to h */
        const int32_t n_h = add32((int32_t)apply_rescale((int64_t)nn - zp_nout, nout_h), zp_h);
        const int64_t oldc = ((int64_t)z - zp_zout) * ((int64_t)hp[j] - zp_h);
        const int64_t newc = ((int64_t)quant_one - z) * ((int64_t)n_h - zp_h);
        const int32_t hn = add32((int32_t)apply_rescale(oldc + newc, old_h), zp_h);
        const size_t hi = (size_t)t * NH + (size_t)b * H + j;
        h_q[hi + NH] = clampi(hn, GB(RXMET_GRU_H), KEEP(h_mask, hi));
        if (v_q) {
          const size_t vb = n * 4 * H + j;
          v_q[vb] = z;
          v_q[vb + H] = r;
          v_q[vb + 2 * H] = nn;
          v_q[vb + 3 * H] = rh[2 * H + j];
        }
      }
    }
#undef GB
#undef KEEP
  free(rgx); free(rbw); free(rgh); free(rbr); free(wx); free(rh);
  return 0;
}
