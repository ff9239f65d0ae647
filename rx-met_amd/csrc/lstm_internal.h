// lstm_internal.h — host-derived execution parameters of the QuantLSTM kernels.
#pragma once

#include <cstdint>
#include <vector>

#include "rxmet_lstm.h"

namespace rxmet {
namespace lstm {

// Integer grid of one quantisation point with its float-carrier clamp endpoints.
struct Grid {
  int32_t lo, hi;      // integer range
  float flo, fhi;      // carrier endpoints (nearest representable values inside [lo, hi])
  float scale;         // standard scale
  int32_t zp;
  // the same values in double, so kernels compare and offset without per-use conversions
  double dlo, dhi, dflo, dfhi, dscale, dzp;
};

// v -> RNE(ldexp(fl(v * mult), -shift)); POT2 encodings use mult = 1.
struct Rescale {
  float mult;
  int32_t shift;
};

// Per-step scalar parameters of the recurrence (uniform across lanes).
struct StepParams {
  Grid x, h, c, ih_lin, hh_lin, gin[4], gout[4], tanh_c;
  Rescale ih_to_gate[4], hh_to_gate[4], hidden;
  // cell ratios: fl(p * ratio_f) when !uses_fp, else (float)ldexp((double)p * mant, exp)
  float cell_ratio[2];
  int64_t cell_q31[2];
  double cell_mant[2];
  int32_t cell_exp[2];
  int32_t cell_fp[2];
};

// Per-channel (4H) parameters, laid out as arrays of length 4H.
struct ChannelParams {
  std::vector<float> w_ih_scale, w_hh_scale, b_ih_scale, b_hh_scale;
  std::vector<Rescale> ih_acc_to_lin, hh_acc_to_lin, ih_bias_to_acc, hh_bias_to_acc;
};

Grid grid_of(const rxmet_lstm_op_config &t, float scale, int32_t zp);
// Derives every encoding; returns 0 or -22 with the error message set.
int derive(const rxmet_lstm_params &p, StepParams *sp, ChannelParams *cp);

}  // namespace lstm
}  // namespace rxmet
