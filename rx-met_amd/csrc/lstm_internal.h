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
  // Reference activation exceptions (device copies of ActExceptions below): for activation k
  // (gates i, f, g, o, then tanh of the cell) the sorted input codes exc_key[exc_off[k] ..
  // + exc_n[k]) and their entries exc_val[...] = (output code - output lo) << 1 | clamp mask.
  const int32_t *exc_key;
  const uint32_t *exc_val;
  int32_t exc_off[5], exc_n[5];
};

// The reference's CPU core evaluates the real activations with the C library's expf / tanhf
// (quantized_fp_math.cuh:21-30, compiled for the host); the kernels evaluate exp / tanh in
// double and round once.  Both are then quantised to the output grid, so the two differ only
// at the input codes listed here: every code of each input grid of at most 2^16 codes is
// evaluated both ways on the host (kActExcMaxCodes), and the codes whose output code or clamp
// mask differ are kept with the reference's result.  Wider grids are not enumerated (n = 0).
constexpr int kActExcMaxCodes = 1 << 16;
struct ActExceptions {
  std::vector<int32_t> key;
  std::vector<uint32_t> val;
  int32_t off[5] = {0, 0, 0, 0, 0}, n[5] = {0, 0, 0, 0, 0};
};

// Per-channel (4H) parameters, laid out as arrays of length 4H.
struct ChannelParams {
  std::vector<float> w_ih_scale, w_hh_scale, b_ih_scale, b_hh_scale;
  std::vector<Rescale> ih_acc_to_lin, hh_acc_to_lin, ih_bias_to_acc, hh_bias_to_acc;
};

Grid grid_of(const rxmet_lstm_op_config &t, float scale, int32_t zp);
// Derives every encoding; returns 0 or -22 with the error message set.
int derive(const rxmet_lstm_params &p, StepParams *sp, ChannelParams *cp);
// Exception lists of the five activations of sp (computed once per set of grids and cached;
// thread-safe; returned by value).
ActExceptions act_exceptions(const StepParams &sp);
// Entry (output code - lo) << 1 | mask of activation k at input code q: the reference CPU
// core's arithmetic (reference = true) or the kernels' double evaluation.
uint32_t act_entry(const StepParams &sp, int k, int32_t q, bool reference);

// Saved state as codes (the module path's training forward, rxmet_lstm_saved_codes): per
// (step t, 16-sequence tile, 16-unit tile) one block of kLckBlock bytes at index
// lck_block(t, b, j): the four gate outputs as code - grid minimum, u16 [16 rows][4 gates][16
// units]; the gate masks (bit 0 hh linear, bit 1 gate input, bit 2 gate output, 1 = clamped),
// u8 [4 gates][16 rows][16 units] at kLckGm; tanh(c) as code - minimum, u16 [16][16] at
// kLckTanh; the cell-phase masks (bit 0 cell, bit 1 tanh, bit 2 hidden), u8 [16][16] at kLckCm.
// The cell codes (code - minimum, u16 [16][16], kLcellBlock per block) are a second array of
// T + 1 steps: step 0 holds c0, step t + 1 the cell after step t.  A recurrence member's 64
// units are four consecutive blocks.
constexpr int kLckBlock = 3840, kLckGm = 2048, kLckTanh = 3072, kLckCm = 3584, kLcellBlock = 256;

#if defined(__HIP__)
__host__ __device__ inline uint32_t lck_block(int t, int b, int j, int B, int H) {
  const uint32_t nt = static_cast<uint32_t>(B + 15) / 16;
  return (static_cast<uint32_t>(t) * nt + static_cast<uint32_t>(b) / 16) *
             (static_cast<uint32_t>(H) / 16) + static_cast<uint32_t>(j) / 16;
}
#endif

}  // namespace lstm
}  // namespace rxmet
