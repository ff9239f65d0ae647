// gru_internal.h — parameter blocks shared by the host code and the GRU kernels.
#pragma once

#include <cstdint>

#include "rxmet_gru.h"

namespace rxmet {
namespace gru {

constexpr int kSegments = 16;

// Clamp interval of one grid in the fp32 carrier: [fl(qmin), fl(qmax)] pulled inside
// the integer range when fp32 rounding moves an end outwards (>24-bit grids).
struct Bounds {
  float lo, hi;
};

// One activation LUT in carrier form: segment i applies to q < thr[i] (last segment
// catches the rest); y = rint(ldexp(qb[i] * (q - zp_x), -n[i])) + c[i].
struct Lut {
  float thr[kSegments];
  float qb[kSegments];
  int32_t n[kSegments];
  float c[kSegments];
  float zp_x;
};

// Everything the per-step kernels need besides per-channel arrays; passed by value.
struct StepParams {
  int32_t H;
  float zp_x, zp_h, zp_wx, zp_rh;
  float zp_zin, zp_zout, zp_rin, zp_rout, zp_nin, zp_nout;
  // rescale ratios of stored scales (src/gru_forward_gpu_quant_fp.cu:454-516)
  float ih_to_zin, hh_to_zin, ih_to_rin, hh_to_rin, ih_to_nin, rmul_to_nin;
  float quant_one, old_to_h, nout_to_h;
  Bounds x, h, wx, rh, zin, zout, rin, rout, nin, nout;
  Lut lut[3];
  // effective (encoded) scales for boundary quantisation / dequantisation
  float eff_x, eff_h, eff_zout, eff_rout, eff_nout, eff_rh;
};

// ---- int32 carrier (gru_int.hip) ----
// Integer rescale x -> round(x * mult / 2^shift), ties to even on |x| (left shift for
// shift <= 0); mult is the 16-bit mantissa, or 1 in power-of-two mode.
struct IRescale {
  int32_t mult, shift;
};
struct IGrid {
  int32_t lo, hi;
};
// One activation LUT on integer codes: segment i applies to q < thr[i] (the last catches the
// rest); y = rshift_round(qb[i] (q - zp_x), n[i]) + c[i].
struct ILut {
  int32_t thr[kSegments], qb[kSegments], n[kSegments], c[kSegments];
  int32_t zp_x;
};
// The gate parameters of the int32 carrier (setRescaleParam's fillGateParams); by value.
struct IntStepParams {
  int32_t H;
  int32_t zp_x, zp_h, zp_wx, zp_rh, zp_zin, zp_zout, zp_rin, zp_rout, zp_nin, zp_nout;
  IRescale ih_zin, hh_zin, ih_rin, hh_rin, ih_nin, rmul_nin, nout_h, old_h;
  int32_t quant_one;
  IGrid x, h, wx, rh, zin, zout, rin, rout, nin, nout;
  ILut lut[3];
  // effective scales of the boundary quantisation and the dequantised outputs
  float eff_x, eff_h, eff_zout, eff_rout, eff_nout, eff_rh;
};

// Host helpers (gru_params.cpp).
Bounds bounds_of(int32_t bits, int32_t is_unsigned);
float effective_scale(float scale, bool use_pot2);
void make_step_params(const rxmet_gru_qparams &p, int H, StepParams *out);
// Per-channel factors: igx = (S_W[c] S_x)/S_wx, ibx = S_bw[c]/(S_W[c] S_x), same for R/h.
void make_channel_factors(const rxmet_gru_qparams &p, int H, float *igx, float *ibx, float *igh,
                          float *ibh, float *eff_w, float *eff_r, float *eff_bw, float *eff_br);

// int32 carrier: gate parameters, and per channel c the four linear rescales
// rs[c] = (gemm_x -> weight_ih_linear), rs[C + c] = (bw -> S_W S_x), rs[2C + c] =
// (gemm_h -> weight_hh_linear), rs[3C + c] = (br -> S_R S_h).  Throw on scales the
// encodings cannot represent or shifts outside [-32, 62].
IGrid igrid_of(int32_t bits, int32_t is_unsigned);
void make_int_step_params(const rxmet_gru_qparams &p, int H, IntStepParams *out);
void make_int_channel_rescales(const rxmet_gru_qparams &p, int H, IRescale *rs);

}  // namespace gru
}  // namespace rxmet
