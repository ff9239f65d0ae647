/*
 * rxmet_gru.h — C ABI of the MI355X QuantGRU (FP32-carrier QAT) path.
 *
 * Replaces the entry points of the reference pybind module gru_interface_binding
 * (operators/quant-gru/pytorch/lib/gru_interface_binding.cc:1331-1788) that the
 * QAT path uses:
 *   calculate_gru_quantitative_parameters -> rxmet_gru_make_params
 *   forward_calibrate (MINMAX)            -> rxmet_gru_forward_calibrate
 *   forward_fp (inference)                -> rxmet_gru_forward_fp
 *   forward_quant_float_storage           -> rxmet_gru_forward_quant
 *   backward_quant_float_storage          -> rxmet_gru_backward_quant
 *   forward_quant_int_storage             -> rxmet_gru_forward_quant_int
 *   backward_quant_int_storage            -> rxmet_gru_backward_quant on the int32 codes
 *                                            converted to fp32 (as the binding does)
 *   forward_quantized_int_io              -> rxmet_gru_forward_int_io
 *   (LUT regeneration in GRUQuantParamsPy::to_cpp) -> rxmet_gru_make_luts
 *
 * Conventions (all as in the reference):
 *   - Gate order inside a 3H block is (z, r, n) ("haste" order); W is [I, 3H], R is
 *     [H, 3H], biases [3H]; x is [T, B, I], h0 [B, H] (row-major fp32).
 *   - Quantized values are integer codes stored in fp32; masks are uint8 with
 *     1 = keep gradient (value was not clamped).
 *   - Boundary quantisation (x, h0, W, R, biases) and all dequantisation use the
 *     effective scale decode(encode(scale)) (16-bit mantissa M * 2^-shift, or the
 *     power of two itself); the in-loop rescales use ratios of the stored scales.
 *
 * Device entry points take device pointers and a hipStream_t (as void*), enqueue work on
 * that stream and return 0 or a negative status (message in rxmet_last_error()).  They
 * never allocate: scratch memory comes from a caller workspace of the size the matching
 * *_workspace_bytes() function returns.
 */
#ifndef RXMET_GRU_H_
#define RXMET_GRU_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scalar operator grids, in this order (reference: quantize_param_types.h:65-142). */
enum {
  RXMET_GRU_X = 0,            /* input x                        */
  RXMET_GRU_H = 1,            /* hidden state / output          */
  RXMET_GRU_WX = 2,           /* weight_ih_linear = W x + bw    */
  RXMET_GRU_RH = 3,           /* weight_hh_linear = R h + br    */
  RXMET_GRU_Z_IN = 4,         /* update_gate_input              */
  RXMET_GRU_R_IN = 5,         /* reset_gate_input               */
  RXMET_GRU_N_IN = 6,         /* new_gate_input                 */
  RXMET_GRU_Z_OUT = 7,        /* update_gate_output             */
  RXMET_GRU_R_OUT = 8,        /* reset_gate_output              */
  RXMET_GRU_N_OUT = 9,        /* new_gate_output                */
  RXMET_GRU_MUL_RH = 10,      /* mul_reset_hidden               */
  RXMET_GRU_MUL_NEW = 11,     /* mul_new_contribution           */
  RXMET_GRU_MUL_OLD = 12,     /* mul_old_contribution           */
  RXMET_GRU_NGRIDS = 13
};

/* Per-channel operators (weights / biases), in this order. */
enum { RXMET_GRU_W = 0, RXMET_GRU_R = 1, RXMET_GRU_BW = 2, RXMET_GRU_BR = 3, RXMET_GRU_NCHAN = 4 };

enum { RXMET_PER_TENSOR = 0, RXMET_PER_GATE = 1, RXMET_PER_CHANNEL = 2 };
enum { RXMET_POT_ROUND = 0, RXMET_POT_COVER_RANGE = 1, RXMET_POT_FLOOR = 2 };

/* Bit-width configuration of one operator (QuantBitWidth + symmetric flag). */
typedef struct rxmet_bitspec {
  int32_t bits;        /* 1..32 */
  int32_t is_unsigned; /* 0: signed grid, 1: unsigned grid */
  int32_t symmetric;   /* 1: zero point forced to 0 */
  int32_t granularity; /* RXMET_PER_*; used by the per-channel operators only */
} rxmet_bitspec;

/* OperatorQuantConfig (quantize_bitwidth_config.h:56-122). */
typedef struct rxmet_gru_config {
  rxmet_bitspec op[RXMET_GRU_NGRIDS];
  rxmet_bitspec chan[RXMET_GRU_NCHAN];
  int32_t use_pot2;
  int32_t pot_method;  /* RXMET_POT_* */
  float pot_tolerance; /* default 0.02 */
} rxmet_gru_config;

/* GRUQuantizationRanges (gru_quantization_ranges.h): scalar min/max per grid and
 * per-channel min/max arrays of length 3H (host memory). */
typedef struct rxmet_gru_ranges {
  int32_t hidden;
  float min[RXMET_GRU_NGRIDS];
  float max[RXMET_GRU_NGRIDS];
  float *chan_min[RXMET_GRU_NCHAN];
  float *chan_max[RXMET_GRU_NCHAN];
} rxmet_gru_ranges;

/* One operator grid: stored scale (continuous, or 2^-n in power-of-two mode), zero
 * point and bit width. */
typedef struct rxmet_grid {
  float scale;
  int32_t zero_point;
  int32_t bits;
  int32_t is_unsigned;
} rxmet_grid;

/* GRUQuantParams (quantize_param_types.h:88-118) without the LUTs; the per-channel
 * scales live in host arrays chan_scale[k] of length 3H (zero points are 0). */
typedef struct rxmet_gru_qparams {
  int32_t hidden;
  int32_t use_pot2;
  rxmet_grid g[RXMET_GRU_NGRIDS];
  int32_t chan_bits[RXMET_GRU_NCHAN];
  int32_t chan_unsigned[RXMET_GRU_NCHAN];
  float *chan_scale[RXMET_GRU_NCHAN];
} rxmet_gru_qparams;

/* One segment of a 16-segment piecewise-linear activation (SegmentParams,
 * quantize_lut_types.h:20-25): y = rint((q_b * (q - zp_x)) * 2^-n) + c for q < threshold. */
typedef struct rxmet_pwl_segment {
  int32_t q_b;
  int32_t n;
  int32_t c;
  int32_t threshold;
} rxmet_pwl_segment;

typedef struct rxmet_pwl_lut {
  rxmet_pwl_segment seg[16];
  int32_t zp_x;
} rxmet_pwl_lut;

/*
 * Quantisation parameters from calibration ranges: calculateGRUQuantitativeParameters
 * (operators/quant-gru/src/gru_host.cc:13-124) with encodeFromRange / calibrateBias /
 * ensureMinRange (include/gru_calibration_helpers.h:15-61, calibration_utils.h:27-44).
 * Host only.  out->chan_scale[k] must point at caller arrays of 3H floats.
 * Weights and biases must be configured symmetric (gru_calibration_helpers.h:7-13).
 */
int rxmet_gru_make_params(const rxmet_gru_ranges *ranges, const rxmet_gru_config *config,
                          rxmet_gru_qparams *out);

/*
 * The three activation LUTs the forward uses, rebuilt from the stored scales
 * (generate_piecewise_linear_lut_to_params, src/quantize_lut.cc:16-48): out[0] sigmoid
 * of the update gate, out[1] sigmoid of the reset gate, out[2] tanh of the new gate.
 * Host only.
 */
int rxmet_gru_make_luts(const rxmet_gru_qparams *params, rxmet_pwl_lut out[3]);

/* Effective scale the kernels use for a stored scale (decode(encode(s))). Host only. */
float rxmet_gru_effective_scale(float scale, int32_t use_pot2);

/* Workspace bytes of rxmet_gru_forward_quant / rxmet_gru_backward_quant. */
int64_t rxmet_gru_forward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);
int64_t rxmet_gru_backward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);

/*
 * Quantised forward, FP32 carrier: quantGRUForwardFP (src/gru_interface.cc:636-716)
 * behind forward_quant_float_storage_wrapper (gru_interface_binding.cc:306-448).
 * Outputs (device, caller-allocated, shapes as the binding returns them):
 *   h [T+1, B, H] dequantised hidden states (h[0] = dequantised h0),
 *   v [T, B, 4H]  dequantised (z, r, n, weight_hh_linear_n) per step,
 *   W_q [I,3H], R_q [H,3H], bw_q [3H], br_q [3H], x_q [T,B,I] codes,
 * and when is_training != 0 the uint8 masks (else they may be null):
 *   x_mask [T,B,I], h0_mask [B,H] (null when h0 is null), W_mask [I,3H], R_mask [H,3H],
 *   bw_mask [3H], br_mask [3H], ih_mask, hh_mask, gate_in_mask, gate_out_mask [T,B,3H],
 *   h_mask [T,B,H].
 * h0 may be null (state starts at the zero point of h).
 */
int rxmet_gru_forward_quant(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                            const float *W, const float *R, const float *bw, const float *br,
                            const float *x, const float *h0, const rxmet_gru_qparams *params,
                            float *h, float *v, float *W_q, float *R_q, float *bw_q, float *br_q,
                            float *x_q, uint8_t *x_mask, uint8_t *h0_mask, uint8_t *W_mask,
                            uint8_t *R_mask, uint8_t *bw_mask, uint8_t *br_mask, uint8_t *ih_mask,
                            uint8_t *hh_mask, uint8_t *gate_in_mask, uint8_t *gate_out_mask,
                            uint8_t *h_mask, void *workspace, void *stream);

/*
 * Both directions of a bidirectional layer in one call.  No counterpart in the reference,
 * which calls forward_quant_float_storage once per direction; it is for QuantGRU's
 * bidirectional forward: the per-direction prologues run first, then one clustered
 * recurrence launch covers both directions so their sequential steps overlap.  dirs[k]
 * holds exactly the arguments of one rxmet_gru_forward_quant call (its own workspace of
 * rxmet_gru_forward_workspace_bytes(T, B, I, H) bytes); the results equal ndir separate
 * calls.  ndir is 1 or 2.
 */
typedef struct rxmet_gru_fwd_dir {
  const float *W, *R, *bw, *br, *x, *h0;
  const rxmet_gru_qparams *params;
  float *h, *v, *W_q, *R_q, *bw_q, *br_q, *x_q;
  uint8_t *x_mask, *h0_mask, *W_mask, *R_mask, *bw_mask, *br_mask, *ih_mask, *hh_mask,
      *gate_in_mask, *gate_out_mask, *h_mask;
  void *workspace;
} rxmet_gru_fwd_dir;

int rxmet_gru_forward_quant_dirs(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                 int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                 void *stream);

/*
 * rxmet_gru_forward_quant_dirs with each direction's x read in place from the caller's input
 * and, optionally, the weights read in PyTorch's layout.  No counterpart in the reference, whose
 * QuantGRU transposes batch-first input, flips it for the reverse direction and reorders the
 * weights with tensor copies (quant_gru.py:714-759, 2151-2205, 2270-2288).
 * x_layout[4 k .. 4 k + 3] = {t stride, b stride, reversed, flags} of direction k in elements
 * (the feature stride is 1): element (t, b, i) of the direction is x[t' st + b sb + i] with
 * t' = reversed ? T-1-t : t.  flags bit 0: W, R, bw, br are PyTorch's weight_ih [3H, I],
 * weight_hh [3H, H], bias_ih, bias_hh in (r, z, n) gate order instead of [I, 3H], [H, 3H] in
 * (z, r, n).  x_q, x_mask, W_q and everything else come out as in rxmet_gru_forward_quant_dirs,
 * in the direction's own [T, B, .] order and the (z, r, n) layouts.  T*B*I < 2^32.
 */
int rxmet_gru_forward_quant_dirs_x(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                   int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                   const int64_t *x_layout, void *stream);

/*
 * Output assembly of a bidirectional layer in one pass; replaces the reference's
 * torch.cat([out_f, out_r.flip(0)], -1) / torch.cat([hn_f, hn_r]) (quant_gru.py:1402-1432)
 * and the batch-first transpose after it.  h_f, h_r: [T+1, B, H] of each direction (row 0 = h0);
 * out element (t, b, k < 2H) at out[t out_st + b out_sb + k] = k < H ? h_f[t+1][b][k] :
 * h_r[T-t][b][k-H]; h_n [2, B, H] (may be null) = {h_f[T], h_r[T]}.  H, out_st and out_sb
 * multiples of 4, pointers 16-byte aligned.
 */
int rxmet_gru_bidir_assemble(int32_t T, int32_t B, int32_t H, const float *h_f, const float *h_r,
                             float *out, int64_t out_st, int64_t out_sb, float *h_n, void *stream);

/*
 * The backward of rxmet_gru_bidir_assemble: writes each direction's dh_new [T+1, B, H]
 * (row 0 zero) from the output gradient g (element (t, b, k) at g[t g_st + b g_sb + k g_sk],
 * strides may be zero, g may be null) and the h_n gradient g_hn ([2, B, H] contiguous, may be
 * null): dh_f[t+1][b][j] = g(t, b, j), dh_r[s+1][b][j] = g(T-1-s, b, H+j), plus g_hn at the last
 * row.  H a multiple of 4, dh_f and dh_r 16-byte aligned.  Replaces the reference's zero-fill
 * and slice copies of the upstream gradient.
 */
int rxmet_gru_bidir_split_grad(int32_t T, int32_t B, int32_t H, const float *g, int64_t g_st,
                               int64_t g_sb, int64_t g_sk, const float *g_hn, float *dh_f,
                               float *dh_r, void *stream);

/*
 * Input gradient of a bidirectional layer in the caller's layout: dx[t dx_st + b dx_sb + i] =
 * dx_f[t][b][i] + dx_r[T-1-t][b][i] (dx_f, dx_r [T, B, I] from the two directions' backward).
 * Replaces the reference's dx_f + dx_r.flip(0) and the batch-first transpose.
 */
int rxmet_gru_bidir_dx(int32_t T, int32_t B, int32_t I, const float *dx_f, const float *dx_r,
                       float *dx, int64_t dx_st, int64_t dx_sb, void *stream);

/*
 * Quantised backward: backward_quant_float_storage_wrapper
 * (gru_interface_binding.cc:789-920) + quantGRUBackward / BackwardPassQuant::Run
 * (src/gru_backward_gpu_quant.cu:379-493).  Inputs are the forward's outputs; unlike
 * the reference the saved codes are not modified.  dh_new [T+1, B, H] is the upstream
 * gradient of h (dh_new[0] unused).  Outputs (device, caller-allocated):
 *   dx [T,B,I], dW [I,3H], dR [H,3H], dbw [3H], dbr [3H], dh0 [B,H].
 * Mask pointers may be null (no masking for that tensor), as in the reference.
 */
int rxmet_gru_backward_quant(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_q,
                             const float *R_q, const float *bw_q, const float *br_q,
                             const float *x_q, const float *dh_new, const float *h,
                             const float *v, const rxmet_gru_qparams *params,
                             const uint8_t *x_mask, const uint8_t *h0_mask,
                             const uint8_t *W_mask, const uint8_t *R_mask,
                             const uint8_t *bw_mask, const uint8_t *br_mask,
                             const uint8_t *ih_mask, const uint8_t *hh_mask,
                             const uint8_t *gate_in_mask, const uint8_t *gate_out_mask,
                             const uint8_t *h_mask, float *dx, float *dW, float *dR, float *dbw,
                             float *dbr, float *dh0, void *workspace, void *stream);

/*
 * Both directions' backward in one call (no counterpart in the reference, which calls
 * backward_quant_float_storage once per direction): one clustered recurrence launch covers
 * both directions, then each direction's bias fold, weight-gradient GEMMs and masks.
 * dirs[k] holds exactly the arguments of one rxmet_gru_backward_quant call; the results
 * equal ndir separate calls.  ndir is 1 or 2.
 */
typedef struct rxmet_gru_bwd_dir {
  const float *W_q, *R_q, *bw_q, *br_q, *x_q, *dh_new, *h, *v;
  const rxmet_gru_qparams *params;
  const uint8_t *x_mask, *h0_mask, *W_mask, *R_mask, *bw_mask, *br_mask, *ih_mask, *hh_mask,
      *gate_in_mask, *gate_out_mask, *h_mask;
  float *dx, *dW, *dR, *dbw, *dbr, *dh0;
  void *workspace;
} rxmet_gru_bwd_dir;

int rxmet_gru_backward_quant_dirs(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                  const rxmet_gru_bwd_dir *dirs, void *stream);

/*
 * rxmet_gru_backward_quant_dirs with, for flags bit 0, the weight gradients written in
 * PyTorch's layout: dW [3H, I], dR [3H, H], dbw, dbr [3H] in (r, z, n) gate order (W and R
 * masks applied as before).  No counterpart in the reference, which reorders the gradients
 * with tensor copies (quant_gru.py:689-702).
 */
int rxmet_gru_backward_quant_dirs_x(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                    const rxmet_gru_bwd_dir *dirs, int32_t flags, void *stream);

/*
 * Saved state as codes, for callers that keep the forward's state only to hand it to the
 * backward (the module path).  No counterpart in the reference, whose forward returns v in
 * fp32 and one byte per mask value (gru_interface_binding.cc:306-448); the gradients equal
 * those of the reference-format pair bit for bit (v is dequantised in the backward with the
 * same (code - zero point) * effective scale).  Per direction, in blocks of 16 sequences x 16
 * units so that a recurrence workgroup writes each step's codes as one contiguous run: block
 * k = (t Bt + b / 16) (H / 16) + j / 16, Bt = ceil(B / 16), row r = b % 16, unit e = j % 16:
 *   v_codes   [T Bt 16 4H]: element (t, b, field f, j) at 1024 k + 64 r + 16 f + e; fields
 *             f = 0..3 the update, reset and new gate outputs and the new gate's recurrent
 *             linear (z, r, n, hh_n), each as its code minus its grid's minimum;
 *   mask_bits [T Bt 16 H]: element (t, b, j) at 256 k + 16 r + e; bit g (gate g = z, r, n) the
 *             weight_ih_linear mask, 3 + g the weight_hh_linear mask, 6 + g the gate input
 *             mask, 9 + g the gate output mask, 12 the h mask.
 * Both 16-byte aligned; rows past B hold unspecified values.  The four grids must span at most
 * 16 bits.  H a multiple of 16.
 */
typedef struct rxmet_gru_saved_codes {
  uint16_t *v_codes;
  uint16_t *mask_bits;
} rxmet_gru_saved_codes;

/*
 * rxmet_gru_forward_quant_dirs_x (x_layout may be null: [T, B, I] contiguous per direction)
 * writing, when is_training, codes[k] instead of dirs[k].v and the five per-step mask
 * families (ih, hh, gate in, gate out, h), which may then be null; the x, h0, W, R, bw and br
 * masks and every other output as before.
 */
int rxmet_gru_forward_quant_dirs_codes(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                       int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                       const int64_t *x_layout, const rxmet_gru_saved_codes *codes,
                                       void *stream);

/*
 * rxmet_gru_backward_quant_dirs_x (flags as there) reading codes[k] from
 * rxmet_gru_forward_quant_dirs_codes instead of dirs[k].v and the five per-step mask families
 * (which may be null).
 */
/*
 * A direction's incoming gradient read in place from the layer's output gradient instead of a
 * dh_new buffer [T+1, B, H]: row s + 1 of dh_new is g at element (t, b, col0 + j), t = s (or
 * T - 1 - s for a reverse direction), element (t, b, k) at g[t st + b sb + k sk] (any strides,
 * zero included), plus g_hn[b H + j] (the gradient of the direction's h_n, [B, H] contiguous)
 * at s = T - 1; row 0 is zero.  g or g_hn may be null (zero).  No counterpart in the reference,
 * which builds dh_new with tensor copies (quant_gru.py:2207-2288).
 */
typedef struct rxmet_gru_grad_view {
  const float *g;
  int64_t st, sb, sk;
  int32_t col0, reverse;
  const float *g_hn;
} rxmet_gru_grad_view;

/* views: null, or one per direction (dirs[k].dh_new is then not read and may be null). */
int rxmet_gru_backward_quant_dirs_codes(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                        const rxmet_gru_bwd_dir *dirs, int32_t flags,
                                        const rxmet_gru_saved_codes *codes,
                                        const rxmet_gru_grad_view *views, void *stream);

/*
 * Quantised forward, int32 carrier: quantGRUForwardInt (src/gru_interface.cc:443-559) behind
 * forward_quant_int_storage_wrapper (gru_interface_binding.cc:451-586), i.e. ForwardPassQuant
 * (src/gru_forward_gpu_quant.cu) and the reference's CPU carrier (src/gru_forward_cpu_quant.cc:
 * 109-343).  Every value between the boundaries is an integer code: GEMM sums exact in int64
 * with the bias rescaled into the accumulator scale, rescales rshift_round(x M, shift) (16-bit
 * mantissa M, or shifts only in power-of-two mode), integer PWL gates.  Arguments and outputs as
 * rxmet_gru_forward_quant, except that W_q [I,3H], R_q [H,3H], bw_q, br_q [3H] and x_q [T,B,I]
 * are int32 codes; h [T+1,B,H] and v [T,B,4H] are dequantised with the effective scales.
 * x, h0 (both may carry any values), W and R in the kernel layout; x and h grids of at most
 * 16 bits, W and R codes within signed 16 bits.  Any hidden size.  Workspace:
 * rxmet_gru_forward_int_workspace_bytes.
 */
int64_t rxmet_gru_forward_int_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);
int rxmet_gru_forward_quant_int(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                                const float *W, const float *R, const float *bw, const float *br,
                                const float *x, const float *h0, const rxmet_gru_qparams *params,
                                float *h, float *v, int32_t *W_q, int32_t *R_q, int32_t *bw_q,
                                int32_t *br_q, int32_t *x_q, uint8_t *x_mask, uint8_t *h0_mask,
                                uint8_t *W_mask, uint8_t *R_mask, uint8_t *bw_mask,
                                uint8_t *br_mask, uint8_t *ih_mask, uint8_t *hh_mask,
                                uint8_t *gate_in_mask, uint8_t *gate_out_mask, uint8_t *h_mask,
                                void *workspace, void *stream);

/*
 * Integer-in, integer-out inference: quantGRUForwardIntIO (src/gru_interface.cc:561-627) behind
 * forward_quantized_int_io_wrapper (gru_interface_binding.cc:588-646).  x_q [T,B,I] and h0_q
 * [B,H] (may be null: the zero point of h) are int32 codes on the x and h grids, used as they
 * are; only the weights are quantised (W_q, R_q, bw_q, br_q written as in
 * rxmet_gru_forward_quant_int).  Writes the int32 h codes h_q [T+1,B,H] (row 0 = h0_q); the
 * reference's output_q and h_n_q are rows 1..T and row T.  Codes outside the x / h grids are
 * rejected (-22); that check synchronises the stream once.  Workspace:
 * rxmet_gru_forward_int_workspace_bytes.
 */
int rxmet_gru_forward_int_io(int32_t T, int32_t B, int32_t I, int32_t H, const float *W,
                             const float *R, const float *bw, const float *br,
                             const int32_t *x_q, const int32_t *h0_q,
                             const rxmet_gru_qparams *params, int32_t *h_q, int32_t *W_q,
                             int32_t *R_q, int32_t *bw_q, int32_t *br_q, void *workspace,
                             void *stream);

/*
 * Both directions of a bidirectional layer on the int32 carrier in one call.  No counterpart
 * in the reference, which calls forward_quant_int_storage / forward_quantized_int_io once per
 * direction (quant_gru.py:2207-2288, 2482-2537): the per-direction prologues run first, then
 * one clustered recurrence launch covers both directions so their sequential steps overlap
 * (each direction stepped where the clustered form does not apply).  dirs[k] holds exactly the
 * arguments of one rxmet_gru_forward_quant_int call (x_q_in == null) or one
 * rxmet_gru_forward_int_io call (x_q_in != null: x_q_in, h0_q_in, h_q as x_q, h0_q, h_q there;
 * is_training must be 0), with its own workspace of rxmet_gru_forward_int_workspace_bytes
 * bytes; the results equal ndir separate calls.  ndir is 1 or 2; both directions have the same
 * kind.
 */
typedef struct rxmet_gru_int_dir {
  const float *W, *R, *bw, *br, *x, *h0;
  const int32_t *x_q_in, *h0_q_in;
  const rxmet_gru_qparams *params;
  float *h, *v;
  int32_t *h_q, *W_q, *R_q, *bw_q, *br_q, *x_q;
  uint8_t *x_mask, *h0_mask, *W_mask, *R_mask, *bw_mask, *br_mask, *ih_mask, *hh_mask,
      *gate_in_mask, *gate_out_mask, *h_mask;
  void *workspace;
} rxmet_gru_int_dir;

int rxmet_gru_forward_quant_int_dirs(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                     int32_t I, int32_t H, const rxmet_gru_int_dir *dirs,
                                     void *stream);

/*
 * Float GRU forward with MinMax calibration statistics: forwardWithCalibrationGPU
 * (src/gru_interface.cc:930-1024) / forwardWithCalibrationCPU
 * (src/gru_forward_cpu.cc:58-151).  Writes h [T+1,B,H] and v [T,B,4H] (float values)
 * and merges (min/max-accumulates) the statistics into stats, a device array of
 * 2*13 + 8*3H floats laid out as: min[13], max[13], then for k in W,R,bw,br:
 * chan_min_k[3H], chan_max_k[3H].  Initialise stats with +FLT_MAX / -FLT_MAX before the
 * first call.  h0 may be null.  Non-finite values are ignored, as in the reference.
 */
int64_t rxmet_gru_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);
int rxmet_gru_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W,
                                const float *R, const float *bw, const float *br,
                                const float *x, const float *h0, float *h, float *v,
                                float *stats, void *workspace, void *stream);

/*
 * Float GRU forward without quantisation: forward_fp
 * (pytorch/lib/gru_interface_binding.cc:656-697, hasteGRUForward).  Same kernel and
 * summation order as rxmet_gru_forward_calibrate, no statistics.  Writes h [T+1,B,H]
 * and, when is_training is non-zero, v [T,B,4H] (z, r, n, hh_n); v may be null
 * otherwise.  h0 may be null (zeros).  Needs no workspace.
 */
int rxmet_gru_forward_fp(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                         const float *W, const float *R, const float *bw, const float *br,
                         const float *x, const float *h0, float *h, float *v, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_GRU_H_ */
