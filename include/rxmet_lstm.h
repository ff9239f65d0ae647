/*
 * rxmet_lstm.h — C ABI of the MI355X QuantLSTM (FP32 q-carrier QAT) path.
 *
 * Replaces the entry points of the reference pybind module _quant_lstm
 * (operators/quant-lstm/pytorch/lib/lstm_interface_binding.cc:917-975) on the QAT path:
 *   CalibrationSession.collect (MinMax)  -> rxmet_lstm_forward_calibrate
 *   CalibrationSession.finalize          -> rxmet_lstm_finalize_params
 *     (finalizeQuantParams, src/lstm/quant_params.cc:248-291, calibrateMinMax /
 *      convertScaleToPot2CoverRange, src/quantization/scale_encoding.cc:30-187)
 *   lstm_forward_quantized               -> rxmet_lstm_forward_quant
 *     (lstmForwardQuantizedFpCuda, src/lstm/forward_quantized_fp_cuda.cu; numerics of
 *      lstmForwardQuantizedFpCpuReference, src/lstm/forward_quantized_fp_cpu.cc:67-197)
 *   lstm_backward_qat                    -> rxmet_lstm_backward_quant
 *     (lstmBackwardQat, lstm_interface_binding.cc:437-480 + lstmBackwardFloatCuda,
 *      src/lstm/backward_float_cuda.cu:189-330)
 *   lstm_forward (float)                 -> rxmet_lstm_forward_float
 *
 * Layouts follow the reference: time-major x [T,B,I], output [T,B,H]; PyTorch weights
 * W_ih [4H,I], W_hh [4H,H], biases [4H]; gate order (i, f, g, o).  Quantised values are
 * carried as fp32 codes.  Masks are uint8 with 1 = the value was clamped (the reference's
 * convention for the LSTM), 0 = kept.
 * Every entry point returns 0 on success or a negative status (rxmet_last_error()).
 */
#ifndef RXMET_LSTM_H_
#define RXMET_LSTM_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The 18 real quantisation points (src/lstm/quant_config.h QuantOperator order). */
enum {
  RXMET_LSTM_INPUT = 0,
  RXMET_LSTM_OUTPUT = 1,
  RXMET_LSTM_CELL_STATE = 2,
  RXMET_LSTM_W_IH = 3,
  RXMET_LSTM_W_HH = 4,
  RXMET_LSTM_B_IH = 5,
  RXMET_LSTM_B_HH = 6,
  RXMET_LSTM_IH_LINEAR = 7,
  RXMET_LSTM_HH_LINEAR = 8,
  RXMET_LSTM_I_GATE_IN = 9,
  RXMET_LSTM_F_GATE_IN = 10,
  RXMET_LSTM_G_GATE_IN = 11,
  RXMET_LSTM_O_GATE_IN = 12,
  RXMET_LSTM_I_GATE_OUT = 13,
  RXMET_LSTM_F_GATE_OUT = 14,
  RXMET_LSTM_G_GATE_OUT = 15,
  RXMET_LSTM_O_GATE_OUT = 16,
  RXMET_LSTM_CELL_TANH = 17,
  RXMET_LSTM_NOPS = 18
};

enum { RXMET_LSTM_PER_TENSOR = 0, RXMET_LSTM_PER_GATE = 1, RXMET_LSTM_PER_CHANNEL = 2 };
enum { RXMET_LSTM_AFFINE = 0, RXMET_LSTM_POT2 = 1 };

/* One quantisation point's integer grid and granularity (QuantizationType + granularity,
 * include/quantization/bit_width.h, src/lstm/quant_config.h). */
typedef struct {
  int32_t bits;          /* 1..32 */
  int32_t is_unsigned;
  int32_t is_symmetric;
  int32_t granularity;   /* parameter operators only; others PER_TENSOR */
} rxmet_lstm_op_config;

typedef struct {
  int32_t scale_mode;    /* RXMET_LSTM_AFFINE or RXMET_LSTM_POT2 */
  rxmet_lstm_op_config op[RXMET_LSTM_NOPS];
} rxmet_lstm_config;

/* Finalised standard scales and zero points (LstmQuantParams, include/lstm/quant_params.h).
 * Non-parameter operators use scale[op] / zero_point[op]; the four parameter operators
 * use chan_scale[k][4H] (k = 0..3 for W_IH, W_HH, B_IH, B_HH; caller-owned host arrays,
 * already expanded from their granularity, zero points 0). */
typedef struct {
  int32_t hidden;
  int32_t bias_enabled;
  rxmet_lstm_config config;
  float scale[RXMET_LSTM_NOPS];
  int32_t zero_point[RXMET_LSTM_NOPS];
  float *chan_scale[4];
} rxmet_lstm_params;

/* Execution encodings derived from the standard scales (LstmExecutionParams,
 * src/lstm/lstm_execution_params.cc:236-328).  Exposed for tests. */
typedef struct {
  int32_t is_mshift;   /* 1: v * M * 2^-shift, 0: POT2 v * 2^-shift */
  int32_t multiplier;  /* M in [32768, 65535] when is_mshift */
  int32_t shift;
} rxmet_lstm_rescale;

typedef struct {
  int64_t multiplier;  /* Q31 multiplier when !uses_fp */
  double mantissa;     /* frexp form when the ratio is not Q31-representable */
  int32_t exponent;
  int32_t uses_fp;
} rxmet_lstm_q31;

/* Statistics buffer of the calibration pass (device floats):
 *   [0, 18)           running minimum of each non-parameter operator
 *   [18, 36)          running maximum
 *   then for k in W_IH, W_HH, B_IH, B_HH: chan_min[4H], chan_max[4H]
 *   then one float: count of non-finite values seen (the reference rejects them).
 * Initialise minima to +inf and maxima to -inf and the counter to 0. */
int64_t rxmet_lstm_stats_size(int32_t hidden);

/* MinMax finalisation on the host: stats (host copy) -> params.  Parameter ranges are
 * reduced per granularity; biases get the 2x / 0.01 training headroom; POT2 uses
 * CoverRange with tolerance 0.02.  params->chan_scale must point to 4 arrays of 4H
 * floats.  Fails (with a message) on an empty range, invalid configuration or a
 * non-finite sample count > 0. */
int rxmet_lstm_finalize_params(const float *stats, const rxmet_lstm_config *config,
                               int32_t hidden, int32_t bias_enabled, rxmet_lstm_params *params);

/* Derived execution encodings, for tests: per channel c < 4H the accumulator->linear
 * and bias->accumulator rescales of both linears (index 0: ih, 1: hh), per gate the
 * linear->gate-input rescales, the two Q31 cell ratios and the hidden rescale. */
int rxmet_lstm_derive_exec(const rxmet_lstm_params *params, int32_t input_size,
                           rxmet_lstm_rescale *acc_to_linear /* [2][4H] */,
                           rxmet_lstm_rescale *bias_to_acc /* [2][4H] */,
                           rxmet_lstm_rescale *linear_to_gate /* [2][4] */,
                           rxmet_lstm_q31 *cell /* [2]: forget, input */,
                           rxmet_lstm_rescale *hidden_rescale /* [1] */);

/* Host-side activation tables, for tests (no counterpart in the reference's binding: they
 * expose what rxmet_lstm_forward_quant applies).  The reference's CPU core evaluates its real
 * activations with the C library's expf / tanhf (realSigmoid / realTanh /
 * realActivationQuantizedCore, operators/quant-lstm/src/lstm/cuda/quantized_fp_math.cuh:21-63);
 * the kernels evaluate exp / tanh in double and take the reference's result at the input codes
 * where the two give different output codes.
 * rxmet_lstm_activation_table: entries (output code - output lo) << 1 | clamp mask of
 * activation k (0..3: gates i, f, g, o; 4: tanh of the cell) for every code lo..hi of its
 * input grid (at most 65536 codes), the reference's arithmetic (reference != 0) or the
 * kernels' double evaluation; returns the number of codes or a negative error.
 * rxmet_lstm_activation_exceptions: the exception lists of all five activations (sorted input
 * codes and the reference's entries, copied up to capacity; off/n [5] per activation; grids
 * wider than 65536 codes are not listed); returns the total count or a negative error. */
int32_t rxmet_lstm_activation_table(const rxmet_lstm_params *params, int32_t k, int32_t reference,
                                    uint32_t *entries, int32_t capacity);
int32_t rxmet_lstm_activation_exceptions(const rxmet_lstm_params *params, int32_t *keys,
                                         uint32_t *entries, int32_t capacity,
                                         int32_t *off /* [5] */, int32_t *n /* [5] */);

/* Tensors kept by a training forward for the STE backward (device pointers).
 * Masters: quantised x, W_ih, W_hh, b_ih, b_hh, h0, c0 (h0/c0 quantised from zeros when
 * absent); checkpoints: gate outputs [T,B,4H], cell states, tanh(cell), hidden [T,B,H]
 * (codes); masks: 1 = clamped.  Bias pointers are null when bias is disabled. */
typedef struct {
  float *x_q, *w_ih_q, *w_hh_q, *b_ih_q, *b_hh_q, *h0_q, *c0_q;
  uint8_t *x_m, *w_ih_m, *w_hh_m, *b_ih_m, *b_hh_m, *h0_m, *c0_m;
  float *gate_out, *cell, *cell_tanh, *hidden;
  uint8_t *ih_linear_m, *hh_linear_m, *gate_in_m, *gate_out_m; /* [T,B,4H] */
  uint8_t *cell_m, *cell_tanh_m, *hidden_m;                    /* [T,B,H] */
} rxmet_lstm_saved;

int64_t rxmet_lstm_forward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);

/* Quantised FP32-carrier forward.  x [T,B,I] time-major; h0/c0 [B,H] both or neither.
 * Writes output [T,B,H], h_n, c_n [B,H] dequantised.  With saved != null (training) every
 * pointer in it must be set (bias ones only with bias).  W_hh within signed 16 bits and H a
 * multiple of 16: W_hh of at most 8 bits and H up to 512 run on the int8-MFMA clustered
 * recurrence, wider W_hh or larger H on the stepped recurrence (exact GEMM + pointwise per
 * step). */
int rxmet_lstm_forward_quant(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0,
                             const rxmet_lstm_params *params, float *output, float *h_n,
                             float *c_n, const rxmet_lstm_saved *saved, void *workspace,
                             void *stream);

int64_t rxmet_lstm_backward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);

/* STE backward: dequantises the saved masters/checkpoints and runs the float LSTM
 * backward with the clamp masks (lstmBackwardQat).  grad_output [T,B,H] time-major,
 * grad_h_n / grad_c_n [B,H] (null = zeros).  Writes dx [T,B,I], dW_ih, dW_hh, db_ih,
 * db_hh (null without bias), dh0, dc0 [B,H]. */
int rxmet_lstm_backward_quant(int32_t T, int32_t B, int32_t I, int32_t H,
                              const rxmet_lstm_params *params, const rxmet_lstm_saved *saved,
                              const float *grad_output, const float *grad_h_n,
                              const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                              float *db_ih, float *db_hh, float *dh0, float *dc0,
                              void *workspace, void *stream);

/*
 * Saved state as codes, for callers that keep a training forward's state only to hand it to
 * the backward (the module path).  No counterpart in the reference, whose forward returns the
 * checkpoints as fp32 codes and every mask as a byte (lstm_interface_binding.cc:437-480); the
 * gradients equal those of the reference-format pair bit for bit.  In blocks of 16 sequences x
 * 16 units, block k = (t Bt + b / 16) (H / 16) + j / 16, Bt = ceil(B / 16), row r = b % 16,
 * unit e = j % 16, of 3840 bytes each (blocks: T Bt H/16 of them):
 *   bytes [0, 2048):     u16 [16 r][4 gates][16 e] the gate outputs, code - grid minimum;
 *   bytes [2048, 3072):  u8 [4 gates][16 r][16 e] bit 0 hh-linear mask, bit 1 gate-input mask,
 *                        bit 2 gate-output mask (1 = clamped);
 *   bytes [3072, 3584):  u16 [16 r][16 e] tanh(c), code - grid minimum;
 *   bytes [3584, 3840):  u8 [16 r][16 e] bit 0 cell mask, bit 1 cell-tanh mask, bit 2 hidden mask.
 * cell_codes: u16 [16 r][16 e] per block (code - grid minimum) for T + 1 steps: step 0 c0,
 * step t + 1 the cell after step t ((T + 1) Bt H/16 blocks).  Rows past B are unspecified.
 * Both 16-byte aligned; the gate-output, cell and tanh grids at most 16 bits; H % 16 == 0.
 */
typedef struct {
  uint8_t *blocks;
  uint16_t *cell_codes;
} rxmet_lstm_saved_codes;

/* rxmet_lstm_forward_quant writing codes (non-null with saved) instead of saved->gate_out,
 * cell, cell_tanh and the six recurrence masks (hh_linear_m, gate_in_m, gate_out_m, cell_m,
 * cell_tanh_m, hidden_m), which may be null; every other saved tensor as before. */
int rxmet_lstm_forward_quant_codes(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                                   const float *W_hh, const float *b_ih, const float *b_hh,
                                   const float *x, const float *h0, const float *c0,
                                   const rxmet_lstm_params *params, float *output, float *h_n,
                                   float *c_n, const rxmet_lstm_saved *saved,
                                   const rxmet_lstm_saved_codes *codes, void *workspace,
                                   void *stream);

/* rxmet_lstm_backward_quant reading the codes of rxmet_lstm_forward_quant_codes instead of
 * saved->gate_out, cell, cell_tanh and the six recurrence masks. */
int rxmet_lstm_backward_quant_codes(int32_t T, int32_t B, int32_t I, int32_t H,
                                    const rxmet_lstm_params *params, const rxmet_lstm_saved *saved,
                                    const rxmet_lstm_saved_codes *codes,
                                    const float *grad_output, const float *grad_h_n,
                                    const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                                    float *db_ih, float *db_hh, float *dh0, float *dc0,
                                    void *workspace, void *stream);

int64_t rxmet_lstm_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H);

/* Float LSTM forward that merges MinMax statistics into `stats` (layout above): x, h
 * (including h0, zeros when absent), c (including c0), both linears, the four gate
 * inputs and outputs, tanh(c), per-channel parameter ranges.  Writes output [T,B,H],
 * h_n, c_n. */
int rxmet_lstm_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                                 const float *W_hh, const float *b_ih, const float *b_hh,
                                 const float *x, const float *h0, const float *c0,
                                 float *output, float *h_n, float *c_n, float *stats,
                                 void *workspace, void *stream);

/* Float LSTM forward without statistics (use_quantization=False inference). */
int rxmet_lstm_forward_float(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0, float *output,
                             float *h_n, float *c_n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_LSTM_H_ */
