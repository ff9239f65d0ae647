/*
 * rxmet_qc.h — C ABI of the ONNX Runtime custom op QcQuantizeOp on MI355X: the reference's
 * ORT plugin (native/onnx/src/QcQuantizeOp.cpp, AimetOpUtils.h, QcQuantizeInfo.h) with its
 * TF-scheme (min / max) BlockTensorQuantizer (native/common/src/TensorQuantizer.cpp:348-469,
 * MinMaxEncodingAnalyzer.cpp, quantization_utils.cpp:59-119, trim_functions.cpp:646-713).
 *
 * The quantizer's statistics and encodings live in device memory of the GPU that was current
 * when it was created, so an op call enqueues its kernels on the caller's stream and does not
 * wait for them: statistics, encoding computation and the quantize-dequantize pass follow
 * each other on that stream.  Only the getters that return values to the host synchronize.
 *
 * Every entry point returns 0 on success or a negative status, with the message in
 * rxmet_last_error() (rxmet_qdq.h), where the reference throws std::runtime_error — the ORT
 * glue turns it into an OrtStatus as RegisterCustomOps.cpp:47-51 does for exceptions.
 *
 * Tensors: f32 or f16 (RXMET_QDQ_F32 / RXMET_QDQ_F16 of rxmet_qdq.h), row-major, device
 * memory.  An f16 tensor is widened exactly to f32, computed on and rounded back to f16 to
 * nearest even, which is what the reference's Float16 kernels do through f32 buffers
 * (QcQuantizeOp.cpp:110-160).
 */
#ifndef RXMET_QC_H_
#define RXMET_QC_H_

#include <stdint.h>

#include "rxmet_qdq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* TensorQuantizerOpMode (native/common/include/DlQuantization/TensorQuantizerOpFacade.h:48-54). */
enum {
  RXMET_QC_UPDATE_STATS = 0,
  RXMET_QC_ONE_SHOT_QUANTIZE_DEQUANTIZE = 1,
  RXMET_QC_QUANTIZE_DEQUANTIZE = 2,
  RXMET_QC_PASS_THROUGH = 3,
};

/* TfEncoding (native/common/include/DlQuantization/Quantization.hpp:114-121). */
typedef struct rxmet_tf_encoding {
  double min, max, delta, offset;
  int32_t bw;
  int32_t reserved; /* 0 */
} rxmet_tf_encoding;

/*
 * BlockTensorQuantizer(shape, bitwidth, QUANTIZATION_TF) (TensorQuantizer.h:265-345,
 * TensorQuantizer.cpp:348-360): one encoding per element of `shape` (the encoding shape;
 * ndim 0 = per tensor), statistics from MinMaxEncodingAnalyzer<float>.  An encoding shape
 * broadcasts against a tensor shape as getBroadcastableShapes does (tensor_utils.cpp:62-88:
 * aligned on the right; an encoding dimension equal to the tensor's, 1, or dividing it into
 * blocks); the encodings may form at most two groups of adjacent dimensions (per-channel,
 * block, and channel + block encodings do).  Created on the current device; NULL on error.
 */
typedef struct rxmet_block_tensor_quantizer rxmet_block_tensor_quantizer;

rxmet_block_tensor_quantizer *rxmet_block_tensor_quantizer_create(const int64_t *shape,
                                                                  int32_t ndim,
                                                                  int32_t bitwidth);
void rxmet_block_tensor_quantizer_destroy(rxmet_block_tensor_quantizer *q);

/* Flags and state (TensorQuantizer.cpp:414-434: setting a flag invalidates the encodings). */
typedef struct rxmet_block_tensor_quantizer_state {
  int64_t num_encodings;
  int32_t bitwidth;
  int32_t use_strict_symmetric;
  int32_t use_unsigned_symmetric;
  int32_t valid_stats;       /* updateStats called since the last reset */
  int32_t is_encoding_valid; /* encodings set */
  int32_t reserved;
} rxmet_block_tensor_quantizer_state;

int rxmet_block_tensor_quantizer_get_state(const rxmet_block_tensor_quantizer *q,
                                           rxmet_block_tensor_quantizer_state *out);
int rxmet_block_tensor_quantizer_set_strict_symmetric(rxmet_block_tensor_quantizer *q,
                                                      int32_t on);
int rxmet_block_tensor_quantizer_set_unsigned_symmetric(rxmet_block_tensor_quantizer *q,
                                                        int32_t on);
int rxmet_block_tensor_quantizer_set_bitwidth(rxmet_block_tensor_quantizer *q, int32_t bw);

/* Workspace bytes update_stats needs for a tensor of this shape and type (0 if none). */
int64_t rxmet_block_tensor_quantizer_workspace_bytes(const rxmet_block_tensor_quantizer *q,
                                                     const int64_t *shape, int32_t ndim,
                                                     int32_t io_dtype);

/* resetEncodingStats (TensorQuantizer.cpp:362-367): statistics to (+max, lowest), no valid
 * stats or encodings. */
int rxmet_block_tensor_quantizer_reset_encoding_stats(rxmet_block_tensor_quantizer *q,
                                                      void *stream);

/* updateStats (TensorQuantizer.cpp:369-376, ContiguousEncodingAnalyzer.cpp:46-97,
 * MinMaxEncodingAnalyzer.cpp:57-70): each encoding's running min / max takes the min / max of
 * its block of x; NaN elements are skipped (math_functions.cpp:356-375).  workspace: device
 * memory of rxmet_block_tensor_quantizer_workspace_bytes(), or NULL for a buffer the quantizer
 * allocates on first need and keeps (grown when a larger tensor arrives). */
int rxmet_block_tensor_quantizer_update_stats(rxmet_block_tensor_quantizer *q, const void *x,
                                              int32_t io_dtype, const int64_t *shape,
                                              int32_t ndim, void *workspace, void *stream);

/* computeEncodings(useSymmetricEncodings) followed by setEncodings
 * (TensorQuantizer.cpp:451-469, MinMaxEncodingAnalyzer.cpp:72-96 with getComputedEncodings,
 * quantization_utils.cpp:59-119), on the device in double arithmetic. */
int rxmet_block_tensor_quantizer_compute_encodings(rxmet_block_tensor_quantizer *q,
                                                   int32_t use_symmetric, void *stream);

/* setEncodings / getEncodings of n = num_encodings TfEncodings (host memory; set takes the
 * bitwidth of enc[0], TensorQuantizer.cpp:461-469).  get synchronizes the stream. */
int rxmet_block_tensor_quantizer_set_encodings(rxmet_block_tensor_quantizer *q,
                                               const rxmet_tf_encoding *enc, int64_t n,
                                               void *stream);
int rxmet_block_tensor_quantizer_get_encodings(const rxmet_block_tensor_quantizer *q,
                                               rxmet_tf_encoding *enc, int64_t n, void *stream);
/* The running statistics (host memory, n = num_encodings); synchronizes the stream. */
int rxmet_block_tensor_quantizer_get_stats(const rxmet_block_tensor_quantizer *q, float *min,
                                           float *max, int64_t n, void *stream);

/* quantizeDequantize (TensorQuantizer.cpp:379-397): y = stableQuantizeDequantize(x, min, max,
 * delta) of x's encoding (quantize_dequantize.hpp:35-46: NaN kept, clip to [min, max], times
 * the correctly rounded fp32 1 / delta, round half to even, times delta; min, max and delta of
 * the double encoding rounded to fp32).  Error before encodings are set. */
int rxmet_block_tensor_quantizer_quantize_dequantize(const rxmet_block_tensor_quantizer *q,
                                                     const void *x, void *y, int32_t io_dtype,
                                                     const int64_t *shape, int32_t ndim,
                                                     void *stream);

/*
 * QcQuantizeInfo (native/onnx/src/QcQuantizeInfo.h:40-75): the per-node state the ONNX graph
 * refers to through the int64 attribute "quant_info" (the struct's address), owned by the
 * caller.  tensor_quantizer may be NULL for a float (fp16 round trip) quantizer.
 * use_per_channel_mode, channel_axis, block_axis and block_size describe how the caller built
 * the quantizer's shape; the op itself only reads the quantizer.
 */
typedef struct rxmet_qc_quantize_info {
  rxmet_block_tensor_quantizer *tensor_quantizer;
  int32_t op_mode; /* RXMET_QC_* */
  int32_t use_symmetric_encoding;
  int32_t enabled;
  int32_t is_int_data_type;
  int32_t use_per_channel_mode;
  int32_t channel_axis;
  int32_t block_axis;
  int32_t reserved; /* 0 */
  int64_t block_size;
  const char *name;
} rxmet_qc_quantize_info;

/*
 * QcQuantizeOp::computeImpl (QcQuantizeOp.cpp:101-170) with modeSpecificActionBroadcastInt /
 * modeSpecificActionFloat (AimetOpUtils.h:58-128) on one tensor:
 *   disabled              -> pass through (a copy);
 *   int data type:  updateStats -> update statistics, copy;  oneShotQuantizeDequantize ->
 *                   reset statistics, update, compute + set encodings, quantize-dequantize;
 *                   quantizeDequantize -> quantize-dequantize;  passThrough -> copy;
 *   float data type: (oneShot)quantizeDequantize -> round to fp16 and back; otherwise copy.
 * After a oneShotQuantizeDequantize call op_mode becomes RXMET_QC_QUANTIZE_DEQUANTIZE (a
 * disabled node keeps its mode).  workspace as for update_stats.
 */
int rxmet_qc_quantize_compute(rxmet_qc_quantize_info *info, const void *x, void *y,
                              int32_t io_dtype, const int64_t *shape, int32_t ndim,
                              void *workspace, void *stream);
int64_t rxmet_qc_quantize_workspace_bytes(const rxmet_qc_quantize_info *info,
                                          const int64_t *shape, int32_t ndim, int32_t io_dtype);

/* The [outer, C0, mid, C1, inner] layout (rxmet_qdq.h) of a tensor against an encoding
 * shape, as the calls above address it; an error when the shapes do not broadcast or need
 * more than two encoding groups. */
int rxmet_qc_broadcast_layout(const int64_t *shape, int32_t ndim, const int64_t *enc_shape,
                              int32_t enc_ndim, rxmet_qdq_layout *out);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_QC_H_ */
