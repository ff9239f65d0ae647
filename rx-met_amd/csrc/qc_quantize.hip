// qc_quantize.hip — the ONNX Runtime custom op QcQuantizeOp and its TF-scheme
// BlockTensorQuantizer on MI355X (C ABI in rxmet_qc.h).
//
// Reference: native/onnx/src/QcQuantizeOp.cpp:101-170 (computeImpl), AimetOpUtils.h:58-128
// (op modes), native/common/src/TensorQuantizer.cpp:348-469 (BlockTensorQuantizer),
// MinMaxEncodingAnalyzer.cpp:57-96 and ContiguousEncodingAnalyzer.cpp:46-97 (statistics),
// quantization_utils.cpp:59-119 (getComputedEncodings), trim_functions.cpp:646-713
// (broadcast quantize-dequantize).
//
// The reference keeps statistics and encodings on the host and, on the GPU, synchronizes for
// every statistics update (GetMinMax_gpu copies each reduction back).  Here they stay in HBM
// next to the op: a oneShot call runs on the caller's stream with no host round
// trip — the streaming min / max of the QDQ kernels (NaN skipped), their per-encoding fold,
// which also replaces the running statistics and derives the TfEncodings in double arithmetic,
// and the stableQuantizeDequantize streaming pass: three launches.
#include <algorithm>
#include <cfloat>
#include <climits>
#include <vector>

#include "qdq_kernels.h"
#include "rxmet_qc.h"

using rxmet::qdq::TfEnc32;

struct rxmet_block_tensor_quantizer {
  std::vector<int64_t> shape;  // encoding shape
  int64_t n = 1;               // encodings
  int32_t bitwidth = 8;
  bool strict = false, unsigned_sym = false;
  bool valid_stats = false, encoding_valid = false;
  int device = 0;
  // device memory, one allocation: running min / max (fp32), the encodings as TfEncoding
  // (double) and as the fp32 form the QDQ pass reads
  void *mem = nullptr;
  float *st_min = nullptr, *st_max = nullptr;
  rxmet_tf_encoding *enc = nullptr;
  TfEnc32 *enc32 = nullptr;
  void *ws = nullptr;  // the quantizer's own workspace (update_stats with none given)
  size_t ws_bytes = 0;
};

namespace rxmet {
namespace qc {

constexpr int kThreads = 256;

// running statistics reset: (numeric_limits<float>::max(), lowest()) as resetStats
__global__ __launch_bounds__(kThreads) void stats_reset(int64_t n, float *mn, float *mx) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  mn[c] = FLT_MAX;
  mx[c] = -FLT_MAX;
}

// MinMaxEncodingAnalyzer::computeEncoding from the running statistics, one thread per encoding.
__global__ __launch_bounds__(kThreads) void compute_encodings(
    int64_t n, const float *st_min, const float *st_max, int bw, int sym, int strict,
    int unsigned_sym, rxmet_tf_encoding *enc, TfEnc32 *enc32) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  rxmet::qdq::tf_encoding(st_min[c], st_max[c], bw, sym, strict, unsigned_sym, enc, enc32, c);
}

// fp32 forms of host-set encodings
__global__ __launch_bounds__(kThreads) void pack_encodings(int64_t n, const rxmet_tf_encoding *enc,
                                                           TfEnc32 *enc32) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= n) return;
  const rxmet_tf_encoding e = enc[c];
  TfEnc32 t;
  t.mn = static_cast<float>(e.min);
  t.mx = static_cast<float>(e.max);
  t.delta = static_cast<float>(e.delta);
  t.inv_delta = 1.0f / t.delta;
  enc32[c] = t;
}

static int64_t numel(const int64_t *shape, int32_t ndim) {
  int64_t n = 1;
  for (int i = 0; i < ndim; ++i) n *= shape[i];
  return n;
}

static unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

// getBroadcastableShapes (tensor_utils.cpp:62-88) and the grouping of the encoding dimensions
// into [outer, C0, mid, C1, inner].
static int broadcast_layout(const int64_t *shape, int32_t ndim, const int64_t *enc_shape,
                            int32_t enc_ndim, rxmet_qdq_layout &out) {
  RXMET_CHECK_ARG(ndim >= 0 && enc_ndim >= 0 && ndim <= 64 && enc_ndim <= 64,
                  "tensor / encoding rank out of range");
  RXMET_CHECK_ARG(ndim == 0 || shape != nullptr, "shape must be non-null");
  RXMET_CHECK_ARG(enc_ndim == 0 || enc_shape != nullptr, "encoding shape must be non-null");
  RXMET_CHECK_ARG(enc_ndim <= ndim, "encoding shape has more dimensions than the tensor");
  std::vector<int64_t> tdims, edims;  // broadcast tensor / encoding shapes
  const int pad = ndim - enc_ndim;
  for (int i = 0; i < ndim; ++i) {
    const int64_t d1 = shape[i];
    const int64_t d2 = i < pad ? 1 : enc_shape[i - pad];
    RXMET_CHECK_ARG(d1 >= 0 && d2 >= 1, "invalid tensor or encoding dimension");
    if (d1 == d2) {
      tdims.push_back(d1);
      edims.push_back(d2);
    } else {
      RXMET_CHECK_ARG(d1 >= d2 && d1 % d2 == 0,
                      "Cannot interpret tensor and encoding dimensions as broadcastable");
      tdims.push_back(d2);
      tdims.push_back(d1 / d2);
      edims.push_back(d2);
      edims.push_back(1);
    }
  }
  // dimensions: encoding (e == t > 1), broadcast (e == 1 < t) or neutral (t == e == 1); the
  // broadcast dimensions before, between and after the encoding groups multiply into
  // outer / mid / inner
  int groups = 0;
  bool in_group = false;
  int64_t g[2] = {1, 1}, bc[3] = {1, 1, 1};
  for (size_t i = 0; i < tdims.size(); ++i) {
    const int64_t t = tdims[i], e = edims[i];
    if (t == 1 && e == 1) continue;
    if (e > 1) {
      if (!in_group) {
        RXMET_CHECK_ARG(groups < 2, "the encodings form more than two groups of dimensions");
        ++groups;
        in_group = true;
      }
      g[groups - 1] *= e;
    } else {
      in_group = false;
      bc[groups] *= t;
    }
  }
  if (groups == 0)
    out = rxmet_qdq_layout{1, 1, 1, 1, bc[0]};
  else if (groups == 1)
    out = rxmet_qdq_layout{1, 1, bc[0], g[0], bc[1]};
  else
    out = rxmet_qdq_layout{bc[0], g[0], bc[1], g[1], bc[2]};
  return 0;
}

static int check_q(const rxmet_block_tensor_quantizer *q) {
  RXMET_CHECK_ARG(q != nullptr, "tensor quantizer must be non-null");
  int dev = -1;
  RXMET_CHECK_HIP(hipGetDevice(&dev));
  RXMET_CHECK_ARG(dev == q->device, "the tensor quantizer belongs to another device");
  return 0;
}

static int check_io(int32_t io) {
  RXMET_CHECK_ARG(io == RXMET_QDQ_F32 || io == RXMET_QDQ_F16,
                  "io_dtype must be RXMET_QDQ_F32 or RXMET_QDQ_F16");
  return 0;
}

// A single encoding covers any tensor (the per-tensor paths of TensorQuantizer.cpp:388-392
// and ContiguousEncodingAnalyzer.cpp:53-56 do not broadcast).
static int layout_of(const rxmet_block_tensor_quantizer *q, const int64_t *shape, int32_t ndim,
                     rxmet_qdq_layout &l) {
  if (q->n == 1) {
    l = rxmet_qdq_layout{1, 1, 1, 1, numel(shape, ndim)};
    return 0;
  }
  return broadcast_layout(shape, ndim, q->shape.empty() ? nullptr : q->shape.data(),
                          static_cast<int32_t>(q->shape.size()), l);
}

static int64_t ws_bytes(const rxmet_qdq_layout &l, int32_t io) {
  return rxmet_qdq_workspace_bytes_ex(&l, io);
}

static int reset_stats(rxmet_block_tensor_quantizer *q, hipStream_t s) {
  hipLaunchKernelGGL(stats_reset, dim3(blocks_for(q->n)), dim3(kThreads), 0, s, q->n, q->st_min,
                     q->st_max);
  RXMET_CHECK_LAUNCH();
  q->valid_stats = false;
  q->encoding_valid = false;
  return 0;
}

// One statistics update folded into the running statistics (reset: in their place), and with
// enc_sym >= 0 the encodings computed from them and set (symmetric = enc_sym) in the same fold.
static int update_stats(rxmet_block_tensor_quantizer *q, const void *x, int32_t io,
                        const int64_t *shape, int32_t ndim, void *workspace, hipStream_t s,
                        bool reset = false, int enc_sym = -1) {
  if (int rc = check_io(io)) return rc;
  rxmet_qdq_layout l;
  if (int rc = layout_of(q, shape, ndim, l)) return rc;
  RXMET_CHECK_ARG(numel(shape, ndim) > 0, "statistics of an empty tensor");
  const int64_t need = ws_bytes(l, io);
  if (workspace == nullptr && need > 0) {
    if (static_cast<size_t>(need) > q->ws_bytes) {
      if (q->ws) RXMET_CHECK_HIP(hipFree(q->ws));
      q->ws = nullptr;
      q->ws_bytes = 0;
      RXMET_CHECK_HIP(hipMalloc(&q->ws, static_cast<size_t>(need)));
      q->ws_bytes = static_cast<size_t>(need);
    }
    workspace = q->ws;
  }
  rxmet::prof::Scope ps__("qc_update_stats", s);
  const rxmet::qdq::StatsSink sink{q->st_min,   q->st_max,         reset ? 1 : 0,
                                   enc_sym >= 0, q->bitwidth,       enc_sym > 0 ? 1 : 0,
                                   q->strict,   q->unsigned_sym,    q->enc,
                                   q->enc32};
  if (int rc = rxmet::qdq::minmax_stats(x, io, l, sink, workspace, s)) return rc;
  q->valid_stats = true;
  if (reset) q->encoding_valid = false;
  if (enc_sym >= 0) q->encoding_valid = true;
  return 0;
}

static int compute_and_set(rxmet_block_tensor_quantizer *q, bool sym, hipStream_t s) {
  RXMET_CHECK_ARG(q->valid_stats, "Cannot compute encodings before updating stats");
  hipLaunchKernelGGL(compute_encodings, dim3(blocks_for(q->n)), dim3(kThreads), 0, s, q->n,
                     q->st_min, q->st_max, q->bitwidth, sym ? 1 : 0, q->strict ? 1 : 0,
                     q->unsigned_sym ? 1 : 0, q->enc, q->enc32);
  RXMET_CHECK_LAUNCH();
  q->encoding_valid = true;
  return 0;
}

static int qdq(const rxmet_block_tensor_quantizer *q, const void *x, void *y, int32_t io,
               const int64_t *shape, int32_t ndim, hipStream_t s) {
  if (int rc = check_io(io)) return rc;
  RXMET_CHECK_ARG(q->encoding_valid, "Cannot perform quantization before computing encodings");
  rxmet_qdq_layout l;
  if (int rc = layout_of(q, shape, ndim, l)) return rc;
  return rxmet::qdq::forward_tf(rxmet::qdq::OP_NATIVE, x, y, io, l, q->enc32, s);
}

static int copy(const void *x, void *y, int32_t io, const int64_t *shape, int32_t ndim,
                hipStream_t s) {
  const int64_t n = numel(shape, ndim);
  if (n == 0 || x == y) return 0;
  RXMET_CHECK_ARG(x != nullptr && y != nullptr, "input/output must be non-null");
  RXMET_CHECK_HIP(hipMemcpyAsync(y, x, static_cast<size_t>(n) * (io == RXMET_QDQ_F32 ? 4 : 2),
                                 hipMemcpyDeviceToDevice, s));
  return 0;
}

}  // namespace qc
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::qc;

extern "C" {

rxmet_block_tensor_quantizer *rxmet_block_tensor_quantizer_create(const int64_t *shape,
                                                                  int32_t ndim,
                                                                  int32_t bitwidth) {
  clear_error();
  if (ndim < 0 || ndim > 64 || (ndim > 0 && shape == nullptr)) {
    set_error("invalid encoding shape");
    return nullptr;
  }
  if (bitwidth < 1 || bitwidth > 32) {
    set_error("bitwidth must be in [1, 32]");
    return nullptr;
  }
  int64_t n = 1;
  for (int i = 0; i < ndim; ++i) {
    if (shape[i] < 1 || n > (INT64_C(1) << 40) / shape[i]) {
      set_error("invalid encoding shape");
      return nullptr;
    }
    n *= shape[i];
  }
  auto *q = new rxmet_block_tensor_quantizer;
  q->shape.assign(shape, shape + ndim);
  q->n = n;
  q->bitwidth = bitwidth;
  if (hipGetDevice(&q->device) != hipSuccess) {
    set_error("hipGetDevice failed");
    delete q;
    return nullptr;
  }
  // 2 fp32 arrays, the TfEncodings, the fp32 encodings (each region 256-byte aligned)
  auto up = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t f = up(sizeof(float) * n), e = up(sizeof(rxmet_tf_encoding) * n),
               e32 = up(sizeof(TfEnc32) * n);
  if (hipMalloc(&q->mem, 2 * f + e + e32) != hipSuccess) {
    set_error("hipMalloc of the quantizer state failed");
    delete q;
    return nullptr;
  }
  char *p = static_cast<char *>(q->mem);
  q->st_min = reinterpret_cast<float *>(p);
  q->st_max = reinterpret_cast<float *>(p + f);
  q->enc = reinterpret_cast<rxmet_tf_encoding *>(p + 2 * f);
  q->enc32 = reinterpret_cast<TfEnc32 *>(p + 2 * f + e);
  // statistics start reset, as the analyzer's constructor leaves them
  if (reset_stats(q, nullptr) != 0 || hipStreamSynchronize(nullptr) != hipSuccess) {
    (void)hipFree(q->mem);
    delete q;
    return nullptr;
  }
  return q;
}

void rxmet_block_tensor_quantizer_destroy(rxmet_block_tensor_quantizer *q) {
  if (q == nullptr) return;
  (void)hipDeviceSynchronize();
  if (q->ws) (void)hipFree(q->ws);
  if (q->mem) (void)hipFree(q->mem);
  delete q;
}

int rxmet_block_tensor_quantizer_get_state(const rxmet_block_tensor_quantizer *q,
                                           rxmet_block_tensor_quantizer_state *out) {
  clear_error();
  RXMET_CHECK_ARG(q != nullptr && out != nullptr, "quantizer and out must be non-null");
  out->num_encodings = q->n;
  out->bitwidth = q->bitwidth;
  out->use_strict_symmetric = q->strict;
  out->use_unsigned_symmetric = q->unsigned_sym;
  out->valid_stats = q->valid_stats;
  out->is_encoding_valid = q->encoding_valid;
  out->reserved = 0;
  return 0;
}

int rxmet_block_tensor_quantizer_set_strict_symmetric(rxmet_block_tensor_quantizer *q,
                                                      int32_t on) {
  clear_error();
  RXMET_CHECK_ARG(q != nullptr, "tensor quantizer must be non-null");
  q->encoding_valid = false;
  q->strict = on != 0;
  return 0;
}

int rxmet_block_tensor_quantizer_set_unsigned_symmetric(rxmet_block_tensor_quantizer *q,
                                                        int32_t on) {
  clear_error();
  RXMET_CHECK_ARG(q != nullptr, "tensor quantizer must be non-null");
  q->encoding_valid = false;
  q->unsigned_sym = on != 0;
  return 0;
}

int rxmet_block_tensor_quantizer_set_bitwidth(rxmet_block_tensor_quantizer *q, int32_t bw) {
  clear_error();
  RXMET_CHECK_ARG(q != nullptr, "tensor quantizer must be non-null");
  RXMET_CHECK_ARG(bw >= 1 && bw <= 32, "bitwidth must be in [1, 32]");
  q->bitwidth = bw;
  return 0;
}

int64_t rxmet_block_tensor_quantizer_workspace_bytes(const rxmet_block_tensor_quantizer *q,
                                                     const int64_t *shape, int32_t ndim,
                                                     int32_t io_dtype) {
  clear_error();
  if (q == nullptr || check_io(io_dtype) != 0) return 0;
  rxmet_qdq_layout l;
  if (layout_of(q, shape, ndim, l) != 0) return 0;
  return ws_bytes(l, io_dtype);
}

int rxmet_block_tensor_quantizer_reset_encoding_stats(rxmet_block_tensor_quantizer *q,
                                                      void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  return reset_stats(q, static_cast<hipStream_t>(stream));
}

int rxmet_block_tensor_quantizer_update_stats(rxmet_block_tensor_quantizer *q, const void *x,
                                              int32_t io_dtype, const int64_t *shape,
                                              int32_t ndim, void *workspace, void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  return update_stats(q, x, io_dtype, shape, ndim, workspace, static_cast<hipStream_t>(stream));
}

int rxmet_block_tensor_quantizer_compute_encodings(rxmet_block_tensor_quantizer *q,
                                                   int32_t use_symmetric, void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  return compute_and_set(q, use_symmetric != 0, static_cast<hipStream_t>(stream));
}

int rxmet_block_tensor_quantizer_set_encodings(rxmet_block_tensor_quantizer *q,
                                               const rxmet_tf_encoding *enc, int64_t n,
                                               void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  RXMET_CHECK_ARG(n == q->n, "Length of encoding vector did not match BlockTensorQuantizer shape");
  RXMET_CHECK_ARG(enc != nullptr, "encodings must be non-null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = upload(q->enc, enc, sizeof(rxmet_tf_encoding) * static_cast<size_t>(n), s))
    return rc;
  hipLaunchKernelGGL(pack_encodings, dim3(blocks_for(n)), dim3(kThreads), 0, s, n, q->enc,
                     q->enc32);
  RXMET_CHECK_LAUNCH();
  q->encoding_valid = true;
  q->bitwidth = enc[0].bw;
  return 0;
}

int rxmet_block_tensor_quantizer_get_encodings(const rxmet_block_tensor_quantizer *q,
                                               rxmet_tf_encoding *enc, int64_t n, void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  RXMET_CHECK_ARG(n == q->n && enc != nullptr, "need num_encodings host encodings");
  hipStream_t s = static_cast<hipStream_t>(stream);
  RXMET_CHECK_HIP(hipMemcpyAsync(enc, q->enc, sizeof(rxmet_tf_encoding) * static_cast<size_t>(n),
                                 hipMemcpyDeviceToHost, s));
  RXMET_CHECK_HIP(hipStreamSynchronize(s));
  return 0;
}

int rxmet_block_tensor_quantizer_get_stats(const rxmet_block_tensor_quantizer *q, float *min,
                                           float *max, int64_t n, void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  RXMET_CHECK_ARG(n == q->n && min != nullptr && max != nullptr,
                  "need num_encodings host floats for min and max");
  hipStream_t s = static_cast<hipStream_t>(stream);
  RXMET_CHECK_HIP(hipMemcpyAsync(min, q->st_min, sizeof(float) * static_cast<size_t>(n),
                                 hipMemcpyDeviceToHost, s));
  RXMET_CHECK_HIP(hipMemcpyAsync(max, q->st_max, sizeof(float) * static_cast<size_t>(n),
                                 hipMemcpyDeviceToHost, s));
  RXMET_CHECK_HIP(hipStreamSynchronize(s));
  return 0;
}

int rxmet_block_tensor_quantizer_quantize_dequantize(const rxmet_block_tensor_quantizer *q,
                                                     const void *x, void *y, int32_t io_dtype,
                                                     const int64_t *shape, int32_t ndim,
                                                     void *stream) {
  clear_error();
  if (int rc = check_q(q)) return rc;
  return qc::qdq(q, x, y, io_dtype, shape, ndim, static_cast<hipStream_t>(stream));
}

int64_t rxmet_qc_quantize_workspace_bytes(const rxmet_qc_quantize_info *info,
                                          const int64_t *shape, int32_t ndim, int32_t io_dtype) {
  if (info == nullptr || info->tensor_quantizer == nullptr || !info->is_int_data_type) return 0;
  return rxmet_block_tensor_quantizer_workspace_bytes(info->tensor_quantizer, shape, ndim,
                                                      io_dtype);
}

int rxmet_qc_quantize_compute(rxmet_qc_quantize_info *info, const void *x, void *y,
                              int32_t io_dtype, const int64_t *shape, int32_t ndim,
                              void *workspace, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(info != nullptr, "quant_info must be non-null");
  if (int rc = check_io(io_dtype)) return rc;
  RXMET_CHECK_ARG(ndim >= 0 && ndim <= 64 && (ndim == 0 || shape != nullptr), "invalid shape");
  for (int i = 0; i < ndim; ++i) RXMET_CHECK_ARG(shape[i] >= 0, "invalid shape");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int mode = info->op_mode;
  RXMET_CHECK_ARG(mode >= RXMET_QC_UPDATE_STATS && mode <= RXMET_QC_PASS_THROUGH,
                  "unknown op mode");
  if (!info->enabled) mode = RXMET_QC_PASS_THROUGH;
  int rc = 0;
  if (info->is_int_data_type) {
    rxmet_block_tensor_quantizer *q = info->tensor_quantizer;
    if (mode != RXMET_QC_PASS_THROUGH)
      if ((rc = check_q(q))) return rc;
    switch (mode) {
      case RXMET_QC_ONE_SHOT_QUANTIZE_DEQUANTIZE:
        // resetEncodingStats, updateStats, computeEncodings + setEncodings: one statistics
        // pass whose fold replaces the statistics and derives the encodings
        if ((rc = update_stats(q, x, io_dtype, shape, ndim, workspace, s, true,
                               info->use_symmetric_encoding ? 1 : 0)))
          return rc;
        [[fallthrough]];
      case RXMET_QC_QUANTIZE_DEQUANTIZE:
        rc = qc::qdq(q, x, y, io_dtype, shape, ndim, s);
        break;
      case RXMET_QC_UPDATE_STATS:
        if ((rc = update_stats(q, x, io_dtype, shape, ndim, workspace, s))) return rc;
        [[fallthrough]];
      default:
        rc = copy(x, y, io_dtype, shape, ndim, s);
    }
  } else if (mode == RXMET_QC_ONE_SHOT_QUANTIZE_DEQUANTIZE ||
             mode == RXMET_QC_QUANTIZE_DEQUANTIZE) {
    const rxmet_qdq_layout l{1, 1, 1, 1, numel(shape, ndim)};
    rc = rxmet::qdq::forward_tf(rxmet::qdq::OP_FP16, x, y, io_dtype, l, nullptr, s);
  } else {
    rc = copy(x, y, io_dtype, shape, ndim, s);
  }
  if (rc) return rc;
  // one-shot runs once; afterwards the node quantizes with the encodings it computed
  if (mode == RXMET_QC_ONE_SHOT_QUANTIZE_DEQUANTIZE) info->op_mode = RXMET_QC_QUANTIZE_DEQUANTIZE;
  return 0;
}

int rxmet_qc_broadcast_layout(const int64_t *shape, int32_t ndim, const int64_t *enc_shape,
                              int32_t enc_ndim, rxmet_qdq_layout *out) {
  clear_error();
  RXMET_CHECK_ARG(out != nullptr, "out must be non-null");
  return broadcast_layout(shape, ndim, enc_shape, enc_ndim, *out);
}

}  // extern "C"
