// qc_ref_shim.cpp — TEST INFRASTRUCTURE: a C surface over the reference's own native CPU code
// for the ONNX Runtime op's quantizer (getComputedEncodings, MinMaxEncodingAnalyzer<float>,
// quantizeDequantize / quantizeDequantizeBroadcast), compiled with those sources where they
// lie under the reference checkout into oracle/_ref/libqc_ref.so.  It drives them the way
// BlockTensorQuantizer does (native/common/src/TensorQuantizer.cpp:362-397, 451-469); tests
// use it only to check oracle/qc_quantize_oracle.py.
#include <cstdint>
#include <stdexcept>
#include <vector>

#include "DlQuantization/Quantization.hpp"
#include "MinMaxEncodingAnalyzer.h"
#include "quantization_utils.hpp"
#include "trim_functions.hpp"

using namespace DlQuantization;

extern "C" {

void qcref_computed_encodings(int bw, double mn, double mx, int sym, int strict, int uns,
                              double *out) {
  const TfEncoding e = getComputedEncodings(static_cast<uint8_t>(bw), mn, mx, sym != 0,
                                            strict != 0, uns != 0);
  out[0] = e.min;
  out[1] = e.max;
  out[2] = e.delta;
  out[3] = e.offset;
}

// ncalls updateStats calls over the tensors at x (each of the shape), then computeEncoding;
// enc: 4 doubles (min, max, delta, offset) per encoding; stats: 2 floats per encoding
int qcref_analyzer(const float *x, const int64_t *shape, int ndim, const int64_t *eshape,
                   int endim, int ncalls, int bw, int sym, int strict, int uns, double *enc) {
  try {
    TensorDims ts(shape, shape + ndim), es(eshape, eshape + endim);
    MinMaxEncodingAnalyzer<float> a(es);
    size_t numel = 1;
    for (int i = 0; i < ndim; ++i) numel *= static_cast<size_t>(shape[i]);
    for (int k = 0; k < ncalls; ++k)
      a.updateStats(x + k * numel, ts, COMP_MODE_CPU, nullptr, nullptr);
    const Encodings e = a.computeEncoding(static_cast<uint8_t>(bw), sym != 0, strict != 0,
                                          uns != 0);
    for (size_t i = 0; i < e.size(); ++i) {
      enc[4 * i] = e[i].min;
      enc[4 * i + 1] = e[i].max;
      enc[4 * i + 2] = e[i].delta;
      enc[4 * i + 3] = e[i].offset;
    }
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

int qcref_qdq(const float *x, float *y, const int64_t *shape, int ndim, const int64_t *eshape,
              int endim, const double *enc, int bw) {
  try {
    TensorDims ts(shape, shape + ndim), es(eshape, eshape + endim);
    size_t n = 1, numel = 1;
    for (int i = 0; i < endim; ++i) n *= static_cast<size_t>(eshape[i]);
    for (int i = 0; i < ndim; ++i) numel *= static_cast<size_t>(shape[i]);
    Encodings e(n);
    for (size_t i = 0; i < n; ++i)
      e[i] = TfEncoding{enc[4 * i], enc[4 * i + 1], enc[4 * i + 2], enc[4 * i + 3], bw};
    if (n == 1)
      quantizeDequantize(x, numel, e[0], y, COMP_MODE_CPU, ROUND_NEAREST, nullptr);
    else
      quantizeDequantizeBroadcast(x, y, e, ts, es, COMP_MODE_CPU, nullptr);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

}  // extern "C"
