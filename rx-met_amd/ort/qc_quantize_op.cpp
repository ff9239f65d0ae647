// qc_quantize_op.cpp — ONNX Runtime plugin of QcQuantizeOp for MI355X: the op library a
// session loads with RegisterCustomOpsLibrary / register_custom_ops_library, as the reference's
// libaimet_onnxrt_ops.so (native/onnx/src/RegisterCustomOps.cpp:27-60, QcQuantizeOp.cpp).
//
// The reference registers CPU kernels and, with ONNX_CUDA, CUDA kernels.  This library
// registers kernels for ONNX Runtime's ROCm execution provider, which run on the provider's
// compute stream (KernelContext_GetGPUComputeStream) with device tensors; the computation is
// rxmet_qc_quantize_compute of librxmet.so.  Both domain names of the reference are
// registered so graphs exported for it load unchanged.  Built only against ONNX Runtime's own
// headers (the ORT C++ API is header-only over the OrtApi table the runtime passes in).
#define ORT_API_MANUAL_INIT
#include "onnxruntime_cxx_api.h"
#undef ORT_API_MANUAL_INIT
#include "onnxruntime_lite_custom_op.h"

#include <memory>
#include <mutex>
#include <type_traits>
#include <vector>

#include "rxmet_qc.h"

namespace {

const char *kDomain = "aimet.customop.cpu";
const char *kDomainGpu = "aimet.customop.cuda";
const char *kProvider = "ROCMExecutionProvider";

template <typename T>
struct QcQuantizeOpRocm {
  // the node's "quant_info" attribute holds the address of its rxmet_qc_quantize_info
  QcQuantizeOpRocm(const OrtApi *api, const OrtKernelInfo *info) {
    int64_t p = 0;
    Ort::ThrowOnError(api->KernelInfoGetAttribute_int64(info, "quant_info", &p));
    info_ = reinterpret_cast<rxmet_qc_quantize_info *>(p);
  }

  void Compute(OrtKernelContext *context, const Ort::Custom::Tensor<T> &input,
               Ort::Custom::Tensor<T> &output) {
    Ort::KernelContext ctx(context);
    void *stream = ctx.GetGPUComputeStream();
    const std::vector<int64_t> shape = input.Shape();
    T *out = output.Allocate(shape);
    const int32_t io = std::is_same<T, Ort::Float16_t>::value ? RXMET_QDQ_F16 : RXMET_QDQ_F32;
    if (rxmet_qc_quantize_compute(info_, input.DataRaw(), out, io, shape.data(),
                                  static_cast<int32_t>(shape.size()), nullptr, stream) != 0)
      ORT_CXX_API_THROW(rxmet_last_error(), ORT_RUNTIME_EXCEPTION);
  }

  rxmet_qc_quantize_info *info_ = nullptr;
};

void add_ops(Ort::CustomOpDomain &domain) {
  static const std::unique_ptr<Ort::Custom::OrtLiteCustomOp> f32{
      Ort::Custom::CreateLiteCustomOp<QcQuantizeOpRocm<float>>("QcQuantizeOp", kProvider)};
  static const std::unique_ptr<Ort::Custom::OrtLiteCustomOp> f16{
      Ort::Custom::CreateLiteCustomOp<QcQuantizeOpRocm<Ort::Float16_t>>("QcQuantizeOp",
                                                                         kProvider)};
  domain.Add(f32.get());
  domain.Add(f16.get());
}

// the domains must outlive every session that uses them
std::mutex g_mu;
std::vector<Ort::CustomOpDomain> g_domains;

}  // namespace

extern "C" OrtStatus *ORT_API_CALL RegisterCustomOps(OrtSessionOptions *options,
                                                     const OrtApiBase *api) {
  Ort::InitApi(api->GetApi(ORT_API_VERSION));
  try {
    Ort::UnownedSessionOptions session_options(options);
    std::lock_guard<std::mutex> lock(g_mu);
    for (const char *name : {kDomain, kDomainGpu}) {
      Ort::CustomOpDomain domain{name};
      add_ops(domain);
      session_options.Add(domain);
      g_domains.push_back(std::move(domain));
    }
  } catch (const std::exception &e) {
    Ort::Status status{e};
    return status.release();
  }
  return nullptr;
}
