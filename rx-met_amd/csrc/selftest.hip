// selftest.hip — device check of the MFMA fragment layouts declared in mfma_frag.h.
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_selftest.h"

namespace rxmet {
namespace {

__global__ __launch_bounds__(64) void mfma_i8_probe(const int8_t *A, const int8_t *B, int *D) {
  const int l = threadIdx.x;
  int a[4], b[4];
  for (int q = 0; q < 4; ++q) {
    const int k0 = 16 * (l / 16) + 4 * q;
    a[q] = pack4_i8(A[(l % 16) * 64 + k0], A[(l % 16) * 64 + k0 + 1], A[(l % 16) * 64 + k0 + 2],
                    A[(l % 16) * 64 + k0 + 3]);
    b[q] = pack4_i8(B[k0 * 16 + l % 16], B[(k0 + 1) * 16 + l % 16], B[(k0 + 2) * 16 + l % 16],
                    B[(k0 + 3) * 16 + l % 16]);
  }
  v4i av = {a[0], a[1], a[2], a[3]}, bv = {b[0], b[1], b[2], b[3]}, acc = {0, 0, 0, 0};
  acc = mfma_i8(av, bv, acc);
  for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + l % 16] = acc[r];
}

__global__ __launch_bounds__(64) void mfma_bf16_probe(const float *A, const float *B, float *D) {
  const int l = threadIdx.x;
  v8bf av, bv;
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * (l / 16) + j;
    av[j] = static_cast<__bf16>(A[(l % 16) * 32 + k]);
    bv[j] = static_cast<__bf16>(B[k * 16 + l % 16]);
  }
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma_bf16(av, bv, acc);
  for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + l % 16] = acc[r];
}

__global__ __launch_bounds__(64) void mfma_f32_probe(const float *A, const float *B, float *D) {
  const int l = threadIdx.x;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma_f32(A[(l % 16) * 4 + l / 16], B[(l / 16) * 16 + l % 16], acc);
  for (int r = 0; r < 4; ++r) D[(4 * (l / 16) + r) * 16 + l % 16] = acc[r];
}

}  // namespace
}  // namespace rxmet

extern "C" int rxmet_selftest_mfma(int which, const void *A, const void *B, void *D, void *stream) {
  rxmet::clear_error();
  RXMET_CHECK_ARG(A && B && D, "null argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (which == 0) {
    hipLaunchKernelGGL(rxmet::mfma_i8_probe, dim3(1), dim3(64), 0, s,
                       static_cast<const int8_t *>(A), static_cast<const int8_t *>(B),
                       static_cast<int *>(D));
  } else if (which == 1) {
    hipLaunchKernelGGL(rxmet::mfma_bf16_probe, dim3(1), dim3(64), 0, s,
                       static_cast<const float *>(A), static_cast<const float *>(B),
                       static_cast<float *>(D));
  } else if (which == 2) {
    hipLaunchKernelGGL(rxmet::mfma_f32_probe, dim3(1), dim3(64), 0, s,
                       static_cast<const float *>(A), static_cast<const float *>(B),
                       static_cast<float *>(D));
  } else {
    rxmet::set_error("which must be 0 (int8), 1 (bf16) or 2 (fp32)");
    return -22;
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}
