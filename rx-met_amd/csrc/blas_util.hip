// blas_util.hip — see blas_util.h.
#include "blas_util.h"

#include <mutex>
#include <vector>

#include "rxmet_common.h"

namespace rxmet {
namespace blas {

rocblas_handle handle(int device) {
  static std::mutex mu;
  static std::vector<rocblas_handle> handles;
  std::lock_guard<std::mutex> g(mu);
  if (static_cast<int>(handles.size()) <= device) handles.resize(device + 1, nullptr);
  if (!handles[device]) rocblas_create_handle(&handles[device]);
  return handles[device];
}

rocblas_status gemm_rm(rocblas_handle h, bool ta, bool tb, int M, int N, int K, const float *A,
                       int lda, const float *Bm, int ldb, float *Cm, int ldc) {
  const float one = 1.0f, zero = 0.0f;
  return rocblas_sgemm(h, tb ? rocblas_operation_transpose : rocblas_operation_none,
                       ta ? rocblas_operation_transpose : rocblas_operation_none, N, M, K, &one, Bm,
                       ldb, A, lda, &zero, Cm, ldc);
}

int splitk_chunks(int64_t K) {
  int64_t s = K / 1024;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return static_cast<int>(s);
}

__global__ __launch_bounds__(256) void sum_partials(int64_t n, int S, const float *__restrict__ part,
                                                    float *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float acc = part[i];
  for (int s = 1; s < S; ++s) acc += part[static_cast<size_t>(s) * n + i];
  out[i] = acc;
}

int gemm_tn_splitk(rocblas_handle h, int Mo, int N, int64_t K, const float *A, int lda,
                   const float *Bm, int ldb, float *out, float *part, int S, hipStream_t stream) {
  const int Kc = static_cast<int>(K / S);
  const float one = 1.0f, zero = 0.0f;
  rocblas_status st = rocblas_sgemm_strided_batched(
      h, rocblas_operation_none, rocblas_operation_transpose, N, Mo, Kc, &one, Bm, ldb,
      static_cast<rocblas_stride>(Kc) * ldb, A, lda, static_cast<rocblas_stride>(Kc) * lda, &zero,
      part, N, static_cast<rocblas_stride>(Mo) * N, S);
  RXMET_CHECK_ARG(st == rocblas_status_success, "rocBLAS strided-batched sgemm failed");
  const int64_t rem = K - static_cast<int64_t>(Kc) * S;
  if (rem > 0) {
    const size_t off = static_cast<size_t>(Kc) * S;
    st = rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_transpose, N, Mo,
                       static_cast<int>(rem), &one, Bm + off * ldb, ldb, A + off * lda, lda, &one,
                       part, N);
    RXMET_CHECK_ARG(st == rocblas_status_success, "rocBLAS sgemm (split-K tail) failed");
  }
  const int64_t n = static_cast<int64_t>(Mo) * N;
  hipLaunchKernelGGL(sum_partials, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, n, S, part, out);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // namespace blas
}  // namespace rxmet
