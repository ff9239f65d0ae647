// blas_util.h — rocBLAS plumbing shared by the recurrent backward passes: one handle per
// device, row-major SGEMM wrappers and a split-K product for long-K weight gradients.
#pragma once

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cstdint>

namespace rxmet {
namespace blas {

// rocBLAS handle of `device`, created on first use (rocBLAS sizes its own workspace then).
rocblas_handle handle(int device);

// Row-major C[M][N] = op(A) op(B).
rocblas_status gemm_rm(rocblas_handle h, bool ta, bool tb, int M, int N, int K, const float *A,
                       int lda, const float *Bm, int ldb, float *Cm, int ldc);

// Number of K chunks used by gemm_tn_splitk for a reduction of length K.
int splitk_chunks(int64_t K);

// Row-major out[Mo][N] = A[K][Mo]^T B[K][N]: K split into S chunks (one strided-batched
// SGEMM into `part`, S x Mo x N floats, the K remainder added to chunk 0) and summed in a
// fixed order.  Returns 0 or a negative status with the error message set.
int gemm_tn_splitk(rocblas_handle h, int Mo, int N, int64_t K, const float *A, int lda,
                   const float *Bm, int ldb, float *out, float *part, int S, hipStream_t stream);

}  // namespace blas
}  // namespace rxmet
