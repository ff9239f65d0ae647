/*
 * rxmet_selftest.h — self-tests of hardware assumptions the kernels rely on.
 *
 * No counterpart in the reference: these entry points exist so that tests can check,
 * on the GPU, the MFMA operand/result lane layouts the GRU kernels are written against.
 */
#ifndef RXMET_SELFTEST_H_
#define RXMET_SELFTEST_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * One wavefront computes D[16x16] = A[16xK] * B[Kx16] with the fragment layouts the GRU
 * kernels use.  which = 0: int8 inputs (K = 64, v_mfma_i32_16x16x64_i8), A/B given as
 * int8, D int32.  which = 1: bf16 inputs (K = 32, v_mfma_f32_16x16x32_bf16), A/B given as
 * fp32 values exactly representable in bf16, D fp32.  which = 2: fp32 inputs (K = 4,
 * v_mfma_f32_16x16x4_f32), D fp32.  All pointers are device memory:
 * A row-major [16][K], B row-major [K][16], D row-major [16][16].
 */
int rxmet_selftest_mfma(int which, const void *A, const void *B, void *D, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_SELFTEST_H_ */
