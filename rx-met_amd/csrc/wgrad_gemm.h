// wgrad_gemm.h — weight-gradient GEMMs of the QAT backward on bf16 MFMA.
//
// Every product here pairs a float gradient with integer quantisation codes.  The codes are
// exact in bf16 (one plane for |code| <= 256; two planes 256 hi + lo for 16-bit codes), and the
// gradient is split exactly into three bf16 terms g = g_hi + g_mid + g_lo (each the RNE bf16 of
// what the previous terms leave).  Every bf16 x bf16 product is exact in fp32 and the MFMA
// accumulates in fp32, so the result has the accuracy of an fp32 GEMM (a different summation
// order), at 3 (or 6) v_mfma_f32_16x16x32_bf16 per 32 K instead of 8 v_mfma_f32_16x16x4_f32.
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace rxmet {
namespace wgrad {

// part[s][p][q] = sum over k in split s of A[k * lda + p] * sum_pl Bt[pl * bplane + q * ldb + k]
// (A: gradient rows k; Bt: codes transposed, k contiguous, zero beyond K up to a multiple of 32).
// colsum (optional, [S][P]): sums of A over each split's k.  S splits of kper rows (kper a
// multiple of 32).  A must be 16-byte aligned, with lda and P multiples of 4.
struct TnArgs {
  const float *A;
  int64_t lda;
  const __bf16 *Bt;
  int64_t ldb, bplane;
  int K, P, Q, S, kper;
  float *part;
  float *colsum;
};

// out[m * ldo + n] = sum_k (A[m * lda + k] * kscale[k]) * sum_pl Bt[pl * bplane + n * ldb + k]
// (A: gradient rows m, k contiguous; Bt: codes, k contiguous, zero beyond K up to a multiple
// of 32; A, kscale and Bt 16-byte aligned, lda a multiple of 4, K a multiple of 16).
struct NtArgs {
  const float *A;
  int64_t lda;
  const float *kscale;
  const __bf16 *Bt;
  int64_t ldb, bplane;
  int M, N, K;
  float *out;
  int64_t ldo;
  // optional K split: split z sums k in [z kper, min((z + 1) kper, K)) into out + z out_split
  int ksplit = 1, kper = 0;
  int64_t out_split = 0;
};

// Number of K splits for a TN product and rows per split (a makespan model over the GPU's CUs
// that also prices the partial sums each split adds).
void tn_plan(int K, int P, int Q, int nplanes, int *S, int *kper);
// K split of an NT product for about two waves per SIMD, at most max_split parts (kper = K
// when S = 1).
void nt_plan(int M, int N, int K, int max_split, int *S, int *kper);
// Launches; nplanes is 1 or 2.
int tn(const TnArgs &a, int nplanes, hipStream_t stream);
int nt(const NtArgs &a, int nplanes, hipStream_t stream);
// out[p * ldo + q] = qscale[q] * sum_s part[s][p][q] (fixed order; out[q * ldo + p] when
// transpose); qscale may be null (1).  bias (optional): bias[p * ldo] = the sum of colsum over
// the splits.
// mask (optional): out is multiplied by mask[q * P + p]; swap_h > 0: row (or column, when
// transpose) p is written at the index with the first two blocks of swap_h swapped (the
// (z, r, n) <-> (r, z, n) gate order of the GRU).
int tn_finish(const float *part, int S, int P, int Q, int nplanes, const float *qscale, float *out,
              int64_t ldo, bool transpose, const float *colsum, float *bias, hipStream_t stream,
              const uint8_t *mask = nullptr, int swap_h = 0);

// Codes as bf16 operand planes, transposed: for r < rows and c < cols,
//   v = rint((x(r, c) - zp) / div),  x(r, c) = r < rows0 ? src0[r rs + c cs] : src1[(r - rows0) rs + c cs]
// (div = 1 for stored codes; div = the scale for dequantised values (q - zp) s, which it
// inverts exactly for |q - zp| < 2^16); with one plane dst[c * ldd + r] = v (|v| <= 256), with
// two planes dst[c * ldd + r] = 256 (v >> 8) and dst[plane + c * ldd + r] = v & 255.  Rows
// rows..ldd-1 are written as zeros.
int codes_t(const float *src0, int64_t rows0, const float *src1, int64_t rows, int cols, int64_t rs,
            int64_t cs, float zp, float div, int nplanes, __bf16 *dst, int64_t ldd, int64_t plane,
            hipStream_t stream);
// Planes needed for integer codes in [lo, hi] centred on zp.
inline int planes_for(double lo, double hi, double zp) {
  const double a = lo - zp < 0 ? zp - lo : lo - zp, b = hi - zp < 0 ? zp - hi : hi - zp;
  return (a > b ? a : b) <= 256.0 ? 1 : 2;
}

}  // namespace wgrad
}  // namespace rxmet
