// exact_gemm.hip — operand packing for the pre-packed exact GEMM (exact_gemm.h), for codes
// stored as fp32 or int32.
#include <type_traits>

#include "exact_gemm.h"

#include "rxmet_common.h"

namespace rxmet {
namespace xgemm {

// A planes: four k per thread, written as one 32-bit word per plane.
template <typename E>
__global__ __launch_bounds__(256) void pack_a_kernel(const E *__restrict__ A, int64_t lda, int M,
                                                     int K, float off, int PA, int8_t *__restrict__ out,
                                                     int Kp) {
  const int64_t words = static_cast<int64_t>(M) * (Kp / 4), plane = static_cast<int64_t>(M) * Kp;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const unsigned kq = static_cast<unsigned>(Kp / 4);
  // whole 4-element groups of a row as one 16-byte load where the rows allow it
  const bool vec = std::is_same<E, float>::value && lda % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(A) & 15) == 0;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < words; w += stride) {
    // 32-bit division where the word index fits (a 64-bit one is a long software sequence)
    int64_t m;
    int k0;
    if (words <= 0x7fffffff) {
      const unsigned mw = static_cast<unsigned>(w) / kq;
      m = mw;
      k0 = static_cast<int>(static_cast<unsigned>(w) - mw * kq) * 4;
    } else {
      m = w / kq;
      k0 = static_cast<int>(w % kq) * 4;
    }
    E a4[4];
    if (vec && k0 + 3 < K) {
      const float4 v4 = *reinterpret_cast<const float4 *>(A + m * lda + k0);
      a4[0] = v4.x; a4[1] = v4.y; a4[2] = v4.z; a4[3] = v4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) a4[e] = k0 + e < K ? A[m * lda + k0 + e] : E(0);
    }
    unsigned lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + e;
      const int v = k < K ? static_cast<int>(a4[e]) - static_cast<int>(off) : 0;
      if (PA == 1) {
        lo |= static_cast<unsigned>(v & 255) << (8 * e);
      } else {
        const int l8 = ((v + 128) & 255) - 128;
        lo |= static_cast<unsigned>(l8 & 255) << (8 * e);
        hi |= static_cast<unsigned>(((v - l8) >> 8) & 255) << (8 * e);
      }
    }
    reinterpret_cast<unsigned *>(out)[w] = lo;
    if (PA == 2) reinterpret_cast<unsigned *>(out + plane)[w] = hi;
  }
}

// B fragments: block (nt, s), lane l packs 16 k of column 16 nt + l % 16; the s == 0 blocks
// also sum each column exactly.
template <typename E>
__global__ __launch_bounds__(64) void pack_b_kernel(const E *__restrict__ B, int64_t sbk,
                                                    int64_t sbn, int K, int N, int PB, int Kp,
                                                    v4i *__restrict__ frag,
                                                    long long *__restrict__ colsum) {
  const int l = threadIdx.x, KS = Kp / 64;
  const int nt = blockIdx.x / KS, s = blockIdx.x % KS;
  const int n = 16 * nt + l % 16;
  const int64_t fplane = static_cast<int64_t>((N + 15) / 16) * KS * 64;
  int w0[4], w1[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int b0 = 0, b1 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 64 * s + 16 * (l / 16) + 4 * q + e;
      const int v = (k < K && n < N) ? static_cast<int>(B[k * sbk + n * sbn]) : 0;
      if (PB == 1) {
        b0 |= (v & 255) << (8 * e);
      } else {
        b0 |= (((v & 255) - 128) & 255) << (8 * e);
        b1 |= ((v >> 8) & 255) << (8 * e);
      }
    }
    w0[q] = b0;
    w1[q] = b1;
  }
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 64 + l;
  frag[idx] = v4i{w0[0], w0[1], w0[2], w0[3]};
  if (PB == 2) frag[fplane + idx] = v4i{w1[0], w1[1], w1[2], w1[3]};
  // column sums (exact in int64, so the order does not matter): the wave of K-step 0, lane
  // group l / 16 taking every fourth k of column n, then the four groups added by shuffles
  if (s == 0) {
    long long sum = 0;
    if (n < N) {
#pragma unroll 4
      for (int k = l / 16; k < K; k += 4) sum += static_cast<long long>(B[k * sbk + n * sbn]);
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (l < 16 && n < N) colsum[n] = sum;
  }
}

template <typename E>
static int pack_a_t(const E *A, int64_t lda, int M, int K, float off, int PA, int8_t *out, int Kp,
                    hipStream_t stream) {
  RXMET_CHECK_ARG((PA == 1 || PA == 2) && Kp % 64 == 0 && Kp >= K, "bad A packing");
  const int64_t words = static_cast<int64_t>(M) * (Kp / 4);
  int64_t blocks = (words + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(pack_a_kernel<E>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     A, lda, M, K, off, PA, out, Kp);
  RXMET_CHECK_LAUNCH();
  return 0;
}

template <typename E>
static int pack_b_t(const E *B, int64_t sbk, int64_t sbn, int K, int N, int PB, int Kp, v4i *frag,
                    long long *colsum, hipStream_t stream) {
  RXMET_CHECK_ARG((PB == 1 || PB == 2) && Kp % 64 == 0 && Kp >= K, "bad B packing");
  const int blocks = ((N + 15) / 16) * (Kp / 64);
  hipLaunchKernelGGL(pack_b_kernel<E>, dim3(blocks), dim3(64), 0, stream, B, sbk, sbn, K, N, PB,
                     Kp, frag, colsum);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int pack_a(const float *A, int64_t lda, int M, int K, float off, int PA, int8_t *out, int Kp,
           hipStream_t stream) {
  return pack_a_t(A, lda, M, K, off, PA, out, Kp, stream);
}
int pack_a(const int32_t *A, int64_t lda, int M, int K, float off, int PA, int8_t *out, int Kp,
           hipStream_t stream) {
  return pack_a_t(A, lda, M, K, off, PA, out, Kp, stream);
}
int pack_b(const float *B, int64_t sbk, int64_t sbn, int K, int N, int PB, int Kp, v4i *frag,
           long long *colsum, hipStream_t stream) {
  return pack_b_t(B, sbk, sbn, K, N, PB, Kp, frag, colsum, stream);
}
int pack_b(const int32_t *B, int64_t sbk, int64_t sbn, int K, int N, int PB, int Kp, v4i *frag,
           long long *colsum, hipStream_t stream) {
  return pack_b_t(B, sbk, sbn, K, N, PB, Kp, frag, colsum, stream);
}

}  // namespace xgemm
}  // namespace rxmet
