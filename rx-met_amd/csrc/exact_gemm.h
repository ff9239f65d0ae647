// exact_gemm.h — exact integer GEMM of fp32-stored quantisation codes on int8 MFMA.
//
//   S[m][n] = sum_k (A[m][k] - base) * B(k, n)
//
// for integer-valued codes.  A is shifted by `off` (from the bottom of its grid) into the
// signed range of PA byte planes: one plane holds [-128, 127], two planes (v = 256 hi + lo,
// both in [-128, 127]) hold [-32896, 32639].  B is used as is: one signed byte plane for codes
// in [-128, 127], or two planes for 16-bit codes, B = 256 bh + bl + 128 with bh = B >> 8 and
// bl = (B & 255) - 128.  Every plane pair accumulates exactly in int32 on
// v_mfma_i32_16x16x64_i8 (|sum| <= K * 2^14 < 2^31 for K < 2^17); the row sums of A and the
// column sums of B come from the same MFMA against an all-ones fragment; everything is
// combined in int64:
//   sum_k (A - off) B  = sum_pa sum_pb 256^pa w_pb acc[pa][pb]  (+ 128 rowsum(A - off) if PB=2)
//   S                  = sum_k (A - off) B + (off - base) colsum(B).
//
// Workgroup: 256 threads, a 64 x 64 block of outputs; wave w owns rows 32 (w / 2) .. +31 and
// columns 32 (w % 2) .. +31 as 2 x 2 tiles of 16 x 16.  K advances in chunks of 64 staged in
// LDS as byte planes ([row][k] for A, [column][k] for B).
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

#include "mfma_frag.h"

namespace rxmet {
namespace xgemm {

constexpr int kTile = 64;
constexpr int kRowBytes = 64 + 16;  // LDS row stride (conflict-free 16-byte reads)

// Codes stored as fp32 (integer valued) or as int32.
template <typename EA, typename EB>
struct OperandsT {
  int M, N, K;
  const EA *A;     // A[m * lda + k]
  int lda;
  float off;       // shift of A (integer valued)
  long long corr;  // off - base
  const EB *B;     // B(k, n) = B[k * sbk + n * sbn]
  int sbk, sbn;
};
using Operands = OperandsT<float, float>;

// Computes the 64 x 64 block at (tm, tn) and calls epi(m, n, S) for every in-range output.
template <int PA, int PB, typename EA, typename EB, typename Epi>
__device__ __forceinline__ void block(const OperandsT<EA, EB> &o, int tm, int tn, Epi epi) {
  __shared__ __align__(16) int8_t As[PA][kTile][kRowBytes];
  __shared__ __align__(16) int8_t Bs[PB][kTile][kRowBytes];
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int wm = 32 * (w / 2), wn = 32 * (w % 2);
  v4i acc[PA][PB][2][2];
  v4i csum[PB][2], rsum[PA][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int pa = 0; pa < PA; ++pa)
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) acc[pa][pb][i][j] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) csum[pb][i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int pa = 0; pa < PA; ++pa) rsum[pa][i] = v4i{0, 0, 0, 0};
  }
  const int one = 0x01010101;
  const v4i ones = {one, one, one, one};
  const bool b_nmajor = o.sbn == 1;  // B stored [K][N]: coalesce along n
  int kp = 0;                        // k positions processed (padding included)
  for (int k0 = 0; k0 < o.K; k0 += kTile, kp += kTile) {
    for (int e = tid; e < kTile * kTile; e += 256) {
      const int r = e / kTile, kk = e % kTile;
      const int gm = tm + r, gk = k0 + kk;
      int v = 0;
      if (gm < o.M && gk < o.K)
        v = static_cast<int>(o.A[static_cast<size_t>(gm) * o.lda + gk]) - static_cast<int>(o.off);
      if (PA == 1) {
        As[0][r][kk] = static_cast<int8_t>(v);
      } else {
        const int lo = ((v + 128) & 255) - 128;
        As[0][r][kk] = static_cast<int8_t>(lo);
        As[PA - 1][r][kk] = static_cast<int8_t>((v - lo) >> 8);
      }
    }
    for (int e = tid; e < kTile * kTile; e += 256) {
      const int n = b_nmajor ? e % kTile : e / kTile, kk = b_nmajor ? e / kTile : e % kTile;
      const int gn = tn + n, gk = k0 + kk;
      int v = 0;
      if (gn < o.N && gk < o.K)
        v = static_cast<int>(o.B[static_cast<size_t>(gk) * o.sbk + static_cast<size_t>(gn) * o.sbn]);
      if (PB == 1) {
        Bs[0][n][kk] = static_cast<int8_t>(v);
      } else {
        Bs[0][n][kk] = static_cast<int8_t>((v & 255) - 128);
        Bs[PB - 1][n][kk] = static_cast<int8_t>(v >> 8);
      }
    }
    __syncthreads();
    v4i af[PA][2], bf[PB][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int pa = 0; pa < PA; ++pa)
        af[pa][i] = *reinterpret_cast<const v4i *>(&As[pa][wm + 16 * i + l % 16][16 * (l / 16)]);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb)
        bf[pb][i] = *reinterpret_cast<const v4i *>(&Bs[pb][wn + 16 * i + l % 16][16 * (l / 16)]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int pa = 0; pa < PA; ++pa)
#pragma unroll
          for (int pb = 0; pb < PB; ++pb)
            acc[pa][pb][i][j] = mfma_i8(af[pa][i], bf[pb][j], acc[pa][pb][i][j]);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) csum[pb][j] = mfma_i8(ones, bf[pb][j], csum[pb][j]);
    if (PB == 2) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int pa = 0; pa < PA; ++pa) rsum[pa][i] = mfma_i8(af[pa][i], ones, rsum[pa][i]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = tn + wn + 16 * j + l % 16;
    long long cs = csum[0][j][0];
    if (PB == 2) cs = 256LL * csum[PB - 1][j][0] + cs + 128LL * kp;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = tm + wm + 16 * i + 4 * (l / 16) + r;
        if (m >= o.M || n >= o.N) continue;
        long long s = o.corr * cs;
#pragma unroll
        for (int pa = 0; pa < PA; ++pa) {
#pragma unroll
          for (int pb = 0; pb < PB; ++pb)
            s += static_cast<long long>(acc[pa][pb][i][j][r]) << (8 * (pa + pb));
          if (PB == 2) s += (static_cast<long long>(rsum[pa][i][r]) << (8 * pa)) * 128;
        }
        epi(m, n, s);
      }
  }
}

// Planes and shift for A codes in [lo, hi]; planes of B for codes in [lo, hi].
inline int a_planes(double lo, double hi) { return hi - lo <= 255.0 ? 1 : 2; }
inline float a_shift(double lo, double hi) {
  return static_cast<float>(hi - lo <= 255.0 ? lo + 128.0 : lo + 32896.0);
}
inline int b_planes(double lo, double hi) { return (lo >= -128.0 && hi <= 127.0) ? 1 : 2; }
// Ranges the planes can carry: A spans at most 2^16 codes, B is within signed 16 bits.
inline bool a_fits(double lo, double hi) { return hi - lo <= 65535.0; }
inline bool b_fits(double lo, double hi) { return lo >= -32768.0 && hi <= 32767.0; }

// ---------------------------------------------------------------------------------
// Pre-packed variant: both operands prepared once per call (pack_a, pack_b below), so the
// GEMM streams 16-byte MFMA fragments straight from L2 with no staging.
//   A planes   : int8 [PA][M][Kp] of v = A - off (low byte first; Kp = K rounded up to 64,
//                zero beyond K),
//   B fragments: v4i [PB][N / 16][Kp / 64][64]; lane l of fragment (nt, s) holds
//                B(64 s + 16 (l / 16) + j, 16 nt + l % 16), j = 0..15 (plane as above),
//   colsum     : int64 [N], sum over k < K of B(k, n).
// S(m, n) = sum_k (A - base) B = sum_k (A - off) B + (off - base) colsum(n).
// ---------------------------------------------------------------------------------
struct Packed {
  const int8_t *A;
  int64_t aplane;   // bytes between A planes (M Kp)
  int Kp;
  const v4i *B;
  int64_t bplane;   // fragments between B planes
  const long long *colsum;
  long long corr;   // off - base
  int M, N;
};

// Rows m0..m0+15 of one wave against every 16-column tile nt0, nt0 + step, ...; per tile each
// lane calls epi(m, n, S, rows) with the S of rows m, m + 1, .., m + rows - 1 of its column n
// (rows <= 4: the in-range ones).
template <int PA, int PB, typename Epi>
__device__ __forceinline__ void rows16(const Packed &p, int m0, int nt0, int step, Epi epi) {
  const int l = threadIdx.x % 64, KS = p.Kp / 64;
  const int ntiles = (p.N + 15) / 16;
  const int mrow = m0 + l % 16;
  const bool rin = mrow < p.M;
  const int8_t *arow = p.A + static_cast<int64_t>(rin ? mrow : 0) * p.Kp + 16 * (l / 16);
  constexpr int kMaxKS = 4;  // K <= 256
  v4i af[PA][kMaxKS];
#pragma unroll
  for (int pa = 0; pa < PA; ++pa)
#pragma unroll
    for (int s = 0; s < kMaxKS; ++s) {
      const v4i v = *reinterpret_cast<const v4i *>(arow + pa * p.aplane + 64 * (s < KS ? s : 0));
      af[pa][s] = (rin && s < KS) ? v : v4i{0, 0, 0, 0};
    }
  long long rs[PA][4];
  if (PB == 2) {
    const int one = 0x01010101;
    const v4i ones = {one, one, one, one};
#pragma unroll
    for (int pa = 0; pa < PA; ++pa) {
      v4i acc = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < kMaxKS; ++s)
        if (s < KS) acc = mfma_i8(af[pa][s], ones, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) rs[pa][r] = acc[r];
    }
  }
  for (int nt = nt0; nt < ntiles; nt += step) {
    v4i acc[PA][PB];
#pragma unroll
    for (int pa = 0; pa < PA; ++pa)
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) acc[pa][pb] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kMaxKS; ++s) {
      if (s >= KS) break;
      v4i bf[PB];
#pragma unroll
      for (int pb = 0; pb < PB; ++pb)
        bf[pb] = p.B[pb * p.bplane + (static_cast<int64_t>(nt) * KS + s) * 64 + l];
#pragma unroll
      for (int pa = 0; pa < PA; ++pa)
#pragma unroll
        for (int pb = 0; pb < PB; ++pb) acc[pa][pb] = mfma_i8(af[pa][s], bf[pb], acc[pa][pb]);
    }
    const int n = 16 * nt + l % 16;
    if (n >= p.N) continue;
    const long long cs = p.corr * p.colsum[n];
    long long sum[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sum[r] = cs;
#pragma unroll
      for (int pa = 0; pa < PA; ++pa) {
#pragma unroll
        for (int pb = 0; pb < PB; ++pb)
          sum[r] += static_cast<long long>(acc[pa][pb][r]) << (8 * (pa + pb));
        if (PB == 2) sum[r] += (rs[pa][r] << (8 * pa)) * 128;
      }
    }
    const int mfirst = m0 + 4 * (l / 16);
    const int rows = p.M - mfirst >= 4 ? 4 : p.M - mfirst;
    if (rows > 0) epi(mfirst, n, sum, rows);
  }
}

// Host launchers (exact_gemm.hip), for codes stored as fp32 or int32.
int pack_a(const float *A, int64_t lda, int M, int K, float off, int PA, int8_t *out, int Kp,
           hipStream_t stream);
int pack_a(const int32_t *A, int64_t lda, int M, int K, float off, int PA, int8_t *out, int Kp,
           hipStream_t stream);
// B(k, n) = B[k sbk + n sbn] (integer codes), PB planes.
int pack_b(const float *B, int64_t sbk, int64_t sbn, int K, int N, int PB, int Kp, v4i *frag,
           long long *colsum, hipStream_t stream);
int pack_b(const int32_t *B, int64_t sbk, int64_t sbn, int K, int N, int PB, int Kp, v4i *frag,
           long long *colsum, hipStream_t stream);
inline int pad_k(int K) { return (K + 63) / 64 * 64; }

}  // namespace xgemm
}  // namespace rxmet
