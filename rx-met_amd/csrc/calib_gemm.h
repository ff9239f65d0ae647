// calib_gemm.h — the calibration passes' input projection on fp32 MFMA (gfx950), shared by the
// GRU (gru_calib.hip) and LSTM (lstm_calib.hip) calibration forwards.
//
// out[m][n] = sum_k x[m][k] B(k, n) + bias[n] for m < M, n < N, with the input statistics
// observed on the way: every in-range element of x once (by the workgroups of column block 0)
// and every output.  B(k, n) is W[k * N + n] (K-major, GRU W [I][3H]) or W[n * K + k] (N-major,
// LSTM W_ih [4H][I]).
//
// A workgroup computes a 128 x 128 block of out: four waves of 64 x 64, each a 4 x 4 array of
// v_mfma_f32_16x16x4f32 tiles.  K advances 16 at a time through LDS tiles of x and B stored
// k-contiguous ([128][kKp] each, double buffered), so that a lane's four k values of one MFMA
// tile are one 16-byte LDS read; the next step's global loads are in flight during this step's
// MFMAs.  MFMA k slot g of lane group g takes k = k0 + 4 g + s at sub-step s, in the A and B
// operands alike.
#pragma once

#include <stdint.h>

#include "mfma_frag.h"
#include "rxmet_common.h"

namespace rxmet {
namespace calgemm {

constexpr int kBM = 128, kBN = 128, kBK = 16;
constexpr int kKp = kBK + 4;  // LDS row: 16 k + 4 pad floats (16-byte aligned rows)

// One workgroup (256 threads): block (blockIdx.x, blockIdx.y) of 128 columns x 128 rows.
template <bool B_KMAJOR, class ObsX, class ObsOut>
__device__ __forceinline__ void gemm_block(int M, int N, int K, const float *__restrict__ x,
                                           const float *__restrict__ W,
                                           const float *__restrict__ bias,
                                           float *__restrict__ out, bool see_x, ObsX obs_x,
                                           ObsOut obs_out) {
  __shared__ __align__(16) float As[2][kBM][kKp];
  __shared__ __align__(16) float Bs[2][kBN][kKp];
  const int tid = threadIdx.x;
  const int w = tid / kWave, l = tid % kWave, r = l % 16, g = l / 16;
  const int wm = w / 2, wn = w % 2;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  // 16-byte loads where rows and bases allow them
  const bool xvec = K % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const bool wvec = (B_KMAJOR ? N % 4 == 0 : K % 4 == 0) &&
                    (reinterpret_cast<uintptr_t>(W) & 15) == 0;
  // global -> register staging of one K step: x rows (tid / 4 + 64 h, k quad tid % 4) and
  // B: K-major, k row tid % 16 with four n from 4 (tid / 16 + 16 h) (lanes vary k fastest, so
  // the transposing LDS stores of a wave fall in distinct banks); N-major, n row tid / 4 + 64 h
  // with k quad tid % 4
  float4 xa[2], wb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = m0 + tid / 4 + 64 * h, kk = k0 + 4 * (tid % 4);
      const float *p = x + static_cast<size_t>(row) * K + kk;
      if (row < M && xvec && kk + 3 < K) {
        xa[h] = *reinterpret_cast<const float4 *>(p);
      } else {
        xa[h].x = row < M && kk < K ? p[0] : 0.0f;
        xa[h].y = row < M && kk + 1 < K ? p[1] : 0.0f;
        xa[h].z = row < M && kk + 2 < K ? p[2] : 0.0f;
        xa[h].w = row < M && kk + 3 < K ? p[3] : 0.0f;
      }
      if (B_KMAJOR) {
        const int k = k0 + tid % 16, n = n0 + 4 * (tid / 16 + 16 * h);
        const float *q = W + static_cast<size_t>(k) * N + n;
        if (wvec && k < K && n + 3 < N) {
          wb[h] = *reinterpret_cast<const float4 *>(q);
        } else {
          wb[h].x = k < K && n < N ? q[0] : 0.0f;
          wb[h].y = k < K && n + 1 < N ? q[1] : 0.0f;
          wb[h].z = k < K && n + 2 < N ? q[2] : 0.0f;
          wb[h].w = k < K && n + 3 < N ? q[3] : 0.0f;
        }
      } else {
        const int n = n0 + tid / 4 + 64 * h, kq = k0 + 4 * (tid % 4);
        const float *q = W + static_cast<size_t>(n) * K + kq;
        if (n < N && wvec && kq + 3 < K) {
          wb[h] = *reinterpret_cast<const float4 *>(q);
        } else {
          wb[h].x = n < N && kq < K ? q[0] : 0.0f;
          wb[h].y = n < N && kq + 1 < K ? q[1] : 0.0f;
          wb[h].z = n < N && kq + 2 < K ? q[2] : 0.0f;
          wb[h].w = n < N && kq + 3 < K ? q[3] : 0.0f;
        }
      }
    }
  };
  auto store = [&](int buf, int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = tid / 4 + 64 * h, kq = 4 * (tid % 4);
      *reinterpret_cast<float4 *>(&As[buf][rl][kq]) = xa[h];
      if (see_x && m0 + rl < M) {  // the zeros loaded past M and K are not values of x
        const int kk = k0 + kq;
        if (kk < K) obs_x(xa[h].x);
        if (kk + 1 < K) obs_x(xa[h].y);
        if (kk + 2 < K) obs_x(xa[h].z);
        if (kk + 3 < K) obs_x(xa[h].w);
      }
      if (B_KMAJOR) {
        const int kl = tid % 16, nl = 4 * (tid / 16 + 16 * h);
        Bs[buf][nl][kl] = wb[h].x;
        Bs[buf][nl + 1][kl] = wb[h].y;
        Bs[buf][nl + 2][kl] = wb[h].z;
        Bs[buf][nl + 3][kl] = wb[h].w;
      } else {
        *reinterpret_cast<float4 *>(&Bs[buf][rl][kq]) = wb[h];
      }
    }
  };
  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  load(0);
  store(0, 0);
  __syncthreads();
  int cur = 0;
  for (int k0 = 0; k0 < K; k0 += kBK) {
    const bool more = k0 + kBK < K;
    if (more) load(k0 + kBK);
    v4f a4[4], b4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a4[i] = *reinterpret_cast<const v4f *>(&As[cur][wm * 64 + 16 * i + r][4 * g]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b4[j] = *reinterpret_cast<const v4f *>(&Bs[cur][wn * 64 + 16 * j + r][4 * g]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_f32(a4[i][s], b4[j][s], acc[i][j]);
    if (more) store(cur ^ 1, k0 + kBK);
    __syncthreads();
    cur ^= 1;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = n0 + wn * 64 + 16 * j + r;
    if (col >= N) continue;
    const float b = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = m0 + wm * 64 + 16 * i + 4 * g + q;
        if (row < M) {
          const float v = acc[i][j][q] + b;
          out[static_cast<size_t>(row) * N + col] = v;
          obs_out(v);
        }
      }
  }
}

}  // namespace calgemm
}  // namespace rxmet
