// gru_bidir.hip — the layout work at the boundary of a bidirectional QuantGRU layer.
//
// A bidirectional layer runs the reverse direction on the time-reversed input and returns
// output[t] = [h_fwd(t), h_rev(T-1-t)] in the caller's layout ([T, B, 2H] or batch-first
// [B, T, 2H]) and h_n = [h_fwd(T), h_rev(T)] (quant_gru.py:2270-2288 and 1402-1432 of the
// reference, which flips, concatenates and transposes with separate tensor copies).  These
// kernels do each of those copies in one pass:
//   bidir_assemble  : both directions' h -> output and h_n,
//   bidir_split_grad: the output gradient (any strides) -> each direction's dh_new [T+1, B, H],
//   bidir_dx        : dx of both directions -> the input gradient in the caller's layout.
// The forward's reversed, strided x reads are part of quant_input (gru_fwd.hip).
#include <cstdint>

#include <hip/hip_runtime.h>

#include "rxmet_common.h"
#include "rxmet_gru.h"

namespace rxmet {
namespace gru {

// One thread per 4 consecutive values of a row of 2H; h_f, h_r: [T+1, B, H] (row 0 = h0).
// Ix: the type of the element index and of its divisions (32-bit whenever the count fits: a
// 64-bit division is a long software sequence on the GPU).
template <typename Ix>
__global__ __launch_bounds__(256) void bidir_assemble(int T, int B, int H, const float *__restrict__ h_f,
                                                      const float *__restrict__ h_r,
                                                      float *__restrict__ out, int64_t st, int64_t sb,
                                                      float *__restrict__ h_n) {
  const Ix q4 = H / 2;  // float4 per output row
  const Ix n = static_cast<Ix>(T) * B * q4;
  const Ix stride = static_cast<Ix>(gridDim.x) * blockDim.x;
  const size_t BH = static_cast<size_t>(B) * H;
  for (Ix i = static_cast<Ix>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const Ix row = i / q4;
    const int q = static_cast<int>(i - row * q4);
    const Ix tq = row / static_cast<Ix>(B);
    const int b = static_cast<int>(row - tq * B), t = static_cast<int>(tq);
    const int k = 4 * q;
    const float4 v = k < H
        ? *reinterpret_cast<const float4 *>(h_f + (t + 1) * BH + static_cast<size_t>(b) * H + k)
        : *reinterpret_cast<const float4 *>(h_r + (T - t) * BH + static_cast<size_t>(b) * H + k - H);
    *reinterpret_cast<float4 *>(out + t * st + b * sb + k) = v;
  }
  if (h_n) {
    const int64_t m = 2 * static_cast<int64_t>(B) * H / 4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < m; i += stride) {
      const int64_t e = 4 * i;
      const float *src = e < static_cast<int64_t>(BH) ? h_f + T * BH + e : h_r + T * BH + (e - BH);
      *reinterpret_cast<float4 *>(h_n + e) = *reinterpret_cast<const float4 *>(src);
    }
  }
}

// dh_f[s + 1][b][j] = g[s][b][j] (+ g_hn[0][b][j] at s = T-1), dh_r[s + 1][b][j] =
// g[T-1-s][b][H + j] (+ g_hn[1][b][j] at s = T-1); row 0 of both is zero.  g element (t, b, k)
// at g[t gt + b gb + k gk] (strides may be zero); g or g_hn may be absent (zero).  One thread
// per four consecutive units, written as one 16-byte store (H is a multiple of 4).
template <typename Ix>
__global__ __launch_bounds__(256) void bidir_split_grad(int T, int B, int H, const float *__restrict__ g,
                                                        int64_t gt, int64_t gb, int64_t gk,
                                                        const float *__restrict__ g_hn,
                                                        float *__restrict__ dh_f,
                                                        float *__restrict__ dh_r) {
  const Ix h4 = H / 4;
  const Ix rows = static_cast<Ix>(T + 1) * B;  // rows of one direction
  const Ix n = 2 * rows * h4;
  const Ix stride = static_cast<Ix>(gridDim.x) * blockDim.x;
  const size_t BH = static_cast<size_t>(B) * H;
  for (Ix i = static_cast<Ix>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const Ix row2 = i / h4;
    const int j = 4 * static_cast<int>(i - row2 * h4);
    const int dir = row2 >= rows ? 1 : 0;
    const Ix row = row2 - dir * rows;
    const Ix sq = row / static_cast<Ix>(B);
    const int s1 = static_cast<int>(sq), b = static_cast<int>(row - sq * B);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (s1 > 0) {
      const int t = dir == 0 ? s1 - 1 : T - s1;
      if (g) {
        const float *src = g + t * gt + b * gb + (static_cast<int64_t>(dir) * H + j) * gk;
        v = make_float4(src[0], src[gk], src[2 * gk], src[3 * gk]);
      }
      if (g_hn && s1 == T) {
        const float *h = g_hn + dir * BH + static_cast<size_t>(b) * H + j;
        v.x += h[0];
        v.y += h[1];
        v.z += h[2];
        v.w += h[3];
      }
    }
    *reinterpret_cast<float4 *>((dir == 0 ? dh_f : dh_r) + static_cast<size_t>(row) * H + j) = v;
  }
}

// dx[t st + b sb + i] = dx_f[t][b][i] + dx_r[T-1-t][b][i].
template <typename Ix>
__global__ __launch_bounds__(256) void bidir_dx(int T, int B, int I, const float *__restrict__ dx_f,
                                                const float *__restrict__ dx_r, float *__restrict__ dx,
                                                int64_t st, int64_t sb) {
  const Ix n = static_cast<Ix>(T) * B * I;
  const Ix stride = static_cast<Ix>(gridDim.x) * blockDim.x;
  const Ix BI = static_cast<Ix>(B) * I;
  for (Ix e = static_cast<Ix>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const Ix tq = e / BI;
    const Ix rem = e - tq * BI;
    const Ix bq = rem / static_cast<Ix>(I);
    const int t = static_cast<int>(tq), b = static_cast<int>(bq), i = static_cast<int>(rem - bq * I);
    dx[t * st + b * sb + i] = dx_f[e] + dx_r[static_cast<size_t>(T - 1 - t) * BI + rem];
  }
}

// Element counts (plus one grid stride) that 32-bit index arithmetic covers.
static bool fits32(int64_t n) { return n + 8192LL * 256 < (1LL << 32); }

static unsigned grid_for(int64_t n) {
  int64_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks > 8192 ? 8192 : (blocks < 1 ? 1 : blocks));
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int rxmet_gru_bidir_assemble(int32_t T, int32_t B, int32_t H, const float *h_f, const float *h_r,
                             float *out, int64_t out_st, int64_t out_sb, float *h_n, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && H >= 1 && H % 4 == 0, "bad dimensions (H a multiple of 4)");
  RXMET_CHECK_ARG(h_f && h_r && out, "required pointer is null");
  RXMET_CHECK_ARG(out_st % 4 == 0 && out_sb % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(h_f) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(h_r) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(h_n) & 15u) == 0,
                  "outputs and strides must allow 16-byte rows");
  const int64_t n = static_cast<int64_t>(T) * B * (H / 2);
  hipLaunchKernelGGL((fits32(n) ? bidir_assemble<uint32_t> : bidir_assemble<int64_t>), dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     T, B, H, h_f, h_r, out, out_st, out_sb, h_n);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_gru_bidir_split_grad(int32_t T, int32_t B, int32_t H, const float *g, int64_t g_st,
                               int64_t g_sb, int64_t g_sk, const float *g_hn, float *dh_f,
                               float *dh_r, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && H >= 1 && H % 4 == 0, "bad dimensions (H a multiple of 4)");
  RXMET_CHECK_ARG(dh_f && dh_r, "required pointer is null");
  RXMET_CHECK_ARG((reinterpret_cast<uintptr_t>(dh_f) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(dh_r) & 15u) == 0,
                  "dh_new buffers must be 16-byte aligned");
  const int64_t n = 2 * static_cast<int64_t>(T + 1) * B * (H / 4);
  hipLaunchKernelGGL((fits32(n) ? bidir_split_grad<uint32_t> : bidir_split_grad<int64_t>), dim3(grid_for(n)), dim3(256),
                     0, static_cast<hipStream_t>(stream),
                     T, B, H, g, g_st, g_sb, g_sk, g_hn, dh_f, dh_r);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_gru_bidir_dx(int32_t T, int32_t B, int32_t I, const float *dx_f, const float *dx_r,
                       float *dx, int64_t dx_st, int64_t dx_sb, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1, "bad dimensions");
  RXMET_CHECK_ARG(dx_f && dx_r && dx, "required pointer is null");
  const int64_t n = static_cast<int64_t>(T) * B * I;
  hipLaunchKernelGGL((fits32(n) ? bidir_dx<uint32_t> : bidir_dx<int64_t>), dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), T, B,
                     I, dx_f, dx_r, dx, dx_st, dx_sb);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
