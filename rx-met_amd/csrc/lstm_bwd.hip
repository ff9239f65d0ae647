// lstm_bwd.hip — MI355X QuantLSTM STE backward, behind rxmet_lstm_backward_quant.
//
// Reference path: lstm_backward_qat (pytorch/lib/lstm_interface_binding.cc:437-480)
// dequantises the saved masters and checkpoints (dequantizeQCarrierKernel, double) and runs
// lstmBackwardFloatCuda (src/lstm/backward_float_cuda.cu:189-330): per step t = T-1..0 the
// pointwise backward with the clamp masks (:50-104) and an SGEMM dh = dgates_hh W_hh, then
// the dx / dW_ih / dW_hh SGEMMs, a bias column reduction and seven mask passes.
//
// Here:
//   1. prologue  : x and h_prev codes and the W_ih codes as bf16 operand planes for the
//                  weight-gradient GEMMs; W_hh codes packed as int8 MFMA fragments of the
//                  transposed product, with their column sums;
//   2. recurrence: a batch tile's dh product over a cluster of workgroups
//                  (lstm_bwd_recurrence_cl; the per-tile fallback lstm_bwd_recurrence keeps
//                  one workgroup per 16 sequences).  Per step: the pointwise backward with
//                  every mask family in the reference's operation order; dgates_hh * scale_W
//                  published as 22-bit block fixed point (a per-sequence exponent from the
//                  row maximum) in three int8 planes; after the cluster barrier,
//                  dh = W_hh_deq^T dgates_hh on int8 MFMA against the resident W_hh codes,
//                  recombined exactly in double; the gate gradients for the GEMMs go out as
//                  16-byte rows staged in LDS while the members wait, and the next step's
//                  checkpoints are copied into LDS meanwhile;
//   3. GEMMs     : dx, dW_ih | db_ih and dW_hh | db_hh on bf16 MFMA with the gradients split
//                  exactly into three bf16 terms (wgrad_gemm.h), the bias columns from fused
//                  column sums; one pass applies the master masks.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <vector>

#include "cluster.h"
#include "lstm_internal.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_lstm.h"
#include "wgrad_gemm.h"

namespace rxmet {
namespace lstm {

constexpr int kBB = 16;          // sequences per workgroup
constexpr int kTPW = 4;          // unit tiles per wave
constexpr int kPlanes = 3;
constexpr int kMaxHB = 512;

__device__ __forceinline__ float deq(float q, double s, double zp) {
  return static_cast<float>((static_cast<double>(q) - zp) * s);
}
__device__ __forceinline__ float keepf(const uint8_t *m, uint32_t i) {
  return m[i] == 0 ? 1.0f : 0.0f;
}

// ---------------------------------------------------------------------------------
// 1. prep
// ---------------------------------------------------------------------------------
// W_hh codes [4H][H] -> B fragments of D[b][j] = sum_c A[b][c] W[c][j]:
// frag[(jt * KS2 + s) * 64 + lane] = W[64 s + 16 (lane / 16) + 0..15][16 jt + lane % 16];
// colsum[j] = sum_c W[c][j].
__global__ __launch_bounds__(64) void lstm_pack_whh_t(int H, int KS2, const float *__restrict__ wq,
                                                      v4i *__restrict__ frag,
                                                      float *__restrict__ colsum) {
  const int lane = threadIdx.x, idx = blockIdx.x;
  const int s = idx % KS2, jt = idx / KS2;
  const int C = 4 * H, j = 16 * jt + lane % 16;
  int wd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int by[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 64 * s + 16 * (lane / 16) + 4 * q + e;
      by[e] = c < C ? static_cast<int>(wq[static_cast<size_t>(c) * H + j]) : 0;
    }
    wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
  }
  frag[static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
  if (s == 0 && lane < 16) {
    int sum = 0;
    for (int c = 0; c < C; ++c) sum += static_cast<int>(wq[static_cast<size_t>(c) * H + j]);
    colsum[j] = static_cast<float>(sum);
  }
}

// ---------------------------------------------------------------------------------
// 2. recurrence
// ---------------------------------------------------------------------------------
struct BwdArgs {
  int T, B, H, KS2, UT;
  const float *grad_out, *grad_hn, *grad_cn;   // grad_hn / grad_cn may be null
  const float *gate_out, *cell, *cell_tanh, *c0_q;
  const uint8_t *ih_m, *hh_m, *gin_m, *gout_m, *cell_m, *tanh_m, *hid_m, *h0_m, *c0_m;
  const v4i *frag;
  const float *colsum;   // [H]
  const float *s_whh;    // [4H]
  double s_gout[4], zp_gout[4], s_c, zp_c, s_t, zp_t;
  float *dli, *dlh;      // [T, B, 4H]
  float *dh0, *dc0;      // [B, H]
  // saved codes (lck_block; instead of gate_out, cell, cell_tanh and the six recurrence masks)
  // and the grid minima their offsets are taken from
  const uint8_t *ckb;
  const uint16_t *cellc;
  int32_t lo_gout[4], lo_c, lo_t;
};

// The STE backward of one (step t, sequence b, unit j) given dh and dc arriving from step t + 1
// (lstm_backward_oracle / backward_float_cpu order: output mask, tanh, cell mask, the four
// gate-output masks and activation derivatives, then the gate-input and linear masks): the
// gate-input gradients of both linears and the cell gradient passed to step t - 1.
struct LstmBwdPoint {
  float li[4], lh[4], dc_prev;
};

// The saved codes of (step t, sequence b, unit j) in the reference format: gate outputs,
// tanh(c) and the previous cell as fp32 codes, the masks as bytes (1 = clamped).
struct LstmCk {
  float go[4], ct, pc;
  uint8_t m_go[4], m_gi[4], m_hh[4], m_c, m_t, m_h;
};
__device__ __forceinline__ LstmCk lstm_ck_codes(const BwdArgs &a, int t, int b, int j) {
  LstmCk k;
  const uint8_t *blk = a.ckb + static_cast<size_t>(lck_block(t, b, j, a.B, a.H)) * kLckBlock;
  const int R = b % 16, e = j % 16;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    k.go[g] = static_cast<float>(reinterpret_cast<const uint16_t *>(blk)[(R * 4 + g) * 16 + e] +
                                 a.lo_gout[g]);
    const uint8_t m = blk[kLckGm + (g * 16 + R) * 16 + e];
    k.m_hh[g] = m & 1;
    k.m_gi[g] = (m >> 1) & 1;
    k.m_go[g] = (m >> 2) & 1;
  }
  k.ct = static_cast<float>(reinterpret_cast<const uint16_t *>(blk + kLckTanh)[R * 16 + e] + a.lo_t);
  const uint8_t m = blk[kLckCm + R * 16 + e];
  k.m_c = m & 1;
  k.m_t = (m >> 1) & 1;
  k.m_h = (m >> 2) & 1;
  k.pc = static_cast<float>(
      a.cellc[static_cast<size_t>(lck_block(t, b, j, a.B, a.H)) * kLcellBlock + R * 16 + e] + a.lo_c);
  return k;
}

__device__ __forceinline__ LstmBwdPoint lstm_bwd_point(const BwdArgs &a, int t, int b, int j,
                                                       float dh_in, float dc_in) {
  const uint32_t H = static_cast<uint32_t>(a.H), C = 4u * H, B = static_cast<uint32_t>(a.B);
  const uint32_t BH = B * H, BC = B * C;
  const uint32_t e = static_cast<uint32_t>(t) * BH + static_cast<uint32_t>(b) * H + j;
  const uint32_t gb = static_cast<uint32_t>(t) * BC + static_cast<uint32_t>(b) * C + j;
  if (a.ckb) {
    // the same arithmetic on the decoded codes
    const LstmCk k = lstm_ck_codes(a, t, b, j);
    const auto kp = [](uint8_t m) { return m == 0 ? 1.0f : 0.0f; };
    const float ig = deq(k.go[0], a.s_gout[0], a.zp_gout[0]);
    const float fg = deq(k.go[1], a.s_gout[1], a.zp_gout[1]);
    const float gg = deq(k.go[2], a.s_gout[2], a.zp_gout[2]);
    const float og = deq(k.go[3], a.s_gout[3], a.zp_gout[3]);
    const float ct = deq(k.ct, a.s_t, a.zp_t);
    const float pc = deq(k.pc, a.s_c, a.zp_c);
    const float dht = (dh_in + a.grad_out[e]) * kp(k.m_h);
    const float d_o = dht * ct;
    const float dct = dht * og * kp(k.m_t);
    const float dc = dc_in + dct * (1.0f - ct * ct);
    const float mdc = dc * kp(k.m_c);
    const float dfg = mdc * pc;
    const float dig = mdc * gg, dgg = mdc * ig;
    const float go0 = dig * kp(k.m_go[0]), go1 = dfg * kp(k.m_go[1]);
    const float go2 = dgg * kp(k.m_go[2]), go3 = d_o * kp(k.m_go[3]);
    const float gi[4] = {go0 * ig * (1.0f - ig), go1 * fg * (1.0f - fg), go2 * (1.0f - gg * gg),
                         go3 * og * (1.0f - og)};
    LstmBwdPoint o;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float grad = gi[g] * kp(k.m_gi[g]);
      o.li[g] = grad * keepf(a.ih_m, gb + g * H);
      o.lh[g] = grad * kp(k.m_hh[g]);
    }
    o.dc_prev = mdc * fg;
    return o;
  }
  const float ig = deq(a.gate_out[gb], a.s_gout[0], a.zp_gout[0]);
  const float fg = deq(a.gate_out[gb + H], a.s_gout[1], a.zp_gout[1]);
  const float gg = deq(a.gate_out[gb + 2 * H], a.s_gout[2], a.zp_gout[2]);
  const float og = deq(a.gate_out[gb + 3 * H], a.s_gout[3], a.zp_gout[3]);
  const float ct = deq(a.cell_tanh[e], a.s_t, a.zp_t);
  const float pc = t == 0 ? deq(a.c0_q[static_cast<uint32_t>(b) * H + j], a.s_c, a.zp_c)
                          : deq(a.cell[e - BH], a.s_c, a.zp_c);
  const float dht = (dh_in + a.grad_out[e]) * keepf(a.hid_m, e);
  const float d_o = dht * ct;
  const float dct = dht * og * keepf(a.tanh_m, e);
  const float dc = dc_in + dct * (1.0f - ct * ct);
  const float mdc = dc * keepf(a.cell_m, e);
  const float dfg = mdc * pc;
  const float dig = mdc * gg, dgg = mdc * ig;
  const float go0 = dig * keepf(a.gout_m, gb), go1 = dfg * keepf(a.gout_m, gb + H);
  const float go2 = dgg * keepf(a.gout_m, gb + 2 * H), go3 = d_o * keepf(a.gout_m, gb + 3 * H);
  const float gi[4] = {go0 * ig * (1.0f - ig), go1 * fg * (1.0f - fg), go2 * (1.0f - gg * gg),
                       go3 * og * (1.0f - og)};
  LstmBwdPoint o;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t gi_ = gb + g * H;
    const float grad = gi[g] * keepf(a.gin_m, gi_);
    o.li[g] = grad * keepf(a.ih_m, gi_);
    o.lh[g] = grad * keepf(a.hh_m, gi_);
  }
  o.dc_prev = mdc * fg;
  return o;
}

__global__ __launch_bounds__(512) void lstm_bwd_recurrence(BwdArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 4 * H, B = a.B;
  const int ROW = a.KS2 * 64 + 16;
  float *dcs = reinterpret_cast<float *>(smem);                              // [16][H]
  unsigned *rowmax = reinterpret_cast<unsigned *>(dcs + kBB * H);            // [16]
  int *rowexp = reinterpret_cast<int *>(rowmax + kBB);                       // [16]
  int8_t *plane = reinterpret_cast<int8_t *>(rowexp + kBB);                  // [3][16][ROW]
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int b0 = blockIdx.x * kBB, nrow0 = 4 * (l / 16);
  for (int i = tid; i < kBB * H; i += blockDim.x) {
    const int n = i / H, j = i % H, b = b0 + n;
    dcs[i] = (a.grad_cn && b < B) ? a.grad_cn[static_cast<size_t>(b) * H + j] : 0.0f;
  }
  for (int i = tid; i < kPlanes * kBB * ROW / 4; i += blockDim.x) reinterpret_cast<int *>(plane)[i] = 0;
  if (tid < kBB) rowmax[tid] = 0u;
  float dh[kTPW][4];
#pragma unroll
  for (int u = 0; u < kTPW; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ut = kTPW * w + u, j = 16 * ut + l % 16, b = b0 + nrow0 + r;
      dh[u][r] = (a.grad_hn && ut < a.UT && b < B) ? a.grad_hn[static_cast<size_t>(b) * H + j] : 0.0f;
    }
  __syncthreads();
  const uint32_t BC = static_cast<uint32_t>(B) * C;

  for (int t = a.T - 1; t >= 0; --t) {
    // ---- pointwise backward; dgates_hh * scale_W kept in registers for the dh GEMM ----
    float sv[kTPW][4][4];
#pragma unroll
    for (int u = 0; u < kTPW; ++u) {
      const int ut = kTPW * w + u;
      const int j = 16 * ut + l % 16;
      const bool tile = ut < a.UT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nr = nrow0 + r, b = b0 + nr;
#pragma unroll
        for (int g = 0; g < 4; ++g) sv[u][r][g] = 0.0f;
        if (!tile || b >= B) continue;
        const uint32_t gb = static_cast<uint32_t>(t) * BC + static_cast<uint32_t>(b) * C + j;
        float &dcr = dcs[nr * H + j];
        const LstmBwdPoint o = lstm_bwd_point(a, t, b, j, dh[u][r], dcr);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          a.dli[gb + g * H] = o.li[g];
          a.dlh[gb + g * H] = o.lh[g];
          sv[u][r][g] = o.lh[g] * a.s_whh[g * H + j];
        }
        dcr = o.dc_prev;
      }
    }
    // row maxima (NaN and inf rows propagate as NaN)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float mx = 0.0f;
#pragma unroll
      for (int u = 0; u < kTPW; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float as = fabsf(sv[u][r][g]);
          mx = (as > mx || as != as) ? as : mx;
        }
      if (!(mx <= 3.0e38f)) mx = INFINITY;
      atomicMax(&rowmax[nrow0 + r], __float_as_uint(mx));
    }
    __syncthreads();
    if (tid < kBB) {
      const float m = __uint_as_float(rowmax[tid]);
      int ex = 0;
      if (m > 0.0f && m <= 3.0e38f) frexpf(m, &ex);
      rowexp[tid] = (m > 0.0f && m <= 3.0e38f) ? 22 - ex : (m == 0.0f ? 0 : 1000);
    }
    __syncthreads();
    // ---- quantise the lane's own values into the three planes ----
#pragma unroll
    for (int u = 0; u < kTPW; ++u) {
      const int ut = kTPW * w + u;
      if (ut >= a.UT) continue;
      const int j = 16 * ut + l % 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nr = nrow0 + r, ex = rowexp[nr];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int q = 0;
          if (ex != 1000) q = static_cast<int>(rintf(ldexpf(sv[u][r][g], ex)));
          const int uq = q + (1 << 23);
          const int c = g * H + j;
          plane[(0 * kBB + nr) * ROW + c] = static_cast<int8_t>((uq & 255) - 128);
          plane[(1 * kBB + nr) * ROW + c] = static_cast<int8_t>(((uq >> 8) & 255) - 128);
          plane[(2 * kBB + nr) * ROW + c] = static_cast<int8_t>((uq >> 16) - 128);
        }
      }
    }
    __syncthreads();
    if (tid < kBB) rowmax[tid] = 0u;
    // ---- dh = W_hh_deq^T dgates_hh on MFMA ----
#pragma unroll
    for (int u = 0; u < kTPW; ++u) {
      const int ut = kTPW * w + u;
      if (ut >= a.UT) continue;
      v4i acc[kPlanes];
#pragma unroll
      for (int q = 0; q < kPlanes; ++q) acc[q] = v4i{0, 0, 0, 0};
      for (int s = 0; s < a.KS2; ++s) {
        const v4i bf = a.frag[(static_cast<uint32_t>(ut) * a.KS2 + s) * 64 + l];
#pragma unroll
        for (int q = 0; q < kPlanes; ++q) {
          const v4i afr = *reinterpret_cast<const v4i *>(plane + (q * kBB + l % 16) * ROW + 64 * s +
                                                         16 * (l / 16));
          acc[q] = mfma_i8(afr, bf, acc[q]);
        }
      }
      const double cs = static_cast<double>(a.colsum[16 * ut + l % 16]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ex = rowexp[nrow0 + r];
        const double comb = 65536.0 * acc[2][r] + 256.0 * acc[1][r] + static_cast<double>(acc[0][r]) +
                            32896.0 * cs;
        dh[u][r] = ex == 1000 ? NAN : static_cast<float>(ldexp(comb, -ex));
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < kTPW; ++u) {
    const int ut = kTPW * w + u;
    if (ut >= a.UT) continue;
    const int j = 16 * ut + l % 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nr = nrow0 + r, b = b0 + nr;
      if (b >= B) continue;
      const uint32_t o = static_cast<uint32_t>(b) * H + j;
      a.dh0[o] = dh[u][r] * keepf(a.h0_m, o);
      a.dc0[o] = dcs[nr * H + j] * keepf(a.c0_m, o);
    }
  }
}

// ---------------------------------------------------------------------------------
// 2'. stepped backward recurrence (W_hh wider than 8 bits or H above 512)
// ---------------------------------------------------------------------------------
// Per step t = T-1..0 one pointwise launch over all (sequence, unit) pairs, then the dh GEMM
// dh = (dgates_hh * scale_W) W_hh codes on bf16 MFMA (wgrad::nt: the gradient split exactly into
// three bf16 terms against exact bf16 code planes, fp32 accumulation) with a K split whose S
// parts the next pointwise adds in a fixed order.
constexpr int kBStepMaxSplit = 16;

__global__ __launch_bounds__(256) void lstm_bstep_point(BwdArgs a, int t, int S, const float *dhr,
                                                        float *dcs) {
  const int H = a.H, C = 4 * H;
  const int64_t n = static_cast<int64_t>(a.B) * H;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int b = static_cast<int>(e / H), j = static_cast<int>(e % H);
  float dh = 0.0f, dc = 0.0f;
  if (t == a.T - 1) {
    dh = a.grad_hn ? a.grad_hn[e] : 0.0f;
    dc = a.grad_cn ? a.grad_cn[e] : 0.0f;
  } else {
    for (int z = 0; z < S; ++z) dh += dhr[z * n + e];
    dc = dcs[e];
  }
  const LstmBwdPoint o = lstm_bwd_point(a, t, b, j, dh, dc);
  const size_t gb = (static_cast<size_t>(t) * a.B + b) * C + j;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    a.dli[gb + g * H] = o.li[g];
    a.dlh[gb + g * H] = o.lh[g];
  }
  dcs[e] = o.dc_prev;
}

// dh0 / dc0 after the last step, with the h0 / c0 master masks.
__global__ __launch_bounds__(256) void lstm_bstep_finish(BwdArgs a, int S, const float *dhr,
                                                         const float *dcs) {
  const int64_t n = static_cast<int64_t>(a.B) * a.H;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= n) return;
  float dh = 0.0f;
  for (int z = 0; z < S; ++z) dh += dhr[z * n + e];
  a.dh0[e] = dh * keepf(a.h0_m, static_cast<uint32_t>(e));
  a.dc0[e] = dcs[e] * keepf(a.c0_m, static_cast<uint32_t>(e));
}

// ---------------------------------------------------------------------------------
// 2b. clustered backward recurrence
// ---------------------------------------------------------------------------------
// Member m of a cluster owns 64 units (four 16-unit tiles) of one 16-sequence batch tile for
// all four gates: 256 channels.  Per step each lane finishes the STE pointwise of two
// (sequence, unit) pairs, the member writes dgates_hh * scale_W of its channels as 22-bit
// block fixed point with one exponent per sequence (three int8 planes) to a global exchange
// buffer, and after the cluster barrier dh = W_hh_deq^T dgates_hh of its units is summed on
// v_mfma_i32_16x16x64_i8.  The contraction's K-steps (64 channels each, member-major) are
// dealt to the eight waves in contiguous runs: each wave loads its own A fragments straight
// from the exchange buffer into VGPRs (every exchanged byte is read by one wave, with no LDS
// staging), multiplies them against the W_hh codes of all four unit tiles of the member (held
// in VGPRs), recombines the exact plane sums of each member segment in double scaled by that
// member's exponent, and the eight waves' partials are added in wave (K) order through LDS.
constexpr int kBcUnits = 64;
constexpr int kBcMaxKs = 4;  // K-steps per wave at most: 4H / 64 / 8 with H <= 512

struct BwdClArgs {
  int ncl, G, ntiles, Bpad;
  int8_t *xp;          // [2][3][ntiles][KS2][16][64] planes of the exchanged dgates, one 1 KB
                       // block per (parity, plane, batch tile, K-step), see xblock
  int *xe;             // [2][Bpad][G] exponents
  const v4i *wfrag;    // W_hh^T fragments in member-major K order, see lstm_pack_whh_t_cl
  const float *csum;   // [KS2][H] column sums of W_hh codes over each K-step's 64 channels
  unsigned *counters;
  int *timeout;
  unsigned spin_limit;  // polls before a wait gives up (cluster::spin_limit())
};

// Byte offset of the exchange buffer's block for (parity, plane, batch tile, K-step): the tile's
// 16 rows x 64 channels of the step, row-major.  A wave reads a block as one MFMA A fragment
// with a contiguous 16-byte load per lane (lane L: row L % 16, channels 16 (L / 16) .. + 15).
__device__ __forceinline__ unsigned xblock(int par, int p, int tile, int ntiles, int KS2, int ks) {
  return (static_cast<unsigned>((par * 3 + p) * ntiles + tile) * KS2 + ks) * 1024;
}

// A position k of the member-major contraction order -> channel c: member m's 256 channels,
// unit-major with the four gates of a unit adjacent (so a lane packs its four gate bytes into
// one word of each plane).
__device__ __forceinline__ int cl_channel(int k, int H) {
  const int m = k / 256, u = (k % 256) / 4, g = k % 4;
  return g * H + 64 * m + u;
}

// frag[(jt * KS2 + s) * 64 + lane] = W[cl_channel(64 s + 16 (lane / 16) + e)][16 jt + lane % 16];
// csum[s][j] = sum over K-step s's channels c of W[c][j].
__global__ __launch_bounds__(64) void lstm_pack_whh_t_cl(int H, int KS2, const float *__restrict__ wq,
                                                         v4i *__restrict__ frag,
                                                         float *__restrict__ csum) {
  const int lane = threadIdx.x, idx = blockIdx.x;
  const int s = idx % KS2, jt = idx / KS2;
  const int j = 16 * jt + lane % 16;
  int wd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int by[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = cl_channel(64 * s + 16 * (lane / 16) + 4 * q + e, H);
      by[e] = static_cast<int>(wq[static_cast<size_t>(c) * H + j]);
    }
    wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
  }
  frag[static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
  if (lane < 16) {
    int sum = 0;
    for (int k = 64 * s; k < 64 * s + 64; ++k)
      sum += static_cast<int>(wq[static_cast<size_t>(cl_channel(k, H)) * H + j]);
    csum[static_cast<size_t>(s) * H + j] = static_cast<float>(sum);
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// The checkpoint block of one step for a member's 64 units of a 16-row batch tile, as copied
// into LDS (16-byte chunks; rows past B repeat row B - 1 and are not used):
//   gate_out  floats [16 rows][4 gates][64]      chunks    0..1023
//   masks     bytes  [4 kinds][16][4 gates][64]  chunks 1024..2047 (gate_out, gate_in, ih, hh)
//   values    floats [3][16][64]                 chunks 2048..2815 (cell_tanh, c_prev, grad_out)
//   masks     bytes  [3][16][64]                 chunks 2816..3007 (hidden, cell_tanh, cell)
constexpr int kCkInst = 47;  // 1 KB copies
constexpr int kCkBytes = kCkInst * 1024;
constexpr int kCkMaskOff = 1024 * 16, kCkValOff = 2048 * 16, kCkBitOff = 2816 * 16;

// Start the copies of step t's checkpoint block into ck: one 1 KB LDS-DMA instruction per wave
// and 64 chunks, dealt to waves 1-7 (wave 0 polls the cluster counter and keeps no loads of its
// own outstanding).  Each instruction lies in one segment, so every branch is wave-uniform.
__device__ __forceinline__ void ck_issue(const BwdArgs &a, int t, int b0, int u0, unsigned char *ck,
                                         int w, int l) {
  if (w == 0) return;
  const int H = a.H, C = 4 * H;
  const uint32_t BH = static_cast<uint32_t>(a.B) * H, BC = static_cast<uint32_t>(a.B) * C;
  for (int k = w - 1; k < kCkInst; k += 7) {
    const int q = k * 64 + l;
    const void *src;
    if (k < 16) {
      const int R = q / 64, g = (q / 16) % 4, c = q % 16, b = min(b0 + R, a.B - 1);
      src = a.gate_out + (static_cast<uint32_t>(t) * BC + static_cast<uint32_t>(b) * C + g * H + u0 + 4 * c);
    } else if (k < 32) {
      const int q2 = q - 1024, kind = q2 / 256, R = (q2 / 16) % 16, g = (q2 / 4) % 4, c = q2 % 4;
      const int b = min(b0 + R, a.B - 1);
      const uint8_t *m = kind == 0 ? a.gout_m : kind == 1 ? a.gin_m : kind == 2 ? a.ih_m : a.hh_m;
      src = m + (static_cast<uint32_t>(t) * BC + static_cast<uint32_t>(b) * C + g * H + u0 + 16 * c);
    } else if (k < 44) {
      const int q3 = q - 2048, kind = q3 / 256, R = (q3 / 16) % 16, c = q3 % 16;
      const uint32_t row = static_cast<uint32_t>(min(b0 + R, a.B - 1)) * H + u0 + 4 * c;
      src = kind == 0 ? a.cell_tanh + (static_cast<uint32_t>(t) * BH + row)
            : kind == 2 ? a.grad_out + (static_cast<uint32_t>(t) * BH + row)
            : t == 0 ? a.c0_q + row
                     : a.cell + (static_cast<uint32_t>(t - 1) * BH + row);
    } else {
      const int q4 = q - 2816, kind = q4 / 64, R = (q4 / 4) % 16, c = q4 % 4;
      const uint32_t row = static_cast<uint32_t>(min(b0 + R, a.B - 1)) * H + u0 + 16 * c;
      const uint8_t *m = kind == 0 ? a.hid_m : kind == 1 ? a.tanh_m : a.cell_m;
      src = m + (static_cast<uint32_t>(t) * BH + row);
    }
    __builtin_amdgcn_global_load_lds(src, (lds_void *)(ck + 1024 * k), 16, 0, 0);
  }
}

// With saved codes the step's block in LDS is instead (16-byte chunks):
//   the member's four code blocks  bytes 0..15359      chunks    0..959  (lck_block layout)
//   its four cell blocks of step t bytes 15360..17407  chunks  960..1087 (the previous cell)
//   grad_out floats [16 rows][64]  bytes 17408..21503  chunks 1088..1343
//   ih masks bytes [16][4 gates][64] bytes 21504..25599 chunks 1344..1599
constexpr int kCkcInst = 25;
constexpr int kCkcCell = 15360, kCkcGrad = 17408, kCkcIh = 21504;

__device__ __forceinline__ void ck_issue_codes(const BwdArgs &a, int t, int tile, int b0, int u0,
                                               unsigned char *ck, int w, int l) {
  if (w == 0) return;
  const int H = a.H, C = 4 * H;
  const uint32_t BH = static_cast<uint32_t>(a.B) * H, BC = static_cast<uint32_t>(a.B) * C;
  const size_t nt = static_cast<size_t>(a.B + 15) / 16;
  const size_t blk0 = (static_cast<size_t>(t) * nt + tile) * (H / 16) + u0 / 16;
  for (int k = w - 1; k < kCkcInst; k += 7) {
    const int q = k * 64 + l;
    const void *src;
    if (k < 15) {
      src = a.ckb + blk0 * kLckBlock + 16 * q;
    } else if (k < 17) {
      src = reinterpret_cast<const unsigned char *>(a.cellc + blk0 * kLcellBlock) + 16 * (q - 960);
    } else if (k < 21) {
      const int q3 = q - 1088, R = q3 / 16, c = q3 % 16;
      const uint32_t row = static_cast<uint32_t>(min(b0 + R, a.B - 1)) * H + u0 + 4 * c;
      src = a.grad_out + (static_cast<uint32_t>(t) * BH + row);
    } else {
      const int q4 = q - 1344, R = q4 / 16, g = (q4 / 4) % 4, c = q4 % 4;
      const int b = min(b0 + R, a.B - 1);
      src = a.ih_m + (static_cast<uint32_t>(t) * BC + static_cast<uint32_t>(b) * C + g * H + u0 + 16 * c);
    }
    __builtin_amdgcn_global_load_lds(src, (lds_void *)(ck + 1024 * k), 16, 0, 0);
  }
}

template <bool CK>
__global__ __launch_bounds__(512) void lstm_bwd_recurrence_cl(BwdArgs a, BwdClArgs cl) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 4 * H, B = a.B, KS2 = a.KS2, G = cl.G;
  // every wave's partial dh: [8 waves][4 unit tiles][64 lanes][4 rows]
  double *pd = reinterpret_cast<double *>(smem);
  unsigned *rowmax = reinterpret_cast<unsigned *>(pd + 8 * 4 * 64 * 4);  // [16]
  int *rowexp = reinterpret_cast<int *>(rowmax + kBB);                  // [16]
  // the step's gate gradients of the member's units, [16 rows][8][64]: dli gates 0-3, dlh 4-7
  float *sdl = reinterpret_cast<float *>(rowexp + kBB);
  // the step's checkpoint block (ck_issue)
  unsigned char *ck = reinterpret_cast<unsigned char *>(sdl + kBB * 8 * kBcUnits);
  const float *ckf = reinterpret_cast<const float *>(ck);
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int utl = w & 3, kh = w >> 2;
  const cluster::Place pl = cluster::place(G, cl.ncl);
  const int m0 = pl.member;
  const int jt = m0 * 4 + utl;  // global unit tile
  const int j = 16 * jt + l % 16;
  const int nrow0 = 4 * (l / 16);
  if (tid < kBB) rowmax[tid] = 0u;
  float sw[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) sw[g] = a.s_whh[g * H + j];
  // the wave's K-steps [ks0, ks0 + nks) (KS2 = 4G with G even, so nks = KS2 / 8 is whole); they
  // belong to member mA, and to mB too when the run crosses a member boundary (G = 6)
  const int nks = KS2 / 8, ks0 = w * nks;
  const int mA = ks0 / 4, mB = (ks0 + nks - 1) / 4;
  // W_hh^T operands of the member's four unit tiles over those K-steps stay in VGPRs
  v4i wr[4][kBcMaxKs];
#pragma unroll
  for (int ut = 0; ut < 4; ++ut)
#pragma unroll
    for (int i = 0; i < kBcMaxKs; ++i)
      wr[ut][i] = i < nks ? cl.wfrag[((static_cast<size_t>(4 * m0 + ut)) * KS2 + ks0 + i) * 64 + l]
                          : v4i{0, 0, 0, 0};
  // column sums of the W_hh codes over each member segment's channels (integers, exact in
  // float); the segment's plane sums carry 32896 times this as their zero-point term
  float zc[2][4];
#pragma unroll
  for (int ut = 0; ut < 4; ++ut) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < kBcMaxKs; ++i) {
      if (i >= nks) continue;
      const float v = cl.csum[static_cast<size_t>(ks0 + i) * H + 64 * m0 + 16 * ut + l % 16];
      if ((ks0 + i) / 4 == mA) s0 += v;
      else s1 += v;
    }
    zc[0][ut] = s0;
    zc[1][ut] = s1;
  }
  unsigned *counter = cl.counters + cluster::kCounterStride * pl.cluster;
  unsigned epoch = 0;
  bool alive = true;
  const uint32_t BC = static_cast<uint32_t>(B) * C;
  const auto xr = cluster::buffer_rsrc(cl.xp, 6u * cl.ntiles * KS2 * 1024);
  __syncthreads();

  for (int tile = pl.cluster; tile < cl.ntiles && alive; tile += cl.ncl) {
    const int b0 = tile * kBB;
    if constexpr (CK)
      ck_issue_codes(a, a.T - 1, tile, b0, kBcUnits * m0, ck, w, l);
    else
      ck_issue(a, a.T - 1, b0, kBcUnits * m0, ck, w, l);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float dh[2], dc[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int b = b0 + nrow0 + 2 * kh + rr;
      dh[rr] = (a.grad_hn && b < B) ? a.grad_hn[static_cast<size_t>(b) * H + j] : 0.0f;
      dc[rr] = (a.grad_cn && b < B) ? a.grad_cn[static_cast<size_t>(b) * H + j] : 0.0f;
    }
    for (int t = a.T - 1; t >= 0 && alive; --t) {
      const int par = t & 1;
      float sv[2][4], lis[2][4], lhs[2][4];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int b = b0 + nrow0 + 2 * kh + rr;
#pragma unroll
        for (int g = 0; g < 4; ++g) sv[rr][g] = lis[rr][g] = lhs[rr][g] = 0.0f;
        if (b >= B) continue;
        // the row's checkpoint values and masks from the step's block in LDS
        const int R = nrow0 + 2 * kh + rr, uu = 16 * utl + l % 16;
        float r_go[4], r_ct, r_pc, r_gd;
        uint8_t r_hid, r_tanh, r_cell, r_gm[4], r_gin[4], r_ih[4], r_hh[4];
        if constexpr (CK) {
          // codes: block utl of the member, e = l % 16
          const unsigned char *bk = ck + utl * kLckBlock;
          const int e = l % 16;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            r_go[g] = static_cast<float>(
                reinterpret_cast<const uint16_t *>(bk)[(R * 4 + g) * 16 + e] + a.lo_gout[g]);
            const uint8_t m = bk[kLckGm + (g * 16 + R) * 16 + e];
            r_hh[g] = m & 1;
            r_gin[g] = (m >> 1) & 1;
            r_gm[g] = (m >> 2) & 1;
            r_ih[g] = ck[kCkcIh + (R * 4 + g) * 64 + uu];
          }
          r_ct = static_cast<float>(reinterpret_cast<const uint16_t *>(bk + kLckTanh)[R * 16 + e] + a.lo_t);
          r_pc = static_cast<float>(
              reinterpret_cast<const uint16_t *>(ck + kCkcCell + utl * 2 * kLcellBlock)[R * 16 + e] + a.lo_c);
          r_gd = ckf[kCkcGrad / 4 + R * 64 + uu];
          const uint8_t m = bk[kLckCm + R * 16 + e];
          r_cell = m & 1;
          r_tanh = (m >> 1) & 1;
          r_hid = (m >> 2) & 1;
        } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          r_go[g] = ckf[(R * 4 + g) * 64 + uu];
          r_gm[g] = ck[kCkMaskOff + ((0 * 16 + R) * 4 + g) * 64 + uu];
          r_gin[g] = ck[kCkMaskOff + ((1 * 16 + R) * 4 + g) * 64 + uu];
          r_ih[g] = ck[kCkMaskOff + ((2 * 16 + R) * 4 + g) * 64 + uu];
          r_hh[g] = ck[kCkMaskOff + ((3 * 16 + R) * 4 + g) * 64 + uu];
        }
        r_ct = ckf[kCkValOff / 4 + (0 * 16 + R) * 64 + uu];
        r_pc = ckf[kCkValOff / 4 + (1 * 16 + R) * 64 + uu];
        r_gd = ckf[kCkValOff / 4 + (2 * 16 + R) * 64 + uu];
        r_hid = ck[kCkBitOff + (0 * 16 + R) * 64 + uu];
        r_tanh = ck[kCkBitOff + (1 * 16 + R) * 64 + uu];
        r_cell = ck[kCkBitOff + (2 * 16 + R) * 64 + uu];
        }
        const auto kp = [](uint8_t m) { return m == 0 ? 1.0f : 0.0f; };
        const float ig = deq(r_go[0], a.s_gout[0], a.zp_gout[0]);
        const float fg = deq(r_go[1], a.s_gout[1], a.zp_gout[1]);
        const float gg = deq(r_go[2], a.s_gout[2], a.zp_gout[2]);
        const float og = deq(r_go[3], a.s_gout[3], a.zp_gout[3]);
        const float ct = deq(r_ct, a.s_t, a.zp_t);
        const float pc = deq(r_pc, a.s_c, a.zp_c);
        const float dht = (dh[rr] + r_gd) * kp(r_hid);
        const float d_o = dht * ct;
        const float dct = dht * og * kp(r_tanh);
        const float dcv = dc[rr] + dct * (1.0f - ct * ct);
        const float mdc = dcv * kp(r_cell);
        const float dfg = mdc * pc;
        const float dig = mdc * gg, dgg = mdc * ig;
        const float go0 = dig * kp(r_gm[0]), go1 = dfg * kp(r_gm[1]);
        const float go2 = dgg * kp(r_gm[2]), go3 = d_o * kp(r_gm[3]);
        const float gi[4] = {go0 * ig * (1.0f - ig), go1 * fg * (1.0f - fg), go2 * (1.0f - gg * gg),
                             go3 * og * (1.0f - og)};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float grad = gi[g] * kp(r_gin[g]);
          lis[rr][g] = grad * kp(r_ih[g]);
          lhs[rr][g] = grad * kp(r_hh[g]);
          sv[rr][g] = lhs[rr][g] * sw[g];
        }
        dc[rr] = mdc * fg;
      }
      // stage the gate gradients for the stores after the arrival
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        float *d = sdl + (nrow0 + 2 * kh + rr) * 8 * kBcUnits + 16 * utl + l % 16;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          d[g * kBcUnits] = lis[rr][g];
          d[(4 + g) * kBcUnits] = lhs[rr][g];
        }
      }
      // per-sequence exponent of this member's channels (NaN and inf rows propagate as NaN)
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        float mx = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float as = fabsf(sv[rr][g]);
          mx = (as > mx || as != as) ? as : mx;
        }
        if (!(mx <= 3.0e38f)) mx = INFINITY;
        // the 16 lanes of a row first (the bits of non-negative floats order as the values),
        // then one LDS atomic per wave and row
        unsigned u = __float_as_uint(mx);
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) u = max(u, static_cast<unsigned>(__shfl_xor(static_cast<int>(u), o, 64)));
        if (l % 16 == 0) atomicMax(&rowmax[nrow0 + 2 * kh + rr], u);
      }
      __syncthreads();
      if (tid < kBB) {
        const float mv = __uint_as_float(rowmax[tid]);
        int ex = 0;
        if (mv > 0.0f && mv <= 3.0e38f) frexpf(mv, &ex);
        const int re = (mv > 0.0f && mv <= 3.0e38f) ? 22 - ex : (mv == 0.0f ? 0 : 1000);
        rowexp[tid] = re;
        rowmax[tid] = 0u;
        cluster::store_coherent(
            reinterpret_cast<unsigned *>(cl.xe + (static_cast<size_t>(par) * cl.Bpad + b0 + tid) * G + m0),
            static_cast<unsigned>(re));
      }
      __syncthreads();
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int nr = nrow0 + 2 * kh + rr;
        const int ex = rowexp[nr];
        unsigned wd[3] = {0u, 0u, 0u};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int q = 0;
          if (ex != 1000) q = static_cast<int>(rintf(ldexpf(sv[rr][g], ex)));
          const int uq = q + (1 << 23);
          wd[0] |= static_cast<unsigned>(((uq & 255) - 128) & 255) << (8 * g);
          wd[1] |= static_cast<unsigned>((((uq >> 8) & 255) - 128) & 255) << (8 * g);
          wd[2] |= static_cast<unsigned>(((uq >> 16) - 128) & 255) << (8 * g);
        }
        // channels 256 m0 + 4 (16 utl + l % 16) + 0..3: K-step 4 m0 + utl, channel 4 (l % 16)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          cluster::store_coherent(
              reinterpret_cast<unsigned *>(cl.xp + xblock(par, p, tile, cl.ntiles, KS2, 4 * m0 + utl) +
                                           64 * nr + 4 * (l % 16)),
              wd[p]);
      }
      // the other members only read the planes and exponents: arrive (which also publishes the
      // staged gate gradients), then store them for the weight GEMMs as 16-byte rows while
      // waiting
      cluster::arrive(counter);
      ++epoch;
      // the next step's checkpoint block (the block of this step was read before the exponent
      // barriers above); complete before the partial-sum barrier below
      if (t > 0) {
        if constexpr (CK)
          ck_issue_codes(a, t - 1, tile, b0, kBcUnits * m0, ck, w, l);
        else
          ck_issue(a, t - 1, b0, kBcUnits * m0, ck, w, l);
      }
      {
        const size_t tb = static_cast<size_t>(t) * BC;
        const int u0 = kBcUnits * m0;
        for (int c = tid; c < kBB * 4 * 16; c += blockDim.x) {
          const int row = c / 64, g = (c / 16) % 4, q = c % 16, b = b0 + row;
          if (b < B)
            *reinterpret_cast<float4 *>(a.dli + tb + static_cast<size_t>(b) * C + g * H + u0 + 4 * q) =
                *reinterpret_cast<const float4 *>(sdl + (row * 8 + g) * kBcUnits + 4 * q);
        }
        for (int c = tid; c < kBB * 4 * 16; c += blockDim.x) {
          const int row = c / 64, g = (c / 16) % 4, q = c % 16, b = b0 + row;
          if (b < B)
            *reinterpret_cast<float4 *>(a.dlh + tb + static_cast<size_t>(b) * C + g * H + u0 + 4 * q) =
                *reinterpret_cast<const float4 *>(sdl + (row * 8 + 4 + g) * kBcUnits + 4 * q);
        }
      }
      alive = cluster::wait(counter, epoch * G, cl.timeout, cl.spin_limit);
      if (!alive) break;
      // dh partial of the wave's K-steps for the member's 64 units: A fragments (row l % 16,
      // channels 64 ks + 16 (l / 16) + 0..15 of each plane) and the rows' exponents loaded
      // together, then the MFMAs, one member segment at a time
      {
        int4 av[kBcMaxKs][3];
#pragma unroll
        for (int i = 0; i < kBcMaxKs; ++i)
#pragma unroll
          for (int p = 0; p < 3; ++p)
            av[i][p] = cluster::load_coherent16(
                xr, xblock(par, p, tile, cl.ntiles, KS2, ks0 + (i < nks ? i : 0)) + 64 * (l % 16) + 16 * (l / 16));
        const unsigned *xe =
            reinterpret_cast<const unsigned *>(cl.xe) + (static_cast<size_t>(par) * cl.Bpad + b0 + nrow0) * G;
        int exA[4], exB[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          exA[r] = static_cast<int>(__hip_atomic_load(xe + r * G + mA, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          exB[r] = static_cast<int>(__hip_atomic_load(xe + r * G + mB, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
        // one unit tile at a time (its three plane sums in 12 VGPRs), K-steps in order
#pragma unroll
        for (int ut = 0; ut < 4; ++ut) {
          double *d = pd + ((static_cast<size_t>(w) * 4 + ut) * 64 + l) * 4;
          v4i acc[3] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
          for (int i = 0; i < kBcMaxKs; ++i) {
            if (i >= nks) continue;
#pragma unroll
            for (int p = 0; p < 3; ++p)
              acc[p] = mfma_i8(v4i{av[i][p].x, av[i][p].y, av[i][p].z, av[i][p].w}, wr[ut][i], acc[p]);
            const int ks = ks0 + i;
            if (i == nks - 1 || (ks & 3) == 3) {
              // the end of a member segment: its exact sums scaled by the member's exponent go
              // to the wave's partial (written by the first segment, the member mA; added to by
              // the second)
              const bool sa = ks / 4 == mA;
              const double z = 32896.0 * static_cast<double>(sa ? zc[0][ut] : zc[1][ut]);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int ex = sa ? exA[r] : exB[r];
                const double comb = 65536.0 * acc[2][r] + 256.0 * acc[1][r] +
                                    static_cast<double>(acc[0][r]) + z;
                const double v = ex == 1000 ? static_cast<double>(NAN) : ldexp(comb, -ex);
                d[r] = sa ? v : d[r] + v;
              }
#pragma unroll
              for (int p = 0; p < 3; ++p) acc[p] = v4i{0, 0, 0, 0};
            }
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's checkpoint copies are in LDS
      __syncthreads();
      // each (unit, row) pair of the lane: the eight partials in wave (K) order
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * kh + rr;
        double sum = 0.0;
#pragma unroll
        for (int w2 = 0; w2 < 8; ++w2) sum += pd[((static_cast<size_t>(w2) * 4 + utl) * 64 + l) * 4 + r];
        dh[rr] = static_cast<float>(sum);
      }
    }
    if (!alive) break;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int b = b0 + nrow0 + 2 * kh + rr;
      if (b >= B) continue;
      const uint32_t o = static_cast<uint32_t>(b) * H + j;
      a.dh0[o] = dh[rr] * keepf(a.h0_m, o);
      a.dc0[o] = dc[rr] * keepf(a.c0_m, o);
    }
  }
}

size_t bwd_cl_lds() {
  return sizeof(double) * 8 * 4 * 64 * 4 + 2 * sizeof(int) * kBB + sizeof(float) * kBB * 8 * kBcUnits +
         kCkBytes;
}

size_t bwd_lds(int H, int KS2) {
  return sizeof(float) * kBB * static_cast<size_t>(H) + 2 * sizeof(int) * kBB +
         static_cast<size_t>(kPlanes) * kBB * (KS2 * 64 + 16);
}

// dx *= keep(x_m); dW = aug[:, :K] * keep(W_m); db = aug[:, K] * keep(b_m) (when bias).
__global__ __launch_bounds__(256) void lstm_bwd_finish(int64_t nx, float *dx, const uint8_t *xm,
                                                       int C, int I, int H, const float *aug_ih,
                                                       const float *aug_hh, float *dwi, float *dwh,
                                                       float *dbi, float *dbh, const uint8_t *wim,
                                                       const uint8_t *whm, const uint8_t *bim,
                                                       const uint8_t *bhm) {
  const int64_t n1 = static_cast<int64_t>(C) * I, n2 = static_cast<int64_t>(C) * H;
  const int64_t total = nx + n1 + n2 + C;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    if (i < nx) {
      if (xm[i]) dx[i] = 0.0f;
    } else if (i < nx + n1) {
      const int64_t e = i - nx, c = e / I, k = e % I;
      dwi[e] = wim[e] ? 0.0f : aug_ih[c * (I + 1) + k];
    } else if (i < nx + n1 + n2) {
      const int64_t e = i - nx - n1, c = e / H, k = e % H;
      dwh[e] = whm[e] ? 0.0f : aug_hh[c * (H + 1) + k];
    } else {
      const int64_t c = i - nx - n1 - n2;
      if (dbi) dbi[c] = bim[c] ? 0.0f : aug_ih[c * (I + 1) + I];
      if (dbh) dbh[c] = bhm[c] ? 0.0f : aug_hh[c * (H + 1) + H];
    }
  }
}

struct BwdWorkspace {
  size_t dli, dlh, xt, wt, ht, qsc, frag, colsum, swih, swhh, aug_ih, aug_hh, part, gsum, wfrag_cl,
      csum, xp, xe, sync, dhr, dcs, whht, total;
  int Mp, S_ih[2], kper_ih[2], S_hh[2], kper_hh[2];  // K splits by number of B planes
  BwdWorkspace(int T, int B, int I, int H) {
    const size_t C = 4 * static_cast<size_t>(H), M = static_cast<size_t>(T) * B;
    const size_t KS2 = (C + 63) / 64;
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t o = 0;
    dli = o; o += al(sizeof(float) * M * C);
    dlh = o; o += al(sizeof(float) * M * C);
    // weight-gradient GEMM operands: codes as bf16 planes, transposed, rows padded to Mp
    Mp = static_cast<int>((M + 31) / 32 * 32);
    xt = o; o += al(sizeof(__bf16) * 2 * I * static_cast<size_t>(Mp));
    wt = o; o += al(sizeof(__bf16) * 2 * I * C);
    ht = o; o += al(sizeof(__bf16) * 2 * H * static_cast<size_t>(Mp));
    qsc = o; o += al(sizeof(float) * (I + H));
    frag = o; o += al(sizeof(v4i) * 64 * (H / 16 + 1) * KS2);
    colsum = o; o += al(sizeof(float) * H);
    swih = o; o += al(sizeof(float) * C);
    swhh = o; o += al(sizeof(float) * C);
    aug_ih = o; o += al(sizeof(float) * C * (I + 1));
    aug_hh = o; o += al(sizeof(float) * C * (H + 1));
    for (int np = 0; np < 2; ++np)
      wgrad::tn_plan(static_cast<int>(M), static_cast<int>(C), I, np + 1, &S_ih[np], &kper_ih[np]);
    for (int np = 0; np < 2; ++np)
      wgrad::tn_plan(static_cast<int>(M), static_cast<int>(C), H, np + 1, &S_hh[np], &kper_hh[np]);
    const size_t sih = std::max(S_ih[0], S_ih[1]), shh = std::max(S_hh[0], S_hh[1]);
    const size_t np = std::max(sih * C * I, shh * C * H);
    part = o; o += al(sizeof(float) * np);
    gsum = o; o += al(sizeof(float) * 4 * C * std::max(sih, shh));
    // clustered recurrence (H a multiple of 64)
    const size_t Bpad = (static_cast<size_t>(B) + kBB - 1) / kBB * kBB, G = H / kBcUnits + 1;
    wfrag_cl = o; o += al(sizeof(v4i) * 64 * (H / 16) * KS2);
    csum = o; o += al(sizeof(float) * KS2 * H);
    xp = o; o += al(2 * 3 * Bpad * C);
    xe = o; o += al(sizeof(int) * 2 * Bpad * G);
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (Bpad / kBB + 1));
    // stepped recurrence: K-split parts of dh, the cell gradient, W_hh codes as bf16 planes
    dhr = o; o += al(sizeof(float) * kBStepMaxSplit * static_cast<size_t>(B) * H);
    dcs = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    whht = o; o += al(sizeof(__bf16) * 2 * static_cast<size_t>(H) * C);
    total = o;
  }
};

}  // namespace lstm
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::lstm;

extern "C" {

int64_t rxmet_lstm_backward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  if (T < 1 || B < 1 || I < 1 || H < 1) return 0;
  return static_cast<int64_t>(BwdWorkspace(T, B, I, H).total);
}

static int lstm_backward_impl(int32_t T, int32_t B, int32_t I, int32_t H,
                              const rxmet_lstm_params *params, const rxmet_lstm_saved *saved,
                              const rxmet_lstm_saved_codes *codes,
                              const float *grad_output, const float *grad_h_n,
                              const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                              float *db_ih, float *db_hh, float *dh0, float *dc0,
                              void *workspace, void *stream_) {
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H % 16 == 0, "hidden_size must be a multiple of 16");
  RXMET_CHECK_ARG(params && saved && grad_output && dx && dW_ih && dW_hh && dh0 && dc0 && workspace,
                  "required pointer is null");
  RXMET_CHECK_ARG(params->hidden == H, "params hidden size does not match");
  const bool bias = params->bias_enabled != 0;
  RXMET_CHECK_ARG(!bias || (db_ih && db_hh), "bias gradients requested but pointers are null");
  const rxmet_lstm_saved &sv = *saved;
  if (codes)
    RXMET_CHECK_ARG(sv.x_q && sv.w_ih_q && sv.w_hh_q && sv.h0_q && sv.c0_q && sv.x_m &&
                        sv.w_ih_m && sv.w_hh_m && sv.h0_m && sv.c0_m && sv.hidden &&
                        sv.ih_linear_m && codes->blocks && codes->cell_codes,
                    "backward needs the masters, hidden, ih_linear_m and the saved codes");
  else
    RXMET_CHECK_ARG(sv.x_q && sv.w_ih_q && sv.w_hh_q && sv.h0_q && sv.c0_q && sv.x_m &&
                        sv.w_ih_m && sv.w_hh_m && sv.h0_m && sv.c0_m && sv.gate_out && sv.cell &&
                        sv.cell_tanh && sv.hidden && sv.ih_linear_m && sv.hh_linear_m &&
                        sv.gate_in_m && sv.gate_out_m && sv.cell_m && sv.cell_tanh_m &&
                        sv.hidden_m,
                    "backward needs every saved tensor");
  RXMET_CHECK_ARG(!bias || (sv.b_ih_m && sv.b_hh_m), "backward with bias needs the bias masks");
  const Grid gwh_b = grid_of(params->config.op[RXMET_LSTM_W_HH], 1.0f, 0);
  RXMET_CHECK_ARG(gwh_b.lo >= -32768 && gwh_b.hi <= 32767, "W_hh codes must fit signed 16 bits");
  // the MFMA recurrences hold W_hh as int8 fragments for at most 512 units: anything else steps
  const bool stepped = gwh_b.lo < -128 || gwh_b.hi > 127 || H > kMaxHB ||
                       std::getenv("RXMET_LSTM_STEPPED") != nullptr;
  RXMET_CHECK_ARG(static_cast<double>(T) * B * 4 * H < 4294967295.0,
                  "T*B*4H too large for 32-bit element offsets");
  StepParams sp;
  ChannelParams cp;
  if (int rc = derive(*params, &sp, &cp)) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int C = 4 * H, KS2 = (C + 63) / 64, UT = H / 16, M = T * B;
  const BwdWorkspace ws(T, B, I, H);
  char *wsb = static_cast<char *>(workspace);
  float *dli = reinterpret_cast<float *>(wsb + ws.dli);
  float *dlh = reinterpret_cast<float *>(wsb + ws.dlh);
  __bf16 *xt = reinterpret_cast<__bf16 *>(wsb + ws.xt);
  __bf16 *wt = reinterpret_cast<__bf16 *>(wsb + ws.wt);
  __bf16 *ht = reinterpret_cast<__bf16 *>(wsb + ws.ht);
  float *qsc = reinterpret_cast<float *>(wsb + ws.qsc);
  float *gsum = reinterpret_cast<float *>(wsb + ws.gsum);
  v4i *frag = reinterpret_cast<v4i *>(wsb + ws.frag);
  float *colsum = reinterpret_cast<float *>(wsb + ws.colsum);
  float *swih = reinterpret_cast<float *>(wsb + ws.swih);
  float *swhh = reinterpret_cast<float *>(wsb + ws.swhh);
  float *aug_ih = reinterpret_cast<float *>(wsb + ws.aug_ih);
  float *aug_hh = reinterpret_cast<float *>(wsb + ws.aug_hh);
  float *part = reinterpret_cast<float *>(wsb + ws.part);
  std::vector<float> host(2 * C);
  for (int c = 0; c < C; ++c) {
    host[c] = cp.w_ih_scale[c];
    host[C + c] = cp.w_hh_scale[c];
  }
  RXMET_CHECK_HIP(hipMemcpyAsync(swih, host.data(), sizeof(float) * 2 * C, hipMemcpyHostToDevice,
                                 stream));

  // weight-gradient operands: x, h_prev and W_ih codes as bf16 planes, transposed
  const Grid gwi = grid_of(params->config.op[RXMET_LSTM_W_IH], 1.0f, 0);
  const int npx = wgrad::planes_for(sp.x.lo, sp.x.hi, sp.x.zp);
  const int nph = wgrad::planes_for(sp.h.lo, sp.h.hi, sp.h.zp);
  const int npw = wgrad::planes_for(gwi.lo, gwi.hi, 0.0);
  const int64_t Mp = ws.Mp;
  if (int rc = wgrad::codes_t(sv.x_q, M, nullptr, M, I, I, 1, static_cast<float>(sp.x.zp), 1.0f, npx, xt, Mp,
                              static_cast<int64_t>(I) * Mp, stream))
    return rc;
  if (int rc = wgrad::codes_t(sv.h0_q, B, sv.hidden, M, H, H, 1, static_cast<float>(sp.h.zp), 1.0f, nph, ht, Mp,
                              static_cast<int64_t>(H) * Mp, stream))
    return rc;
  if (int rc = wgrad::codes_t(sv.w_ih_q, C, nullptr, C, I, I, 1, 0.0f, 1.0f, npw, wt, C,
                              static_cast<int64_t>(I) * C, stream))
    return rc;
  {
    std::vector<float> qs(I + H);
    for (int k = 0; k < I; ++k) qs[k] = static_cast<float>(sp.x.dscale);
    for (int k = 0; k < H; ++k) qs[I + k] = static_cast<float>(sp.h.dscale);
    RXMET_CHECK_HIP(hipMemcpyAsync(qsc, qs.data(), sizeof(float) * (I + H), hipMemcpyHostToDevice,
                                   stream));
  }

  BwdArgs ba;
  ba.T = T; ba.B = B; ba.H = H; ba.KS2 = KS2; ba.UT = UT;
  ba.grad_out = grad_output; ba.grad_hn = grad_h_n; ba.grad_cn = grad_c_n;
  ba.gate_out = sv.gate_out; ba.cell = sv.cell; ba.cell_tanh = sv.cell_tanh; ba.c0_q = sv.c0_q;
  ba.ih_m = sv.ih_linear_m; ba.hh_m = sv.hh_linear_m; ba.gin_m = sv.gate_in_m;
  ba.gout_m = sv.gate_out_m; ba.cell_m = sv.cell_m; ba.tanh_m = sv.cell_tanh_m;
  ba.hid_m = sv.hidden_m; ba.h0_m = sv.h0_m; ba.c0_m = sv.c0_m;
  ba.frag = frag; ba.colsum = colsum; ba.s_whh = swhh;
  for (int g = 0; g < 4; ++g) {
    ba.s_gout[g] = sp.gout[g].dscale;
    ba.zp_gout[g] = sp.gout[g].dzp;
  }
  ba.s_c = sp.c.dscale; ba.zp_c = sp.c.dzp; ba.s_t = sp.tanh_c.dscale; ba.zp_t = sp.tanh_c.dzp;
  ba.dli = dli; ba.dlh = dlh; ba.dh0 = dh0; ba.dc0 = dc0;
  ba.ckb = nullptr; ba.cellc = nullptr;
  if (codes) {
    ba.gate_out = ba.cell = ba.cell_tanh = nullptr;
    ba.hh_m = ba.gin_m = ba.gout_m = ba.cell_m = ba.tanh_m = ba.hid_m = nullptr;
    ba.ckb = codes->blocks;
    ba.cellc = codes->cell_codes;
    for (int g = 0; g < 4; ++g) ba.lo_gout[g] = sp.gout[g].lo;
    ba.lo_c = sp.c.lo;
    ba.lo_t = sp.tanh_c.lo;
  }
  bool recurrence_done = false;  // set by the stepped or the clustered recurrence
  int *timeout_flag = nullptr;
  if (stepped) {
    const int npwh = wgrad::planes_for(gwh_b.lo, gwh_b.hi, 0.0);
    __bf16 *whht = reinterpret_cast<__bf16 *>(wsb + ws.whht);
    float *dhr = reinterpret_cast<float *>(wsb + ws.dhr);
    float *dcs = reinterpret_cast<float *>(wsb + ws.dcs);
    // W_hh codes [4H][H] transposed: row j (unit) holds the 4H channels
    if (int rc = wgrad::codes_t(sv.w_hh_q, C, nullptr, C, H, H, 1, 0.0f, 1.0f, npwh, whht, C,
                                static_cast<int64_t>(H) * C, stream))
      return rc;
    wgrad::NtArgs na;
    na.lda = C;
    na.kscale = swhh;
    na.Bt = whht; na.ldb = C; na.bplane = static_cast<int64_t>(H) * C;
    na.M = B; na.N = H; na.K = C; na.out = dhr; na.ldo = H;
    // a K split that fills the GPU (the parts are summed in order by the next step's pointwise)
    wgrad::nt_plan(B, H, C, kBStepMaxSplit, &na.ksplit, &na.kper);
    na.out_split = static_cast<int64_t>(B) * H;
    const int64_t n = static_cast<int64_t>(B) * H;
    const dim3 pgrid(static_cast<unsigned>((n + 255) / 256));
    {
      rxmet::prof::Scope ps__("lstm_bwd_recurrence", stream);
      for (int t = T - 1; t >= 0; --t) {
        hipLaunchKernelGGL(lstm_bstep_point, pgrid, dim3(256), 0, stream, ba, t, na.ksplit, dhr,
                           dcs);
        RXMET_CHECK_LAUNCH();
        na.A = dlh + static_cast<size_t>(t) * B * C;
        if (int rc = wgrad::nt(na, npwh, stream)) return rc;
      }
      hipLaunchKernelGGL(lstm_bstep_finish, pgrid, dim3(256), 0, stream, ba, na.ksplit, dhr, dcs);
      RXMET_CHECK_LAUNCH();
    }
    recurrence_done = true;
  }
  // (the exchange buffer, 6 Bpad C bytes, is addressed with 32-bit buffer offsets; checkpoint
  // rows are copied into LDS as 16-byte chunks)
  const auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool ck_aligned =
      codes ? a16(codes->blocks) && a16(codes->cell_codes) && a16(grad_output) && a16(sv.ih_linear_m)
            : a16(sv.gate_out) && a16(sv.cell) && a16(sv.cell_tanh) && a16(sv.c0_q) &&
                  a16(grad_output) && a16(sv.ih_linear_m) && a16(sv.hh_linear_m) &&
                  a16(sv.gate_in_m) && a16(sv.gate_out_m) && a16(sv.cell_m) &&
                  a16(sv.cell_tanh_m) && a16(sv.hidden_m);
  if (!stepped && H % (2 * kBcUnits) == 0 && KS2 <= 8 * kBcMaxKs && ck_aligned &&
      6.0 * ((B + kBB - 1) / kBB * kBB) * C < 2147483648.0 &&
      std::getenv("RXMET_NO_CLUSTER") == nullptr) {
    const void *fn = codes ? reinterpret_cast<const void *>(&lstm_bwd_recurrence_cl<true>)
                           : reinterpret_cast<const void *>(&lstm_bwd_recurrence_cl<false>);
    const size_t lds_cl = bwd_cl_lds();
    int device = 0, ncu = 0, per_cu = 0;
    RXMET_CHECK_HIP(hipGetDevice(&device));
    RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
    RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds_cl)));
    RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 512, lds_cl));
    BwdClArgs cl;
    cl.G = H / kBcUnits;
    cl.ntiles = (B + kBB - 1) / kBB;
    cl.Bpad = cl.ntiles * kBB;
    int ncl = per_cu * ncu / cl.G;
    if (ncl > cl.ntiles) ncl = cl.ntiles;
    if (ncl >= 8) ncl -= ncl % 8;
    if (ncl >= 1) {
      cl.ncl = ncl;
      v4i *wf = reinterpret_cast<v4i *>(wsb + ws.wfrag_cl);
      float *cs = reinterpret_cast<float *>(wsb + ws.csum);
      cl.wfrag = wf;
      cl.csum = cs;
      cl.xp = reinterpret_cast<int8_t *>(wsb + ws.xp);
      cl.xe = reinterpret_cast<int *>(wsb + ws.xe);
      cl.counters = reinterpret_cast<unsigned *>(wsb + ws.sync);
      cl.timeout = reinterpret_cast<int *>(cl.counters + cluster::kCounterStride * ncl);
      cl.spin_limit = cluster::spin_limit();
      hipLaunchKernelGGL(lstm_pack_whh_t_cl, dim3((H / 16) * KS2), dim3(64), 0, stream, H, KS2,
                         sv.w_hh_q, wf, cs);
      RXMET_CHECK_LAUNCH();
      hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, cl.counters,
                     cluster::kCounterStride * ncl + 1);
      RXMET_CHECK_LAUNCH();
      void *args[] = {&ba, &cl};
      {
        rxmet::prof::Scope ps__("lstm_bwd_recurrence", stream);
        RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * cl.G), dim3(512), args,
                                                   static_cast<unsigned>(lds_cl), stream));
      }
      timeout_flag = cl.timeout;
      recurrence_done = true;
    }
  }
  if (!recurrence_done) {
    hipLaunchKernelGGL(lstm_pack_whh_t, dim3(UT * KS2), dim3(64), 0, stream, H, KS2, sv.w_hh_q, frag,
                       colsum);
    RXMET_CHECK_LAUNCH();
    const size_t lds = bwd_lds(H, KS2);
    rxmet::prof::Scope ps__("lstm_bwd_recurrence", stream);
    RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&lstm_bwd_recurrence),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
    hipLaunchKernelGGL(lstm_bwd_recurrence, dim3((B + kBB - 1) / kBB),
                       dim3(64 * ((UT + kTPW - 1) / kTPW)), lds, stream, ba);
    RXMET_CHECK_LAUNCH();
  }

  {
    rxmet::prof::Scope ps__("lstm_bwd_weight_gemms", stream);
    // dx[M][I] = sum_c (dli[m][c] s_wih[c]) W_ih_q[c][i]
    wgrad::NtArgs na;
    na.A = dli; na.lda = C; na.kscale = swih;
    na.Bt = wt; na.ldb = C; na.bplane = static_cast<int64_t>(I) * C;
    na.M = M; na.N = I; na.K = C; na.out = dx; na.ldo = I;
    if (int rc = wgrad::nt(na, npw, stream)) return rc;
    // aug_ih[c][i] = s_x sum_m dli[m][c] (x_q - zp_x)[m][i], aug_ih[c][I] = sum_m dli[m][c]
    wgrad::TnArgs ta;
    ta.A = dli; ta.lda = C; ta.Bt = xt; ta.ldb = Mp; ta.bplane = static_cast<int64_t>(I) * Mp;
    ta.K = M; ta.P = C; ta.Q = I; ta.S = ws.S_ih[npx - 1]; ta.kper = ws.kper_ih[npx - 1];
    ta.part = part;
    ta.colsum = gsum;
    if (int rc = wgrad::tn(ta, npx, stream)) return rc;
    if (int rc = wgrad::tn_finish(part, ta.S, C, I, npx, qsc, aug_ih, I + 1, false, gsum, aug_ih + I,
                                  stream))
      return rc;
    // aug_hh[c][j] = s_h sum_m dlh[m][c] (h_prev - zp_h)[m][j], aug_hh[c][H] = sum_m dlh[m][c]
    ta.A = dlh; ta.Bt = ht; ta.bplane = static_cast<int64_t>(H) * Mp;
    ta.Q = H; ta.S = ws.S_hh[nph - 1]; ta.kper = ws.kper_hh[nph - 1];
    if (int rc = wgrad::tn(ta, nph, stream)) return rc;
    if (int rc = wgrad::tn_finish(part, ta.S, C, H, nph, qsc + I, aug_hh, H + 1, false, gsum,
                                  aug_hh + H, stream))
      return rc;
  }
  {
    const int64_t nx = static_cast<int64_t>(M) * I;
    const int64_t n = nx + static_cast<int64_t>(C) * (I + H + 1);
    int64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(lstm_bwd_finish, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       nx, dx, sv.x_m, C, I, H, aug_ih, aug_hh, dW_ih, dW_hh, bias ? db_ih : nullptr,
                       bias ? db_hh : nullptr, sv.w_ih_m, sv.w_hh_m, sv.b_ih_m, sv.b_hh_m);
    RXMET_CHECK_LAUNCH();
  }
  if (timeout_flag != nullptr) {
    // a clustered wait that timed out: every gradient becomes NaN
    const int64_t n_state = static_cast<int64_t>(B) * H;
    cluster::PoisonList pl{};
    float *ps[7] = {dx, dW_ih, dW_hh, bias ? db_ih : nullptr, bias ? db_hh : nullptr, dh0, dc0};
    const int64_t ns[7] = {static_cast<int64_t>(M) * I, static_cast<int64_t>(C) * I,
                           static_cast<int64_t>(C) * H, C, C, n_state, n_state};
    for (int j = 0; j < 7; ++j) {
      pl.p[j] = ps[j];
      pl.n[j] = ns[j];
    }
    pl.count = 7;
    hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, timeout_flag, pl);
    RXMET_CHECK_LAUNCH();
  }
  return 0;
}

int rxmet_lstm_backward_quant(int32_t T, int32_t B, int32_t I, int32_t H,
                              const rxmet_lstm_params *params, const rxmet_lstm_saved *saved,
                              const float *grad_output, const float *grad_h_n,
                              const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                              float *db_ih, float *db_hh, float *dh0, float *dc0,
                              void *workspace, void *stream_) {
  clear_error();
  return lstm_backward_impl(T, B, I, H, params, saved, nullptr, grad_output, grad_h_n, grad_c_n,
                            dx, dW_ih, dW_hh, db_ih, db_hh, dh0, dc0, workspace, stream_);
}

int rxmet_lstm_backward_quant_codes(int32_t T, int32_t B, int32_t I, int32_t H,
                                    const rxmet_lstm_params *params, const rxmet_lstm_saved *saved,
                                    const rxmet_lstm_saved_codes *codes,
                                    const float *grad_output, const float *grad_h_n,
                                    const float *grad_c_n, float *dx, float *dW_ih, float *dW_hh,
                                    float *db_ih, float *db_hh, float *dh0, float *dc0,
                                    void *workspace, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(codes != nullptr, "codes must be non-null");
  return lstm_backward_impl(T, B, I, H, params, saved, codes, grad_output, grad_h_n, grad_c_n,
                            dx, dW_ih, dW_hh, db_ih, db_hh, dh0, dc0, workspace, stream_);
}

}  // extern "C"
