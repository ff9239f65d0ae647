// gru_fwd.hip — MI355X QuantGRU forward (FP32-carrier QAT), behind rxmet_gru_forward_quant.
//
// Reference path: quantGRUForwardFP (operators/quant-gru/src/gru_interface.cc:636-716):
// four per-channel quantisation launches with a device sync each, x/h0 quantisation,
// one cuBLAS SGEMM for the input projection, then a host loop of T iterations each
// launching one SGEMM (R h) and one pointwise kernel (src/gru_forward_gpu_quant_fp.cu:
// 604-801), and two in-place dequantisation passes over h and v.
//
// Here:
//   1. quant_weights : W/R/bw/br quantisation (codes, masks), read in the kernel layout or in
//      PyTorch's layout and gate order; the fp32 column sums of codes times the input zero
//      points and the bias terms rint(b_q * ratio) the pointwise step needs (rows split over
//      eight threads per column where the float sums are exact);
//   2. quant_input   : x (read in place from the caller's layout, time-reversed for a reverse
//      direction) and h0 quantisation (codes + masks), h[0] dequantised;
//   3. code_gemm     : the time-parallel input projection W_q x_q summed exactly on int8 MFMA
//      over pre-packed byte planes and rounded once to fp32 (exact_gemm.h);
//   4. recurrence    : both directions' T steps in one clustered cooperative launch
//      (recurrence_cl; cluster.h): a batch tile's hidden units split over a cluster of
//      workgroups, the new h codes exchanged through global memory each step.  R_q lives in
//      VGPRs as int8 MFMA fragments for the whole kernel; h_t arrives as int8 planes (16-bit
//      codes as a high and a low byte plane); the pointwise update (bias rescale, gate
//      inputs, PWL sigmoid/tanh, hidden update, clamps and masks) is fused in registers, and
//      the step's outputs leave as 16-byte rows staged in LDS while the members wait.  The
//      per-tile fallback (recurrence) keeps one workgroup per 16 sequences.
#include <cmath>
#include <cstdlib>
#include <vector>

#include "cluster.h"
#include "exact_gemm.h"
#include "gru_internal.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_gru.h"

namespace rxmet {
namespace gru {

constexpr int kTileB = 16;   // sequences per recurrent workgroup (MFMA N)
constexpr int kMaxH = 256;   // 16 waves x 16 units
constexpr int kChanParams = 7;  // igx, igh, wsum, rsum, btx, bth, rcol

__device__ __forceinline__ float clamp_keep(float v, Bounds b, uint8_t &keep) {
  keep = (v < b.lo || v > b.hi) ? 0 : 1;
  return fmaxf(b.lo, fminf(v, b.hi));
}

// ---------------------------------------------------------------------------------
// 1. weights
// ---------------------------------------------------------------------------------
struct WeightArgs {
  const float *W, *R, *bw, *br;
  // element (k, c) of W / R at W[k w_sk + c' w_sc]; c' = c, or with swap set the column of
  // the (r, z, n) gate order (PyTorch's weight_ih [3H, I] / weight_hh [3H, H]); biases at [c']
  int64_t w_sk, w_sc, r_sk, r_sc;
  int swap;
  const float *eff;  // 8 x C host block: W, R, bw, br effective scales, ibx, ibh, igx, igh
  const float *ibx, *ibh;
  Bounds bW, bR, bbw, bbr;
  float zp_x, zp_h;
  float *Wq, *Rq, *bwq, *brq;
  uint8_t *Wm, *Rm, *bwm, *brm;
  float *chan;  // kChanParams x C, fills wsum, rsum, btx, bth, rcol
};

// One thread per gate column; rows are processed in blocks of kQwRows whose loads are all
// issued before any code is stored (the sums stay sequential in k, as the reference's).
constexpr int kQwRows = 32;
__global__ __launch_bounds__(64) void quant_weights(int I, int H, WeightArgs a) {
  const int C = 3 * H;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  uint8_t keep;
  const float ew = a.eff[c], er = a.eff[C + c], ebw = a.eff[2 * C + c], ebr = a.eff[3 * C + c];
  const int cs = a.swap ? (c < H ? c + H : (c < 2 * H ? c - H : c)) : c;
  float s = 0.0f;
  for (int k0 = 0; k0 < I; k0 += kQwRows) {
    float v[kQwRows];
#pragma unroll
    for (int r = 0; r < kQwRows; ++r)
      v[r] = k0 + r < I ? a.W[(k0 + r) * a.w_sk + cs * a.w_sc] : 0.0f;
#pragma unroll
    for (int r = 0; r < kQwRows; ++r) {
      if (k0 + r >= I) break;
      const size_t i = static_cast<size_t>(k0 + r) * C + c;
      const float q = clamp_keep(rintf(v[r] / ew) + 0.0f, a.bW, keep);
      a.Wq[i] = q;
      if (a.Wm) a.Wm[i] = keep;
      s += q;
    }
  }
  a.chan[c] = a.eff[6 * C + c];      // igx
  a.chan[C + c] = a.eff[7 * C + c];  // igh
  a.chan[2 * C + c] = a.zp_x != 0.0f ? s * a.zp_x : 0.0f;  // wsum
  s = 0.0f;
  int exact = 0;
  for (int k0 = 0; k0 < H; k0 += kQwRows) {
    float v[kQwRows];
#pragma unroll
    for (int r = 0; r < kQwRows; ++r)
      v[r] = k0 + r < H ? a.R[(k0 + r) * a.r_sk + cs * a.r_sc] : 0.0f;
#pragma unroll
    for (int r = 0; r < kQwRows; ++r) {
      if (k0 + r >= H) break;
      const size_t i = static_cast<size_t>(k0 + r) * C + c;
      const float q = clamp_keep(rintf(v[r] / er) + 0.0f, a.bR, keep);
      a.Rq[i] = q;
      if (a.Rm) a.Rm[i] = keep;
      s += q;
      exact += static_cast<int>(q);
    }
  }
  a.chan[3 * C + c] = a.zp_h != 0.0f ? s * a.zp_h : 0.0f;  // rsum
  a.chan[6 * C + c] = static_cast<float>(exact);            // rcol (exact)
  const float qbw = clamp_keep(rintf(a.bw[cs] / ebw) + 0.0f, a.bbw, keep);
  a.bwq[c] = qbw;
  if (a.bwm) a.bwm[c] = keep;
  const float qbr = clamp_keep(rintf(a.br[cs] / ebr) + 0.0f, a.bbr, keep);
  a.brq[c] = qbr;
  if (a.brm) a.brm[c] = keep;
  a.chan[4 * C + c] = rintf(qbw * a.ibx[c]);  // btx
  a.chan[5 * C + c] = rintf(qbr * a.ibh[c]);  // bth
}

// The same with the rows of each column split over kQsGroups threads, for grids where every
// partial sum of codes stays below 2^24: the float sums are then exact, so the split order gives
// the sequential sums bit for bit.  8 columns x 32 row groups per 256-thread block.
constexpr int kQsCols = 8, kQsGroups = 32;
__global__ __launch_bounds__(256) void quant_weights_split(int I, int H, WeightArgs a) {
  __shared__ float red[2][kQsGroups][kQsCols];
  __shared__ int redi[kQsGroups][kQsCols];
  const int C = 3 * H;
  const int cx = threadIdx.x % kQsCols, rg = threadIdx.x / kQsCols;
  const int c = blockIdx.x * kQsCols + cx;
  const bool on = c < C;
  const int cc = on ? c : 0;
  const int cs = a.swap ? (cc < H ? cc + H : (cc < 2 * H ? cc - H : cc)) : cc;
  uint8_t keep;
  float sw = 0.0f, sr = 0.0f;
  int exact = 0;
  if (on) {
    const float ew = a.eff[c], er = a.eff[C + c];
    // rows in batches of kQsBatch whose loads are all issued before any code is stored
    constexpr int kQsBatch = 8;
    for (int k0 = rg; k0 < I; k0 += kQsGroups * kQsBatch) {
      float v[kQsBatch];
#pragma unroll
      for (int r = 0; r < kQsBatch; ++r) {
        const int k = k0 + kQsGroups * r;
        v[r] = k < I ? a.W[k * a.w_sk + cs * a.w_sc] : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < kQsBatch; ++r) {
        const int k = k0 + kQsGroups * r;
        if (k < I) {
          const size_t i = static_cast<size_t>(k) * C + c;
          const float q = clamp_keep(rintf(v[r] / ew) + 0.0f, a.bW, keep);
          a.Wq[i] = q;
          if (a.Wm) a.Wm[i] = keep;
          sw += q;
        }
      }
    }
    for (int k0 = rg; k0 < H; k0 += kQsGroups * kQsBatch) {
      float v[kQsBatch];
#pragma unroll
      for (int r = 0; r < kQsBatch; ++r) {
        const int k = k0 + kQsGroups * r;
        v[r] = k < H ? a.R[k * a.r_sk + cs * a.r_sc] : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < kQsBatch; ++r) {
        const int k = k0 + kQsGroups * r;
        if (k < H) {
          const size_t i = static_cast<size_t>(k) * C + c;
          const float q = clamp_keep(rintf(v[r] / er) + 0.0f, a.bR, keep);
          a.Rq[i] = q;
          if (a.Rm) a.Rm[i] = keep;
          sr += q;
          exact += static_cast<int>(q);
        }
      }
    }
  }
  red[0][rg][cx] = sw;
  red[1][rg][cx] = sr;
  redi[rg][cx] = exact;
  __syncthreads();
  if (rg != 0 || !on) return;
  for (int g = 1; g < kQsGroups; ++g) {
    sw += red[0][g][cx];
    sr += red[1][g][cx];
    exact += redi[g][cx];
  }
  a.chan[c] = a.eff[6 * C + c];      // igx
  a.chan[C + c] = a.eff[7 * C + c];  // igh
  a.chan[2 * C + c] = a.zp_x != 0.0f ? sw * a.zp_x : 0.0f;  // wsum
  a.chan[3 * C + c] = a.zp_h != 0.0f ? sr * a.zp_h : 0.0f;  // rsum
  a.chan[6 * C + c] = static_cast<float>(exact);             // rcol (exact)
  const float ebw = a.eff[2 * C + c], ebr = a.eff[3 * C + c];
  const float qbw = clamp_keep(rintf(a.bw[cs] / ebw) + 0.0f, a.bbw, keep);
  a.bwq[c] = qbw;
  if (a.bwm) a.bwm[c] = keep;
  const float qbr = clamp_keep(rintf(a.br[cs] / ebr) + 0.0f, a.bbr, keep);
  a.brq[c] = qbr;
  if (a.brm) a.brm[c] = keep;
  a.chan[4 * C + c] = rintf(qbw * a.ibx[c]);  // btx
  a.chan[5 * C + c] = rintf(qbr * a.ibh[c]);  // bth
}

// ---------------------------------------------------------------------------------
// 2. inputs
// ---------------------------------------------------------------------------------
// Where x element (t, b, k) of the direction lies in the caller's input: t stride, b stride
// (elements, k stride 1) and whether the direction reads time reversed.
struct XLayout {
  int64_t st, sb;
  int rev;
  int torch_w;  // W, R, bw, br in PyTorch's layout and (r, z, n) gate order
};

__global__ __launch_bounds__(256) void quant_input(int64_t nx, int64_t nh, const float *x,
                                                   XLayout xl, int T, uint32_t BI, uint32_t I,
                                                   const float *h0, float eff_x, float zp_x,
                                                   Bounds bx, float eff_h, float zp_h, Bounds bh,
                                                   float *xq, uint8_t *xm, float *h0codes,
                                                   uint8_t *h0m, float *hout0) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  uint8_t keep;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nx + nh;
       i += stride) {
    if (i < nx) {
      // canonical [T, B, I] order of the direction; the source follows the caller's layout
      int64_t src = i;
      if (xl.rev || xl.st != static_cast<int64_t>(BI) || xl.sb != static_cast<int64_t>(I)) {
        const uint32_t ii = static_cast<uint32_t>(i), t = ii / BI, r = ii - t * BI, b = r / I;
        src = (xl.rev ? T - 1 - static_cast<int>(t) : static_cast<int>(t)) * xl.st + b * xl.sb +
              (r - b * I);
      }
      xq[i] = clamp_keep(rintf(x[src] / eff_x) + zp_x, bx, keep);
      if (xm) xm[i] = keep;
    } else {
      const int64_t j = i - nx;
      float q = zp_h;
      if (h0) {
        q = clamp_keep(rintf(h0[j] / eff_h) + zp_h, bh, keep);
        if (h0m) h0m[j] = keep;
      }
      h0codes[j] = q;
      hout0[j] = (q - zp_h) * eff_h;
    }
  }
}

// ---------------------------------------------------------------------------------
// 3. exact code GEMM  C[M][N] = A[M][K] * B[K][N]  (integer codes stored as fp32)
// ---------------------------------------------------------------------------------
// On int8 MFMA with byte planes (exact_gemm.h); the exact integer is rounded once to fp32.
template <int PA, int PB>
__global__ __launch_bounds__(256) void code_gemm(xgemm::Operands o, float *__restrict__ Cm) {
  xgemm::block<PA, PB>(o, blockIdx.y * xgemm::kTile, blockIdx.x * xgemm::kTile,
                       [&](int m, int n, long long s) {
                         Cm[static_cast<size_t>(m) * o.N + n] = static_cast<float>(s);
                       });
}

// Pre-packed variant (I <= kPackedMaxK): one wave per 16 rows and every fourth column tile.
constexpr int kPackedMaxK = 256;
template <int PA, int PB>
__global__ __launch_bounds__(256) void code_gemm_packed(xgemm::Packed p, float *__restrict__ Cm) {
  xgemm::rows16<PA, PB>(p, 16 * blockIdx.x, threadIdx.x / 64, 4,
                        [&](int m, int n, const long long *s, int rows) {
#pragma unroll
                          for (int r = 0; r < 4; ++r)
                            if (r < rows)
                              Cm[static_cast<size_t>(m + r) * p.N + n] = static_cast<float>(s[r]);
                        });
}

template <int PA>
static void launch_code_gemm(int pb, dim3 grid, hipStream_t stream, const xgemm::Operands &o,
                             float *C) {
  if (pb == 1)
    hipLaunchKernelGGL((code_gemm<PA, 1>), grid, dim3(256), 0, stream, o, C);
  else
    hipLaunchKernelGGL((code_gemm<PA, 2>), grid, dim3(256), 0, stream, o, C);
}

// ---------------------------------------------------------------------------------
// 4. persistent recurrence
// ---------------------------------------------------------------------------------
struct RecArgs {
  int T, B, H, KS;          // KS = ceil(H / 64) MFMA K-steps
  int training;
  float h_offset;           // 0 (signed h grid) or 2^(bits-1) (unsigned): centred codes
  const float *gih;         // [T, B, 3H] exact W_q x_q
  const v4i *rfrag;         // R_q as int8 MFMA B fragments, [H/16][3][KS][64]
  const float *chan;        // kChanParams x 3H
  const float *h0codes;     // [B, H]
  float *hout;              // [T+1, B, H] dequantised (row 0 written by quant_input)
  float *v;                 // [T, B, 4H] dequantised
  uint8_t *ih_m, *hh_m, *gin_m, *gout_m, *h_m;
  // saved state as codes (training, instead of v and the five mask arrays above): v_codes
  // [T, B, 4H] code minus grid minimum of z, r, n, hh_n; mask_bits [T, B, H] (code_mask_bits)
  uint16_t *vc, *mb;
  int8_t *hx;               // clustered path: [2][NPL][Bpad / 16][KS][16][64] exchanged h codes
                            // (1 KB blocks of 16 rows x 64 units, see hx_offset)
  int wide_out;             // clustered path: outputs 16-byte aligned (H % 16 == 0), stored
                            // through the LDS staging area as 16-byte rows
  int wide_acc;             // |R_q h| can reach 2^31: recombine the plane sums in int64
};

// R_q h of one element from its plane sums (exact).  With wide_acc clear the exact value fits
// in int32 and the modular uint32 combination is exact; otherwise it is combined in int64.
// Either way it is rounded once to fp32, as the exact sum of the oracle.
template <int NPL>
__device__ __forceinline__ float recombine_rh(int wide_acc, int lo, int hi, float plane_off,
                                              float h_offset, float colsum) {
  const int col = static_cast<int>(colsum);
  if (NPL == 2) {
    if (wide_acc)
      return static_cast<float>(256LL * hi + lo + static_cast<long long>(static_cast<int>(plane_off)) * col);
    return static_cast<float>(static_cast<int>(256u * static_cast<uint32_t>(hi) + static_cast<uint32_t>(lo) +
                                               static_cast<uint32_t>(static_cast<int>(plane_off)) *
                                                   static_cast<uint32_t>(col)));
  }
  return static_cast<float>(static_cast<int>(static_cast<uint32_t>(lo) +
                                             static_cast<uint32_t>(static_cast<int>(h_offset)) *
                                                 static_cast<uint32_t>(col)));
}

// R_q [H][3H] (fp32 codes) -> int8 B fragments of v_mfma_i32_16x16x64_i8:
// frag[((ut * 3 + g) * KS + s) * 64 + lane] holds R[k][c] for c = g*H + 16*ut + lane % 16,
// k = 64*s + 16*(lane / 16) + 0..15 (zero beyond H).
__global__ __launch_bounds__(64) void pack_r_frags(int H, int KS, const float *__restrict__ Rq,
                                                   v4i *__restrict__ frag) {
  const int lane = threadIdx.x;
  const int idx = blockIdx.x;  // (ut * 3 + g) * KS + s
  const int s = idx % KS, g = (idx / KS) % 3, ut = idx / (3 * KS);
  const int C = 3 * H;
  const int c = g * H + 16 * ut + lane % 16;
  int wd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int by[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 64 * s + 16 * (lane / 16) + 4 * q + e;
      by[e] = k < H ? static_cast<int>(Rq[static_cast<size_t>(k) * C + c]) : 0;
    }
    wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
  }
  frag[static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
}

// PWL activation on the carrier: segment = #thresholds <= q (capped at 15).
__device__ __forceinline__ float pwl_eval(float q, const float *thr, const float *qb,
                                          const int *nsh, const float *cc, float zp_x, Bounds ob,
                                          uint8_t &keep) {
  int idx = 0;
#pragma unroll
  for (int s = 8; s > 0; s >>= 1)
    if (thr[idx + s - 1] <= q) idx += s;
  const float prod = qb[idx] * (q - zp_x);
  const float val = rintf(ldexpf(prod, -nsh[idx])) + cc[idx];
  return clamp_keep(val, ob, keep);
}

// Gate activations by table.  A gate input is an integer code clamped to its grid (clamp_keep
// drops NaN), so when the grid has at most kGateTabMax codes the clustered recurrence
// tabulates pwl_eval over it once per launch: entry e of a gate holds code << 1 | keep for the
// input lo + e, one LDS read in place of the threshold search.
constexpr int kGateTabMax = 1024;
__device__ __forceinline__ float gate_tab(float q, const int *tab, float lo, uint8_t &keep) {
  const int e = tab[static_cast<int>(q - lo)];
  keep = static_cast<uint8_t>(e & 1);
  return static_cast<float>(e >> 1);
}

// One (sequence, unit) step of the FP carrier (gru_forward_gpu_quant_fp.cu:138-393): both
// linears from their exact sums (zero-point and bias terms, rescale, clamp), the three gates
// through the PWL LUTs (thresholds, slopes, offsets in lut_f, shifts in lut_n; 48 floats and
// 16 ints per gate; or the gate tables `tab`, three of kGateTabMax entries, when not null) and
// the hidden update, with the keep flag of every clamp.
struct PointOut {
  float h, z, r, n, rh_n;  // codes: new h, the gate outputs, the new gate's recurrent linear
  uint8_t k_ih[3], k_hh[3], k_gi[3], k_go[3], k_h;
};

__device__ __forceinline__ PointOut gru_point(const float gih[3], const float ghh[3],
                                              const float (&cst)[3][kChanParams],
                                              const StepParams &p, const float *lut_f,
                                              const int *lut_n, float hold,
                                              const int *tab = nullptr) {
  PointOut o;
  float wx[3], rh[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    float val = gih[g] - cst[g][2];
    wx[g] = clamp_keep(rintf((val + cst[g][4]) * cst[g][0]) + p.zp_wx, p.wx, o.k_ih[g]);
    val = ghh[g] - cst[g][3];
    rh[g] = clamp_keep(rintf((val + cst[g][5]) * cst[g][1]) + p.zp_rh, p.rh, o.k_hh[g]);
  }
  // update gate
  float in = rintf((wx[0] - p.zp_wx) * p.ih_to_zin) + rintf((rh[0] - p.zp_rh) * p.hh_to_zin);
  in += p.zp_zin;
  in = clamp_keep(in, p.zin, o.k_gi[0]);
  o.z = tab ? gate_tab(in, tab, p.zin.lo, o.k_go[0])
            : pwl_eval(in, lut_f, lut_f + 16, lut_n, lut_f + 32, p.lut[0].zp_x, p.zout, o.k_go[0]);
  // reset gate
  in = rintf((wx[1] - p.zp_wx) * p.ih_to_rin) + rintf((rh[1] - p.zp_rh) * p.hh_to_rin);
  in += p.zp_rin;
  in = clamp_keep(in, p.rin, o.k_gi[1]);
  o.r = tab ? gate_tab(in, tab + kGateTabMax, p.rin.lo, o.k_go[1])
            : pwl_eval(in, lut_f + 48, lut_f + 64, lut_n + 16, lut_f + 80, p.lut[1].zp_x, p.rout,
                       o.k_go[1]);
  // new gate
  const float rmul = (o.r - p.zp_rout) * (rh[2] - p.zp_rh);
  in = rintf((wx[2] - p.zp_wx) * p.ih_to_nin) + rintf(rmul * p.rmul_to_nin);
  in += p.zp_nin;
  in = clamp_keep(in, p.nin, o.k_gi[2]);
  o.n = tab ? gate_tab(in, tab + 2 * kGateTabMax, p.nin.lo, o.k_go[2])
            : pwl_eval(in, lut_f + 96, lut_f + 112, lut_n + 32, lut_f + 128, p.lut[2].zp_x, p.nout,
                       o.k_go[2]);
  // hidden update
  const float n_h = rintf((o.n - p.zp_nout) * p.nout_to_h) + p.zp_h;
  const float oldc = (o.z - p.zp_zout) * (hold - p.zp_h);
  const float newc = (p.quant_one - o.z) * (n_h - p.zp_h);
  const float h2 = rintf((oldc + newc) * p.old_to_h) + p.zp_h;
  o.h = clamp_keep(h2, p.h, o.k_h);
  o.rh_n = rh[2];
  return o;
}

// The 13 mask values of one element as bits: gate g's weight_ih_linear mask at bit g, its
// weight_hh_linear mask at 3 + g, gate input 6 + g, gate output 9 + g, the h mask at 12.
__device__ __forceinline__ unsigned code_mask_bits(const PointOut &o) {
  unsigned m = static_cast<unsigned>(o.k_h) << 12;
#pragma unroll
  for (int g = 0; g < 3; ++g)
    m |= static_cast<unsigned>(o.k_ih[g]) << g | static_cast<unsigned>(o.k_hh[g]) << (3 + g) |
         static_cast<unsigned>(o.k_gi[g]) << (6 + g) | static_cast<unsigned>(o.k_go[g]) << (9 + g);
  return m;
}

// A saved code as its offset from the grid's minimum (grids of at most 16 bits).
__device__ __forceinline__ unsigned code_u16(float code, float lo) {
  return static_cast<unsigned>(static_cast<int>(code - lo));
}

// Saved codes are blocked so that a workgroup's outputs of one step are contiguous: block
// ((t ceil(B/16) + b / 16) H/16 + j / 16) holds 16 rows (b % 16) of 16 units (j % 16); v codes
// as [16 rows][4 fields][16 units] (1024 per block), mask bits as [16 rows][16 units] (256).
// Returns block * 16 + b % 16: the row's index in units of 64 v codes / 16 mask words.
__device__ __forceinline__ uint32_t codes_row(int t, int b, int j, int B, int H) {
  const uint32_t nt = static_cast<uint32_t>(B + 15) / 16;
  return ((static_cast<uint32_t>(t) * nt + static_cast<uint32_t>(b) / 16) *
              (static_cast<uint32_t>(H) / 16) + static_cast<uint32_t>(j) / 16) * 16 +
         static_cast<uint32_t>(b) % 16;
}

// The outputs of one (step t, sequence b, unit j): dequantised h at row t + 1, and in
// training v (z, r, n, hh_n dequantised) and the five mask families, one element at a time
// (or their codes, with a.vc set).
__device__ __forceinline__ void store_point(const RecArgs &a, const StepParams &p, int t, int b,
                                            int j, const PointOut &o) {
  const uint32_t H = static_cast<uint32_t>(a.H), B = static_cast<uint32_t>(a.B), C = 3u * H;
  const uint32_t stepH = static_cast<uint32_t>(t) * B * H;
  const uint32_t oH = static_cast<uint32_t>(b) * H + j;
  a.hout[stepH + B * H + oH] = (o.h - p.zp_h) * p.eff_h;
  if (a.training && a.vc) {
    const uint32_t row = codes_row(t, b, j, a.B, a.H), e = static_cast<uint32_t>(j) % 16;
    a.vc[64 * row + e] = static_cast<uint16_t>(code_u16(o.z, p.zout.lo));
    a.vc[64 * row + 16 + e] = static_cast<uint16_t>(code_u16(o.r, p.rout.lo));
    a.vc[64 * row + 32 + e] = static_cast<uint16_t>(code_u16(o.n, p.nout.lo));
    a.vc[64 * row + 48 + e] = static_cast<uint16_t>(code_u16(o.rh_n, p.rh.lo));
    a.mb[16 * row + e] = static_cast<uint16_t>(code_mask_bits(o));
  } else if (a.training) {
    const uint32_t v0 = 4u * stepH + 4u * static_cast<uint32_t>(b) * H + j;
    a.v[v0] = (o.z - p.zp_zout) * p.eff_zout;
    a.v[v0 + H] = (o.r - p.zp_rout) * p.eff_rout;
    a.v[v0 + 2 * H] = (o.n - p.zp_nout) * p.eff_nout;
    a.v[v0 + 3 * H] = (o.rh_n - p.zp_rh) * p.eff_rh;
    const uint32_t m = static_cast<uint32_t>(t) * B * C + 3u * static_cast<uint32_t>(b) * H + j;
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      a.ih_m[m + g * H] = o.k_ih[g];
      a.hh_m[m + g * H] = o.k_hh[g];
      a.gin_m[m + g * H] = o.k_gi[g];
      a.gout_m[m + g * H] = o.k_go[g];
    }
    a.h_m[stepH + oH] = o.k_h;
  }
}

// One workgroup = 16 sequences x all H units; wave w owns unit tiles 2w and 2w+1.
// MFMA orientation: D[b][c] = h[b][:] . R[:, c]  (A = h planes from LDS, B = R_q fragments
// resident in VGPRs), so lane l owns unit 16u + (l % 16) for batch rows 4 (l / 16) + r.
template <int NPL>
__global__ __launch_bounds__(512) void recurrence(RecArgs a, StepParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 3 * H, B = a.B;
  const int ROW = a.KS * 64 + 16;  // plane row stride in bytes (conflict-free 16-B reads)
  float *hcode = reinterpret_cast<float *>(smem);                      // 2 * 16 * H
  float *lut_f = hcode + 2 * kTileB * H;                               // 3 * 16 * 3 (thr, qb, c)
  int *lut_n = reinterpret_cast<int *>(lut_f + 3 * 16 * 3);            // 3 * 16
  int8_t *plane = reinterpret_cast<int8_t *>(lut_n + 3 * 16);          // 2 * NPL * 16 * ROW

  const int tid = threadIdx.x;
  const int w = tid / 64, l = tid % 64;
  const int b0 = blockIdx.x * kTileB;
  const int nthreads = blockDim.x;

  for (int i = tid; i < 3 * 16; i += nthreads) {
    const int g = i / 16, s = i % 16;
    lut_f[g * 48 + s] = p.lut[g].thr[s];
    lut_f[g * 48 + 16 + s] = p.lut[g].qb[s];
    lut_f[g * 48 + 32 + s] = p.lut[g].c[s];
    lut_n[g * 16 + s] = p.lut[g].n[s];
  }
  for (int i = tid; i < 2 * NPL * kTileB * ROW / 4; i += nthreads)
    reinterpret_cast<int *>(plane)[i] = 0;
  __syncthreads();
  for (int i = tid; i < kTileB * H; i += nthreads) {
    const int n = i / H, j = i % H;
    const int b = b0 + n;
    const float q = b < B ? a.h0codes[static_cast<size_t>(b) * H + j] : p.zp_h;
    hcode[i] = q;
    const int hc = static_cast<int>(q - a.h_offset);
    if (NPL == 1) {
      plane[n * ROW + j] = static_cast<int8_t>(hc);
    } else {
      plane[n * ROW + j] = static_cast<int8_t>((hc & 255) - 128);            // low byte plane
      plane[(kTileB + n) * ROW + j] = static_cast<int8_t>(hc >> 8);         // high byte plane
    }
  }

  // R_q fragments (B operand) and per-channel constants of the two unit tiles.
  v4i rfr[2][3][4];
  float cst[2][3][kChanParams];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int unit = 16 * (2 * w + u) + (l % 16);
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const int c = g * H + unit;
#pragma unroll
      for (int q = 0; q < kChanParams; ++q) cst[u][g][q] = unit < H ? a.chan[q * C + c] : 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        rfr[u][g][s] = (s < a.KS && unit < H)
                           ? a.rfrag[(((2 * w + u) * 3 + g) * a.KS + s) * 64 + l]
                           : v4i{0, 0, 0, 0};
    }
  }
  __syncthreads();

  const float plane_off = 128.0f + a.h_offset;  // added back with the column sums (NPL == 2)
  const int nrow0 = 4 * (l / 16);                // first of the 4 batch rows owned

  for (int t = 0; t < a.T; ++t) {
    const int cur = t & 1, nxt = cur ^ 1;
    const int8_t *pc = plane + cur * NPL * kTileB * ROW;
    int8_t *pn = plane + nxt * NPL * kTileB * ROW;
    const float *hc = hcode + cur * kTileB * H;
    float *hn = hcode + nxt * kTileB * H;

#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 16 * (2 * w + u) + (l % 16);  // unit owned in this tile
      if (16 * (2 * w + u) >= H) continue;
      __builtin_amdgcn_sched_barrier(0);
      v4i acc[3][NPL];
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) acc[g][q] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s >= a.KS) break;
        v4i hfr[NPL];  // A fragments: h planes of the 16 sequences
#pragma unroll
        for (int q = 0; q < NPL; ++q)
          hfr[q] = *reinterpret_cast<const v4i *>(pc + (q * kTileB + l % 16) * ROW + 64 * s +
                                                  16 * (l / 16));
#pragma unroll
        for (int g = 0; g < 3; ++g)
#pragma unroll
          for (int q = 0; q < NPL; ++q) acc[g][q] = mfma_i8(hfr[q], rfr[u][g][s], acc[g][q]);
      }

#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nr = nrow0 + r;
        const int b = b0 + nr;
        const bool valid = b < B;
        // 32-bit element offsets from uniform bases keep the per-row addressing cheap
        float gi3[3], gh3[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) {
          // R_q h = 256 R hi + R lo' + (128 + offset) colsum(R)
          gh3[g] = recombine_rh<NPL>(a.wide_acc, acc[g][0][r], acc[g][NPL - 1][r], plane_off,
                                     a.h_offset, cst[u][g][6]);
          gi3[g] = valid ? a.gih[(static_cast<size_t>(t) * B + b) * C + g * H + j] : 0.0f;
        }
        const PointOut o = gru_point(gi3, gh3, cst[u], p, lut_f, lut_n, hc[nr * H + j]);
        const float h2 = o.h;
        if (valid) store_point(a, p, t, b, j, o);
        // next state into LDS
        hn[nr * H + j] = h2;
        const int hcv = static_cast<int>(h2 - a.h_offset);
        if (NPL == 1) {
          pn[nr * ROW + j] = static_cast<int8_t>(hcv);
        } else {
          pn[nr * ROW + j] = static_cast<int8_t>((hcv & 255) - 128);
          pn[(kTileB + nr) * ROW + j] = static_cast<int8_t>(hcv >> 8);
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------
// 4a'. stepped recurrence (recurrent weights wider than 8 bits)
// ---------------------------------------------------------------------------------
// Per step one exact GEMM ghh = h_q R_q (xgemm::block: byte planes on int8 MFMA, combined in
// int64, rounded once to fp32, as the oracle's exact sums) and one pointwise launch over all
// (sequence, unit) pairs; the h codes go through two fp32 [B, H] buffers.
template <int PA, int PB>
__global__ __launch_bounds__(256) void step_rh_gemm(xgemm::Operands o, float *ghh) {
  xgemm::block<PA, PB>(o, blockIdx.x * xgemm::kTile, blockIdx.y * xgemm::kTile,
                       [&](int m, int n, long long sum) {
                         ghh[static_cast<size_t>(m) * o.N + n] = static_cast<float>(sum);
                       });
}

__global__ __launch_bounds__(256) void step_point(RecArgs a, StepParams p, int t, const float *ghh,
                                                  const float *hcur, float *hnext) {
  __shared__ float lut_f[3 * 48];
  __shared__ int lut_n[3 * 16];
  for (int i = threadIdx.x; i < 3 * 16; i += blockDim.x) {
    const int g = i / 16, s = i % 16;
    lut_f[g * 48 + s] = p.lut[g].thr[s];
    lut_f[g * 48 + 16 + s] = p.lut[g].qb[s];
    lut_f[g * 48 + 32 + s] = p.lut[g].c[s];
    lut_n[g * 16 + s] = p.lut[g].n[s];
  }
  __syncthreads();
  const int H = a.H, C = 3 * H;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<int64_t>(a.B) * H) return;
  const int b = static_cast<int>(e / H), j = static_cast<int>(e % H);
  float gi[3], gh[3], cst[3][kChanParams];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const int c = g * H + j;
    gi[g] = a.gih[(static_cast<size_t>(t) * a.B + b) * C + c];
    gh[g] = ghh[static_cast<size_t>(b) * C + c];
#pragma unroll
    for (int q = 0; q < kChanParams; ++q) cst[g][q] = a.chan[q * C + c];
  }
  const PointOut o = gru_point(gi, gh, cst, p, lut_f, lut_n, hcur[e]);
  hnext[e] = o.h;
  store_point(a, p, t, b, j, o);
}

// ---------------------------------------------------------------------------------
// 4b. clustered recurrence: a batch tile's units split over G workgroups
// ---------------------------------------------------------------------------------
// Member m of a cluster owns UT unit tiles (16 units each) of one 16-sequence batch tile.
// Four waves per unit tile split the recurrent sum over the K-steps (wave q takes steps
// q, q+4, ...) with R_q fragments resident in VGPRs, add their partial sums through LDS, and
// then each finishes one of the four batch rows a lane's MFMA output holds.  The new h codes
// are exchanged through global memory (coherent accesses, double-buffered by step parity) and
// the members meet at a counter barrier once per step (cluster.h).
constexpr int kClMaxKPerWave = 4;  // K-steps per wave: H <= 1024
constexpr int kHsMax = 4;          // 16-byte h chunks staged per thread and step
constexpr int kStageMinH = 512;    // H from which the h tile is staged in LDS

struct ClArgs {
  int ncl, G, UT, ntiles, Bpad, ndir;  // clusters walk (direction, batch tile) pairs
  int stage_h;                         // h tile staged in LDS once per workgroup (large H)
  int gate_tab;                        // gate activations by table (every gate grid fits)
  unsigned *counters;                  // [ncl], kCounterStride words apart
  int *timeout;
  unsigned spin_limit;  // polls before a wait gives up (cluster::spin_limit())
};

// Staged mask bytes of fields f0..f0+ng-1 ([16 rows][13][UW] in LDS) to a mask array
// [T][B][ng][H] as 16-byte rows; c0 is this thread's first chunk.
__device__ __forceinline__ void flush_masks(uint8_t *arr, int f0, int ng, const uint8_t *sb, int UW,
                                            int bq, int b0, int B, int H, int member, size_t stepH,
                                            int c0, int nthr) {
  for (int c = c0; c < 16 * ng * bq; c += nthr) {
    const int row = c / (ng * bq), g = (c / bq) % ng, q = c % bq, bb = b0 + row;
    if (bb < B)
      *reinterpret_cast<uint4 *>(arr + ng * (stepH + static_cast<size_t>(bb) * H) + g * H +
                                 member * UW + 16 * q) =
          *reinterpret_cast<const uint4 *>(sb + (row * 13 + f0 + g) * UW + 16 * q);
  }
}

// Byte offset of (row b, unit j) in one plane of the exchange buffer: blocks of 16 rows x 64
// units, row-major inside, one per (batch tile, K-step), so that a wave reads an MFMA A fragment
// (lane L: row L % 16, units 16 (L / 16) .. + 15 of the step) as 1 KB of contiguous bytes.
__device__ __forceinline__ unsigned hx_offset(int b, int j, int KS) {
  return ((static_cast<unsigned>(b / kTileB) * KS + j / 64) * kTileB + b % kTileB) * 64 + j % 64;
}

// One (direction, batch tile) pair of the clustered recurrence, run by one member.
template <int NPL, bool STAGE>
__device__ __forceinline__ void recurrence_cl_pair(const RecArgs &a, const StepParams &p,
                                                   const ClArgs &cl, int tile, int member,
                                                   unsigned *counter, unsigned &epoch,
                                                   bool &alive) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 3 * H, B = a.B, KS = a.KS;
  float *lut_f = reinterpret_cast<float *>(smem);               // 3 * 16 * 3 (thr, qb, c)
  int *lut_n = reinterpret_cast<int *>(lut_f + 3 * 16 * 3);     // 3 * 16
  v4i *red = reinterpret_cast<v4i *>(smem + 1024);              // [UT][4][3][NPL][64]
  // output staging of one step: [16 rows][5][UW] floats (h, the four v fields) and
  // [16 rows][13][UW] mask bytes (ih, hh, gate in, gate out per gate; h)
  const int UW = 16 * cl.UT;
  float *sf = reinterpret_cast<float *>(red + static_cast<size_t>(cl.UT) * 4 * 3 * NPL * 64);
  uint8_t *sb = reinterpret_cast<uint8_t *>(sf + 16 * 5 * UW);
  // the tile's h codes of the step, [NPL][16][H + 16] bytes
  int8_t *hs = reinterpret_cast<int8_t *>(sb + 16 * 13 * UW);
  // gate tables, [3][kGateTabMax] (16-byte aligned: H is a multiple of 16)
  int *gtab = reinterpret_cast<int *>(hs + NPL * kTileB * (H + 16));
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int utl = w / 4, kq = w % 4;
  const int ut = member * cl.UT + utl;
  const int j = 16 * ut + l % 16;
  const int jj = 16 * utl + l % 16;  // unit within the member's slice of UW units
  const int nr = 4 * (l / 16) + kq;  // batch row finished by this lane

  for (int i = tid; i < 3 * 16; i += blockDim.x) {
    const int g = i / 16, s = i % 16;
    lut_f[g * 48 + s] = p.lut[g].thr[s];
    lut_f[g * 48 + 16 + s] = p.lut[g].qb[s];
    lut_f[g * 48 + 32 + s] = p.lut[g].c[s];
    lut_n[g * 16 + s] = p.lut[g].n[s];
  }
  // gate activations by table: only in the unstaged kernel (the staged one has no table; a
  // runtime branch there measured 5% slower on H = 1024 steps that never take it)
  const int *tab = nullptr;
  if (!STAGE && cl.gate_tab) {
    __syncthreads();  // the LUT is in LDS
    for (int i = tid; i < 3 * kGateTabMax; i += blockDim.x) {
      const int g = i / kGateTabMax, e = i % kGateTabMax;
      // selected, not indexed: a local array indexed by g would live in scratch memory
      const Bounds gi = g == 0 ? p.zin : (g == 1 ? p.rin : p.nin);
      const Bounds go = g == 0 ? p.zout : (g == 1 ? p.rout : p.nout);
      const float zpx = g == 0 ? p.lut[0].zp_x : (g == 1 ? p.lut[1].zp_x : p.lut[2].zp_x);
      if (e <= static_cast<int>(gi.hi - gi.lo)) {
        uint8_t k = 0;
        const float v = pwl_eval(gi.lo + static_cast<float>(e), lut_f + 48 * g, lut_f + 48 * g + 16,
                                 lut_n + 16 * g, lut_f + 48 * g + 32, zpx, go, k);
        gtab[i] = static_cast<int>(v) * 2 | k;
      }
    }
    tab = gtab;  // read after the first cluster barrier (a workgroup barrier as well)
  }
  v4i rfr[kClMaxKPerWave][3];
#pragma unroll
  for (int i = 0; i < kClMaxKPerWave; ++i) {
    const int s = kq + 4 * i;
#pragma unroll
    for (int g = 0; g < 3; ++g)
      rfr[i][g] = s < KS ? a.rfrag[((ut * 3 + g) * KS + s) * 64 + l] : v4i{0, 0, 0, 0};
  }
  float cst[3][kChanParams];
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int q = 0; q < kChanParams; ++q) cst[g][q] = a.chan[q * C + g * H + j];

  const float plane_off = 128.0f + a.h_offset;
  const unsigned plane_stride = static_cast<unsigned>(cl.Bpad) * KS * 64;
  // the exchange buffer, 2 NPL planes (32-bit byte offsets: checked by the launcher)
  const auto xr = cluster::buffer_rsrc(a.hx, 2u * NPL * plane_stride);
  v4i *myred = red + (static_cast<size_t>(utl) * 4 + kq) * 3 * NPL * 64;

  {
    const int b0 = tile * kTileB, b = b0 + nr;
    const bool valid = b < B;
    float hold = valid ? a.h0codes[static_cast<size_t>(b) * H + j] : p.zp_h;
    {
      const int hcv = static_cast<int>(hold - a.h_offset);
      unsigned char *dst = reinterpret_cast<unsigned char *>(a.hx) + hx_offset(b, j, KS);
#pragma unroll
      for (int q = 0; q < NPL; ++q)
        cluster::store_bytes_coherent(dst + q * plane_stride,
                                      NPL == 1 ? hcv : (q == 0 ? (hcv & 255) - 128 : hcv >> 8));
    }
    float gi_next[3];
    auto load_gih = [&](int t) {
#pragma unroll
      for (int g = 0; g < 3; ++g)
        gi_next[g] = valid ? a.gih[(static_cast<size_t>(t) * B + b) * C + g * H + j] : 0.0f;
    };
    load_gih(0);
    alive = cluster::sync(counter, ++epoch * cl.G, cl.timeout, cl.spin_limit);

    for (int t = 0; t < a.T && alive; ++t) {
      const int par = t & 1;
      const unsigned hin = par * NPL * plane_stride;  // byte offset of the step's planes
      int8_t *hout = a.hx + (par ^ 1) * NPL * plane_stride;
      float gih[3] = {gi_next[0], gi_next[1], gi_next[2]};
      // partial recurrent sums over this wave's K-steps
      v4i acc[3][NPL];
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) acc[g][q] = v4i{0, 0, 0, 0};
      if constexpr (STAGE) {
        // the tile's h codes are read from the exchange buffer once per workgroup (16-byte
        // coherent loads, all issued before any is stored) into LDS, where the unit tiles
        // share them (at H >= 512; at smaller H the extra barrier costs more than it saves)
        // 16-byte chunk e -> plane p, K-step s, row r, chunk c of the step: the tile's blocks
        // in order, 1 KB per 64 threads; chunks past H (a partial last step) are not stored
        const int rs = H + 16, n = NPL * KS * 64, nt = blockDim.x;
        const unsigned tb = hin + static_cast<unsigned>(tile) * KS * 1024;
        int4 hv[kHsMax];
#pragma unroll
        for (int i = 0; i < kHsMax; ++i) {
          const int e0 = tid + nt * i, e = e0 < n ? e0 : 0;
          const int p = e / (KS * 64), s = (e / 64) % KS;
          hv[i] = cluster::load_coherent16(xr, tb + p * plane_stride + s * 1024 + 16 * (e % 64));
        }
#pragma unroll
        for (int i = 0; i < kHsMax; ++i) {
          const int e = tid + nt * i;
          const int p = e / (KS * 64), s = (e / 64) % KS, r = (e / 4) % kTileB, c = 4 * s + e % 4;
          if (e < n && 16 * c < H)
            *reinterpret_cast<int4 *>(hs + (p * kTileB + r) * rs + 16 * c) = hv[i];
        }
        __syncthreads();
        const int8_t *hrow = hs + (l % 16) * rs + 16 * (l / 16);
        v4i hfr[kClMaxKPerWave][NPL];
#pragma unroll
        for (int i = 0; i < kClMaxKPerWave; ++i)
#pragma unroll
          for (int q = 0; q < NPL; ++q)
            if (kq + 4 * i < KS)
              hfr[i][q] = *reinterpret_cast<const v4i *>(hrow + q * kTileB * rs + 64 * (kq + 4 * i));
#pragma unroll
        for (int i = 0; i < kClMaxKPerWave; ++i)
          if (kq + 4 * i < KS) {
#pragma unroll
            for (int g = 0; g < 3; ++g)
#pragma unroll
              for (int q = 0; q < NPL; ++q) acc[g][q] = mfma_i8(hfr[i][q], rfr[i][g], acc[g][q]);
          }
      } else {
        // lane l: row l % 16, units 16 (l / 16) .. + 15 of K-step kq + 4 i
        const unsigned hrow = hin + static_cast<unsigned>(tile) * KS * 1024 + 64 * (l % 16) + 16 * (l / 16);
        v4i hfr[kClMaxKPerWave][NPL];
#pragma unroll
        for (int i = 0; i < kClMaxKPerWave; ++i)
#pragma unroll
          for (int q = 0; q < NPL; ++q)
            if (kq + 4 * i < KS) {
              const int4 v = cluster::load_coherent16(xr, hrow + q * plane_stride + 1024 * (kq + 4 * i));
              hfr[i][q] = v4i{v.x, v.y, v.z, v.w};
            }
#pragma unroll
        for (int i = 0; i < kClMaxKPerWave; ++i)
          if (kq + 4 * i < KS) {
#pragma unroll
            for (int g = 0; g < 3; ++g)
#pragma unroll
              for (int q = 0; q < NPL; ++q) acc[g][q] = mfma_i8(hfr[i][q], rfr[i][g], acc[g][q]);
          }
      }
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) myred[(g * NPL + q) * 64 + l] = acc[g][q];
      __syncthreads();
      int sum[3][NPL];
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) {
          int v = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int *src = reinterpret_cast<const int *>(
                red + ((static_cast<size_t>(utl) * 4 + k) * 3 * NPL + g * NPL + q) * 64 + l);
            v += src[kq];
          }
          sum[g][q] = v;
        }
      // pointwise update of (row b, unit j)
      float gh3[3];
#pragma unroll
      for (int g = 0; g < 3; ++g)
        gh3[g] = recombine_rh<NPL>(a.wide_acc, sum[g][0], sum[g][NPL - 1], plane_off, a.h_offset,
                                   cst[g][6]);
      const PointOut o = gru_point(gih, gh3, cst, p, lut_f, lut_n, hold, tab);
      const float h2 = o.h;
      hold = h2;
      {
        const int hcv = static_cast<int>(h2 - a.h_offset);
        unsigned char *dst = reinterpret_cast<unsigned char *>(hout) + hx_offset(b, j, KS);
#pragma unroll
        for (int q = 0; q < NPL; ++q)
          cluster::store_bytes_coherent(dst + q * plane_stride,
                                        NPL == 1 ? hcv : (q == 0 ? (hcv & 255) - 128 : hcv >> 8));
      }
      if (a.wide_out) {
        float *f = sf + nr * 5 * UW + jj;
        f[0] = (h2 - p.zp_h) * p.eff_h;
        if (a.training && a.vc) {
          // codes in their blocked layout (codes_row), over the mask bytes: the member's UT
          // v-code blocks, then its UT mask-bit blocks
          uint16_t *c16 = reinterpret_cast<uint16_t *>(sb) + (utl * 16 + nr) * 64 + l % 16;
          c16[0] = static_cast<uint16_t>(code_u16(o.z, p.zout.lo));
          c16[16] = static_cast<uint16_t>(code_u16(o.r, p.rout.lo));
          c16[32] = static_cast<uint16_t>(code_u16(o.n, p.nout.lo));
          c16[48] = static_cast<uint16_t>(code_u16(o.rh_n, p.rh.lo));
          reinterpret_cast<uint16_t *>(sb)[1024 * cl.UT + (utl * 16 + nr) * 16 + l % 16] =
              static_cast<uint16_t>(code_mask_bits(o));
        } else if (a.training) {
          f[UW] = (o.z - p.zp_zout) * p.eff_zout;
          f[2 * UW] = (o.r - p.zp_rout) * p.eff_rout;
          f[3 * UW] = (o.n - p.zp_nout) * p.eff_nout;
          f[4 * UW] = (o.rh_n - p.zp_rh) * p.eff_rh;
          uint8_t *m8 = sb + nr * 13 * UW + jj;
#pragma unroll
          for (int g = 0; g < 3; ++g) {
            m8[g * UW] = o.k_ih[g];
            m8[(3 + g) * UW] = o.k_hh[g];
            m8[(6 + g) * UW] = o.k_gi[g];
            m8[(9 + g) * UW] = o.k_go[g];
          }
          m8[12 * UW] = o.k_h;
        }
      }
      // the other members only read the h codes: arrive now, store the outputs while waiting
      // (the arrival's workgroup barrier also publishes the staged outputs)
      cluster::arrive(counter);
      ++epoch;
      if (a.wide_out) {
        // 16-byte rows of the staged outputs, spread over the whole workgroup (each array
        // in a loop of its own: a pointer chosen per lane would put the arguments in scratch)
        const size_t stepH = static_cast<size_t>(t) * B * H;
        const int nthr = blockDim.x, fq = UW / 4;
        for (int c = tid; c < 16 * fq; c += nthr) {
          const int row = c / fq, q = c % fq, bb = b0 + row;
          if (bb < B)
            *reinterpret_cast<float4 *>(a.hout + stepH + static_cast<size_t>(B + bb) * H +
                                        member * UW + 4 * q) =
                *reinterpret_cast<const float4 *>(sf + row * 5 * UW + 4 * q);
        }
        if (a.training && a.vc) {
          // one contiguous run of UT blocks per array (the batch tile's padding rows too)
          const uint4 *c16 = reinterpret_cast<const uint4 *>(sb);
          const size_t blk = (static_cast<size_t>(t) * cl.ntiles + tile) * (H / 16) +
                             static_cast<size_t>(member) * cl.UT;
          uint4 *dv = reinterpret_cast<uint4 *>(a.vc + blk * 1024);
          uint4 *dm = reinterpret_cast<uint4 *>(a.mb + blk * 256);
          const int nv = 128 * cl.UT, nm = 32 * cl.UT;  // 16-byte chunks
          for (int c = (tid + nthr - (16 * fq) % nthr) % nthr; c < nv; c += nthr) dv[c] = c16[c];
          for (int c = (tid + nthr - (16 * fq + nv) % nthr) % nthr; c < nm; c += nthr)
            dm[c] = c16[nv + c];
        } else if (a.training) {
          for (int c = (tid + nthr - (16 * fq) % nthr) % nthr; c < 64 * fq; c += nthr) {
            const int row = c / (4 * fq), fld = (c / fq) % 4, q = c % fq, bb = b0 + row;
            if (bb < B)
              *reinterpret_cast<float4 *>(a.v + 4 * (stepH + static_cast<size_t>(bb) * H) +
                                          fld * H + member * UW + 4 * q) =
                  *reinterpret_cast<const float4 *>(sf + (row * 5 + 1 + fld) * UW + 4 * q);
          }
          const int bq = UW / 16;
          flush_masks(a.ih_m, 0, 3, sb, UW, bq, b0, B, H, member, stepH, (tid + 0 * 48 * bq) % nthr, nthr);
          flush_masks(a.hh_m, 3, 3, sb, UW, bq, b0, B, H, member, stepH, (tid + nthr - (48 * bq) % nthr) % nthr, nthr);
          flush_masks(a.gin_m, 6, 3, sb, UW, bq, b0, B, H, member, stepH, (tid + nthr - (96 * bq) % nthr) % nthr, nthr);
          flush_masks(a.gout_m, 9, 3, sb, UW, bq, b0, B, H, member, stepH, (tid + nthr - (144 * bq) % nthr) % nthr, nthr);
          flush_masks(a.h_m, 12, 1, sb, UW, bq, b0, B, H, member, stepH, (tid + nthr - (192 * bq) % nthr) % nthr, nthr);
        }
      } else if (valid) {
        store_point(a, p, t, b, j, o);
      }
      if (t + 1 < a.T) load_gih(t + 1);
      alive = cluster::wait(counter, epoch * cl.G, cl.timeout, cl.spin_limit);
    }
  }
}

template <int NPL, bool STAGE>
__global__ __launch_bounds__(512) void recurrence_cl(RecArgs a0, RecArgs a1,
                                                     const StepParams *__restrict__ ps,
                                                     ClArgs cl) {
  const cluster::Place pl = cluster::place(cl.G, cl.ncl);
  unsigned *counter = cl.counters + cluster::kCounterStride * pl.cluster;
  unsigned epoch = 0;
  bool alive = true;
  for (int pair = pl.cluster; pair < cl.ndir * cl.ntiles && alive; pair += cl.ncl) {
    const int d = pair / cl.ntiles, tile = pair % cl.ntiles;
    // the previous pair's readers of the LUT and the partial-sum buffer are done
    __syncthreads();
    // one copy of the step code for both directions (d is uniform across the workgroup)
    recurrence_cl_pair<NPL, STAGE>(d == 0 ? a0 : a1, ps[d], cl, tile, pl.member, counter, epoch,
                                   alive);
  }
}

size_t recurrence_cl_lds_bytes(int UT, int npl, int H, bool gate_tab) {
  return 1024 + sizeof(v4i) * static_cast<size_t>(UT) * 4 * 3 * npl * 64 +
         static_cast<size_t>(16) * 16 * UT * (5 * sizeof(float) + 13) +
         static_cast<size_t>(npl) * kTileB * (H + 16) + (gate_tab ? sizeof(int) * 3 * kGateTabMax : 0);
}


size_t recurrence_lds_bytes(int H, int KS, int npl) {
  const int ROW = KS * 64 + 16;
  return sizeof(float) * (2 * kTileB * H + 3 * 16 * 3) + sizeof(int) * 3 * 16 +
         static_cast<size_t>(2) * npl * kTileB * ROW;
}

// Workspace layout of the forward (bytes, 256-aligned pieces).
struct FwdWorkspace {
  size_t gih, chan, h0codes, hostblk, rfrag, hx, sync, sparams, xa, bfrag, colsum, sh, sg, total;
  FwdWorkspace(int T, int B, int I, int H) {
    const size_t C = 3 * static_cast<size_t>(H);
    const size_t Kp = static_cast<size_t>(xgemm::pad_k(I));
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t o = 0;
    gih = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * C);
    chan = o; o += al(sizeof(float) * kChanParams * C);
    h0codes = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    hostblk = o; o += al(sizeof(float) * 8 * C);  // eff[4C], ibx, ibh, igx, igh
    rfrag = o; o += al(sizeof(v4i) * 64 * static_cast<size_t>(H / 16) * 3 * ((H + 63) / 64));
    const size_t Bpad = (static_cast<size_t>(B) + kTileB - 1) / kTileB * kTileB;
    hx = o; o += al(2 * 2 * Bpad * ((H + 63) / 64) * 64);
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (2 * (Bpad / kTileB) + 2));  // clusters of both directions
    sparams = o; o += al(2 * sizeof(StepParams));
    // packed operands of the input projection (I <= 256): x planes, W fragments, W column sums
    const size_t ip = static_cast<size_t>(I) <= kPackedMaxK ? 1 : 0;
    xa = o; o += al(ip * 2 * static_cast<size_t>(T) * B * Kp);
    bfrag = o; o += al(ip * 2 * ((C + 15) / 16 * 16) * Kp);  // fragments of 16-column tiles
    colsum = o; o += al(ip * sizeof(long long) * C);
    // stepped recurrence: two h code buffers [B, H] and the recurrent sums [B, 3H]
    sh = o; o += al(sizeof(float) * 2 * static_cast<size_t>(B) * H);
    sg = o; o += al(sizeof(float) * static_cast<size_t>(B) * C);
    total = o;
  }
};

// Recurrent weights wider than signed 8 bits run on the stepped recurrence (two byte planes).
static bool needs_stepped(const rxmet_gru_qparams &p) {
  return p.chan_bits[RXMET_GRU_R] > 8 || p.chan_unsigned[RXMET_GRU_R] != 0;
}

static int host_bits_check(const rxmet_gru_qparams &p) {
  const Bounds br = bounds_of(p.chan_bits[RXMET_GRU_R], p.chan_unsigned[RXMET_GRU_R]);
  RXMET_CHECK_ARG(xgemm::b_fits(br.lo, br.hi),
                  "recurrent weights must fit signed 16 bits");
  RXMET_CHECK_ARG(p.g[RXMET_GRU_H].bits <= 16, "hidden-state grids wider than 16 bits are not supported");
  RXMET_CHECK_ARG(p.g[RXMET_GRU_X].bits <= 16 && p.chan_bits[RXMET_GRU_W] <= 16,
                  "input or input-weight grids wider than 16 bits are not supported");
  return 0;
}

}  // namespace gru
}  // namespace rxmet

namespace rxmet {
namespace gru {

// One direction's prologue (quantisation, input projection, R_q fragments) and the
// recurrence arguments it leaves for the launch.
struct FwdPlan {
  RecArgs ra;
  StepParams sp;
  int npl;
  bool stepped;  // recurrent weights wider than 8 bits: forward_recurrence_stepped
  const float *rq;  // R_q codes [H, 3H]
  char *wsb;
};

static int forward_prologue(bool training, int T, int B, int I, int H, const rxmet_gru_fwd_dir &d,
                            const XLayout &xl, const rxmet_gru_saved_codes *codes,
                            hipStream_t stream, FwdPlan *plan) {
  const rxmet_gru_qparams *params = d.params;
  RXMET_CHECK_ARG(params != nullptr, "params must be non-null");
  RXMET_CHECK_ARG(params->hidden == H, "params.hidden != hidden_size");
  RXMET_CHECK_ARG(d.W && d.R && d.bw && d.br && d.x && d.h && d.W_q && d.R_q && d.bw_q && d.br_q &&
                      d.x_q && d.workspace,
                  "required pointer is null");
  if (int rc = host_bits_check(*params)) return rc;
  if (training && codes) {
    RXMET_CHECK_ARG(codes->v_codes && codes->mask_bits && d.x_mask && d.W_mask && d.R_mask &&
                        d.bw_mask && d.br_mask && (d.h0 == nullptr || d.h0_mask),
                    "training needs the saved codes and the x, W, R and bias mask outputs");
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    RXMET_CHECK_ARG(a16(codes->v_codes) && a16(codes->mask_bits),
                    "v_codes and mask_bits must be 16-byte aligned");
    for (int gi : {RXMET_GRU_Z_OUT, RXMET_GRU_R_OUT, RXMET_GRU_N_OUT, RXMET_GRU_RH}) {
      const Bounds b = bounds_of(params->g[gi].bits, params->g[gi].is_unsigned);
      RXMET_CHECK_ARG(b.hi - b.lo <= 65535.0f,
                      "saved codes need gate output and weight_hh_linear grids of at most 16 bits");
    }
  } else if (training) {
    RXMET_CHECK_ARG(d.v && d.x_mask && d.W_mask && d.R_mask && d.bw_mask && d.br_mask &&
                        d.ih_mask && d.hh_mask && d.gate_in_mask && d.gate_out_mask && d.h_mask &&
                        (d.h0 == nullptr || d.h0_mask),
                    "training needs v and every mask output");
  }
  RXMET_CHECK_ARG(I < (1 << 17), "input_size must be below 131072 for the exact input GEMM");
  {
    const Bounds bx = bounds_of(params->g[RXMET_GRU_X].bits, params->g[RXMET_GRU_X].is_unsigned);
    const Bounds bw = bounds_of(params->chan_bits[RXMET_GRU_W], params->chan_unsigned[RXMET_GRU_W]);
    RXMET_CHECK_ARG(xgemm::a_fits(bx.lo, bx.hi) && xgemm::b_fits(bw.lo, bw.hi),
                    "x and W codes must fit 16 bits (signed W) for the exact input GEMM");
  }
  const int C = 3 * H;
  const FwdWorkspace ws(T, B, I, H);
  char *wsb = static_cast<char *>(d.workspace);
  float *gih = reinterpret_cast<float *>(wsb + ws.gih);
  float *chan = reinterpret_cast<float *>(wsb + ws.chan);
  float *h0codes = reinterpret_cast<float *>(wsb + ws.h0codes);
  float *hostblk = reinterpret_cast<float *>(wsb + ws.hostblk);

  StepParams &sp = plan->sp;
  std::vector<float> host(8 * static_cast<size_t>(C));
  try {
    make_step_params(*params, H, &sp);
    // host block: eff[4C] | ibx | ibh | igx | igh
    make_channel_factors(*params, H, host.data() + 6 * C, host.data() + 4 * C, host.data() + 7 * C,
                         host.data() + 5 * C, host.data(), host.data() + C, host.data() + 2 * C,
                         host.data() + 3 * C);
  } catch (const std::exception &e) {
    set_error(e.what());
    return -22;
  }
  // one upload; quant_weights copies igx / igh into the per-channel block
  RXMET_CHECK_HIP(hipMemcpyAsync(hostblk, host.data(), sizeof(float) * host.size(),
                                 hipMemcpyHostToDevice, stream));
  const rxmet_grid *g = params->g;
  WeightArgs wa;
  wa.W = d.W; wa.R = d.R; wa.bw = d.bw; wa.br = d.br;
  wa.swap = xl.torch_w;
  wa.w_sk = xl.torch_w ? 1 : C; wa.w_sc = xl.torch_w ? I : 1;
  wa.r_sk = xl.torch_w ? 1 : C; wa.r_sc = xl.torch_w ? H : 1;
  wa.eff = hostblk;
  wa.ibx = hostblk + 4 * C;
  wa.ibh = hostblk + 5 * C;
  wa.bW = bounds_of(params->chan_bits[RXMET_GRU_W], params->chan_unsigned[RXMET_GRU_W]);
  wa.bR = bounds_of(params->chan_bits[RXMET_GRU_R], params->chan_unsigned[RXMET_GRU_R]);
  wa.bbw = bounds_of(params->chan_bits[RXMET_GRU_BW], params->chan_unsigned[RXMET_GRU_BW]);
  wa.bbr = bounds_of(params->chan_bits[RXMET_GRU_BR], params->chan_unsigned[RXMET_GRU_BR]);
  wa.zp_x = static_cast<float>(g[RXMET_GRU_X].zero_point);
  wa.zp_h = static_cast<float>(g[RXMET_GRU_H].zero_point);
  wa.Wq = d.W_q; wa.Rq = d.R_q; wa.bwq = d.bw_q; wa.brq = d.br_q;
  wa.Wm = training ? d.W_mask : nullptr;
  wa.Rm = training ? d.R_mask : nullptr;
  wa.bwm = training ? d.bw_mask : nullptr;
  wa.brm = training ? d.br_mask : nullptr;
  wa.chan = chan;
  {
    rxmet::prof::Scope ps__("gru_fwd_quant_weights", stream);
    // partial sums of codes exact in float (below 2^24): rows split over 8 threads
    const double wmax = std::max(std::fabs(static_cast<double>(wa.bW.lo)), std::fabs(static_cast<double>(wa.bW.hi)));
    const double rmax = std::max(std::fabs(static_cast<double>(wa.bR.lo)), std::fabs(static_cast<double>(wa.bR.hi)));
    if (wmax * I < 16777216.0 && rmax * H < 16777216.0)
      hipLaunchKernelGGL(quant_weights_split, dim3((C + kQsCols - 1) / kQsCols), dim3(256), 0, stream,
                         I, H, wa);
    else
      hipLaunchKernelGGL(quant_weights, dim3((C + 63) / 64), dim3(64), 0, stream, I, H, wa);
  }
  RXMET_CHECK_LAUNCH();

  const int64_t nx = static_cast<int64_t>(T) * B * I, nh = static_cast<int64_t>(B) * H;
  int64_t blocks = (nx + nh + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  {
    rxmet::prof::Scope ps__("gru_fwd_quant_input", stream);
    hipLaunchKernelGGL(quant_input, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, nx,
                       nh, d.x, xl, T, static_cast<uint32_t>(static_cast<int64_t>(B) * I),
                       static_cast<uint32_t>(I), d.h0, sp.eff_x, sp.zp_x, sp.x, sp.eff_h, sp.zp_h,
                       sp.h, d.x_q,
                       training ? d.x_mask : nullptr, h0codes, training ? d.h0_mask : nullptr,
                       d.h);
  }
  RXMET_CHECK_LAUNCH();

  const int M = T * B;
  {
    // x codes lie on the x grid, W codes on the (symmetric or not) W grid
    const Bounds bx = bounds_of(g[RXMET_GRU_X].bits, g[RXMET_GRU_X].is_unsigned);
    const double xlo = bx.lo, xhi = bx.hi;
    const float off = xgemm::a_shift(xlo, xhi);
    const int pa = xgemm::a_planes(xlo, xhi), pb = xgemm::b_planes(wa.bW.lo, wa.bW.hi);
    rxmet::prof::Scope ps__("gru_fwd_input_gemm", stream);
    if (I <= kPackedMaxK) {
      const int Kp = xgemm::pad_k(I);
      int8_t *xa = reinterpret_cast<int8_t *>(wsb + ws.xa);
      v4i *bf = reinterpret_cast<v4i *>(wsb + ws.bfrag);
      long long *cs = reinterpret_cast<long long *>(wsb + ws.colsum);
      if (int rc = xgemm::pack_a(d.x_q, I, M, I, off, pa, xa, Kp, stream)) return rc;
      if (int rc = xgemm::pack_b(d.W_q, C, 1, I, C, pb, Kp, bf, cs, stream)) return rc;
      xgemm::Packed p;
      p.A = xa; p.aplane = static_cast<int64_t>(M) * Kp; p.Kp = Kp;
      p.B = bf; p.bplane = static_cast<int64_t>((C + 15) / 16) * (Kp / 64) * 64;
      p.colsum = cs; p.corr = static_cast<long long>(off); p.M = M; p.N = C;
      const dim3 grid((M + 15) / 16);
      auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p, gih); };
      if (pa == 1)
        pb == 1 ? go(code_gemm_packed<1, 1>) : go(code_gemm_packed<1, 2>);
      else
        pb == 1 ? go(code_gemm_packed<2, 1>) : go(code_gemm_packed<2, 2>);
    } else {
      xgemm::Operands o;
      o.M = M; o.N = C; o.K = I;
      o.A = d.x_q; o.lda = I;
      o.off = off;
      o.corr = static_cast<long long>(o.off);
      o.B = d.W_q; o.sbk = C; o.sbn = 1;
      const dim3 grid((C + 63) / 64, (M + 63) / 64);
      if (pa == 1)
        launch_code_gemm<1>(pb, grid, stream, o, gih);
      else
        launch_code_gemm<2>(pb, grid, stream, o, gih);
    }
  }
  RXMET_CHECK_LAUNCH();

  RecArgs &ra = plan->ra;
  ra.T = T; ra.B = B; ra.H = H; ra.KS = (H + 63) / 64;
  v4i *rfrag = reinterpret_cast<v4i *>(wsb + ws.rfrag);
  plan->stepped = needs_stepped(*params) || std::getenv("RXMET_FWD_STEPPED") != nullptr;
  if (!plan->stepped) {
    hipLaunchKernelGGL(pack_r_frags, dim3((H / 16) * 3 * ra.KS), dim3(64), 0, stream, H, ra.KS,
                       d.R_q, rfrag);
    RXMET_CHECK_LAUNCH();
  }
  ra.training = training ? 1 : 0;
  const rxmet_grid &gh = g[RXMET_GRU_H];
  const bool h_uns = gh.bits < 32 && gh.is_unsigned;
  ra.h_offset = h_uns ? std::ldexp(1.0f, gh.bits - 1) : 0.0f;
  plan->npl = (gh.bits <= 8) ? 1 : 2;
  {
    // bound of |R_q h| over the h grid and the R grid
    const Bounds brq = bounds_of(params->chan_bits[RXMET_GRU_R], params->chan_unsigned[RXMET_GRU_R]);
    const double rmax = std::max(std::fabs(brq.lo), std::fabs(brq.hi));
    const Bounds bhq = bounds_of(gh.bits, gh.is_unsigned);
    const double hmax = std::max(std::fabs(bhq.lo), std::fabs(bhq.hi));
    ra.wide_acc = hmax * rmax * H >= 2147483648.0 ? 1 : 0;
  }
  ra.gih = gih; ra.rfrag = rfrag; ra.chan = chan; ra.h0codes = h0codes; ra.hout = d.h; ra.v = d.v;
  ra.ih_m = d.ih_mask; ra.hh_m = d.hh_mask; ra.gin_m = d.gate_in_mask;
  ra.gout_m = d.gate_out_mask; ra.h_m = d.h_mask;
  ra.vc = nullptr; ra.mb = nullptr;
  if (training && codes) {
    ra.v = nullptr;
    ra.ih_m = ra.hh_m = ra.gin_m = ra.gout_m = ra.h_m = nullptr;
    ra.vc = codes->v_codes;
    ra.mb = codes->mask_bits;
  }
  ra.hx = reinterpret_cast<int8_t *>(wsb + ws.hx);
  {
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    bool wide = H % 16 == 0 && a16(ra.hout);
    if (training && ra.vc)
      wide = wide && a16(ra.vc) && a16(ra.mb);
    else if (training)
      wide = wide && a16(ra.v) && a16(ra.ih_m) && a16(ra.hh_m) && a16(ra.gin_m) &&
             a16(ra.gout_m) && a16(ra.h_m);
    ra.wide_out = wide ? 1 : 0;
  }
  plan->rq = d.R_q;
  plan->wsb = wsb;
  return 0;
}

// Clustered launch over every direction when the grid can be resident at once; returns 1
// when launched, 0 when the caller must use the per-tile recurrence.
static int forward_recurrence_clustered(FwdPlan *plans, int ndir, int T, int B, int I, int H,
                                        hipStream_t stream) {
  const int npl = plans[0].npl, KS = plans[0].ra.KS;
  for (int k = 1; k < ndir; ++k)
    if (plans[k].npl != npl) return 0;
  if (KS > 4 * kClMaxKPerWave || std::getenv("RXMET_NO_CLUSTER") != nullptr) return 0;
  // the exchange buffer (2 npl planes of Bpad KS 64 bytes) is addressed with 32-bit offsets
  if (2.0 * npl * ((B + kTileB - 1) / kTileB * kTileB) * KS * 64 >= 2147483648.0) return 0;
  const bool stage = H >= kStageMinH;
  int device = 0, ncu = 0;
  RXMET_CHECK_HIP(hipGetDevice(&device));
  RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
  ClArgs cl;
  cl.ndir = ndir;
  cl.ntiles = (B + kTileB - 1) / kTileB;
  cl.Bpad = cl.ntiles * kTileB;
  const int pairs = ndir * cl.ntiles;
  // the smallest unit slice per workgroup whose grid fits one workgroup per CU (two
  // workgroups sharing a CU step no faster than one doing both), else the largest slice
  int chosen = 0, ncl = 0;
  for (int UT = 1; UT <= 2 && !chosen; ++UT) {
    if ((H / 16) % UT) continue;
    // the staged h tile takes at most kHsMax chunks per thread
    if (H >= kStageMinH && npl * KS * 64 > kHsMax * 256 * UT) continue;
    const int G = H / (16 * UT);
    if (static_cast<int64_t>(pairs) * G <= ncu || UT == 2) {
      chosen = UT;
      cl.G = G;
    }
  }
  if (!chosen) return 0;
  // gate tables (unstaged kernel only) when every gate grid has at most kGateTabMax codes
  cl.gate_tab = stage ? 0 : 1;
  for (int k = 0; k < ndir; ++k) {
    const StepParams &sp = plans[k].sp;
    for (const Bounds &g : {sp.zin, sp.rin, sp.nin})
      if (!(g.hi - g.lo < static_cast<float>(kGateTabMax))) cl.gate_tab = 0;
  }
  const bool tab = cl.gate_tab != 0;
  const void *fn = npl == 1 ? (stage ? reinterpret_cast<const void *>(&recurrence_cl<1, true>)
                                     : reinterpret_cast<const void *>(&recurrence_cl<1, false>))
                            : (stage ? reinterpret_cast<const void *>(&recurrence_cl<2, true>)
                                     : reinterpret_cast<const void *>(&recurrence_cl<2, false>));
  const size_t lds_cl = recurrence_cl_lds_bytes(chosen, npl, H, tab);
  RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds_cl)));
  int per_cu = 0;
  RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256 * chosen, lds_cl));
  ncl = per_cu * ncu / cl.G;
  if (ncl < 1) return 0;
  if (ncl > pairs) ncl = pairs;
  if (ncl >= 8) ncl -= ncl % 8;
  cl.UT = chosen;
  cl.stage_h = stage ? 1 : 0;
  cl.ncl = ncl;
  const FwdWorkspace ws(T, B, I, H);
  cl.counters = reinterpret_cast<unsigned *>(plans[0].wsb + ws.sync);
  cl.timeout = reinterpret_cast<int *>(cl.counters + cluster::kCounterStride * ncl);
  cl.spin_limit = cluster::spin_limit();
  hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, cl.counters,
                     cluster::kCounterStride * ncl + 1);
  RXMET_CHECK_LAUNCH();
  RecArgs &a1 = plans[ndir > 1 ? 1 : 0].ra;
  // both directions' step parameters in device memory (read with scalar loads)
  StepParams host_ps[2] = {plans[0].sp, plans[ndir > 1 ? 1 : 0].sp};
  StepParams *ps = reinterpret_cast<StepParams *>(plans[0].wsb + ws.sparams);
  RXMET_CHECK_HIP(hipMemcpyAsync(ps, host_ps, sizeof(host_ps), hipMemcpyHostToDevice, stream));
  void *args[] = {&plans[0].ra, &a1, &ps, &cl};
  {
    rxmet::prof::Scope ps__("gru_fwd_recurrence", stream);
    RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * cl.G), dim3(256 * cl.UT), args,
                                               static_cast<unsigned>(lds_cl), stream));
  }
  // a wait that timed out: h and v of every direction become NaN
  cluster::PoisonList pl{};
  for (int k = 0; k < ndir; ++k) {
    pl.p[pl.count] = plans[k].ra.hout;
    pl.n[pl.count++] = static_cast<int64_t>(T + 1) * B * H;
    if (plans[k].ra.v) {
      pl.p[pl.count] = plans[k].ra.v;
      pl.n[pl.count++] = static_cast<int64_t>(T) * B * 4 * H;
    }
  }
  hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, cl.timeout, pl);
  RXMET_CHECK_LAUNCH();
  return 1;
}

// The stepped recurrence of one direction: 2 T launches.
static int forward_recurrence_stepped(FwdPlan &plan, const rxmet_gru_qparams &params, int T, int B,
                                      int I, int H, hipStream_t stream) {
  const int C = 3 * H;
  const FwdWorkspace ws(T, B, I, H);
  float *hb = reinterpret_cast<float *>(plan.wsb + ws.sh);
  float *ghh = reinterpret_cast<float *>(plan.wsb + ws.sg);
  const Bounds bh = bounds_of(params.g[RXMET_GRU_H].bits, params.g[RXMET_GRU_H].is_unsigned);
  const Bounds br = bounds_of(params.chan_bits[RXMET_GRU_R], params.chan_unsigned[RXMET_GRU_R]);
  RXMET_CHECK_ARG(xgemm::a_fits(bh.lo, bh.hi), "h codes must span at most 16 bits");
  const int pa = xgemm::a_planes(bh.lo, bh.hi), pb = xgemm::b_planes(br.lo, br.hi);
  xgemm::Operands o{};
  o.M = B; o.N = C; o.K = H;
  o.lda = H;
  o.off = xgemm::a_shift(bh.lo, bh.hi);
  o.corr = static_cast<long long>(o.off);  // raw codes: base 0
  o.sbk = C; o.sbn = 1;
  const dim3 ggrid((B + xgemm::kTile - 1) / xgemm::kTile, (C + xgemm::kTile - 1) / xgemm::kTile);
  const int64_t n = static_cast<int64_t>(B) * H;
  const dim3 pgrid(static_cast<unsigned>((n + 255) / 256));
  rxmet::prof::Scope ps__("gru_fwd_recurrence", stream);
  const float *hcur = plan.ra.h0codes;
  for (int t = 0; t < T; ++t) {
    float *hnext = hb + static_cast<size_t>(t & 1) * n;
    o.A = hcur;
    o.B = plan.rq;
    if (pa == 1 && pb == 1)
      hipLaunchKernelGGL((step_rh_gemm<1, 1>), ggrid, dim3(256), 0, stream, o, ghh);
    else if (pa == 1)
      hipLaunchKernelGGL((step_rh_gemm<1, 2>), ggrid, dim3(256), 0, stream, o, ghh);
    else if (pb == 1)
      hipLaunchKernelGGL((step_rh_gemm<2, 1>), ggrid, dim3(256), 0, stream, o, ghh);
    else
      hipLaunchKernelGGL((step_rh_gemm<2, 2>), ggrid, dim3(256), 0, stream, o, ghh);
    RXMET_CHECK_LAUNCH();
    hipLaunchKernelGGL(step_point, pgrid, dim3(256), 0, stream, plan.ra, plan.sp, t, ghh, hcur,
                       hnext);
    RXMET_CHECK_LAUNCH();
    hcur = hnext;
  }
  return 0;
}

static int forward_recurrence_tiles(FwdPlan &plan, int B, int H, hipStream_t stream) {
  RecArgs &ra = plan.ra;
  const size_t lds = recurrence_lds_bytes(H, ra.KS, plan.npl);
  const dim3 grid((B + kTileB - 1) / kTileB), block(64 * ((H + 31) / 32));
  const void *fn = plan.npl == 1 ? reinterpret_cast<const void *>(&recurrence<1>)
                                 : reinterpret_cast<const void *>(&recurrence<2>);
  RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
  rxmet::prof::Scope ps__("gru_fwd_recurrence", stream);
  if (plan.npl == 1)
    hipLaunchKernelGGL(recurrence<1>, grid, block, lds, stream, ra, plan.sp);
  else
    hipLaunchKernelGGL(recurrence<2>, grid, block, lds, stream, ra, plan.sp);
  RXMET_CHECK_LAUNCH();
  return 0;
}

static int forward_dirs(int ndir, bool training, int T, int B, int I, int H,
                        const rxmet_gru_fwd_dir *dirs, const int64_t *x_layout,
                        hipStream_t stream, const rxmet_gru_saved_codes *codes = nullptr) {
  RXMET_CHECK_ARG(ndir == 1 || ndir == 2, "ndir must be 1 or 2");
  RXMET_CHECK_ARG(dirs != nullptr, "dirs must be non-null");
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H % 16 == 0 && H <= 64 * 4 * kClMaxKPerWave,
                  "hidden_size must be a multiple of 16 and at most 1024");
  RXMET_CHECK_ARG(static_cast<double>(T + 1) * B * 4 * H < 4294967295.0,
                  "T*B*H too large for the recurrence's 32-bit element offsets");
  FwdPlan plans[2];
  for (int k = 0; k < ndir; ++k) {
    XLayout xl{static_cast<int64_t>(B) * I, I, 0, 0};
    if (x_layout) {
      xl = XLayout{x_layout[4 * k], x_layout[4 * k + 1], x_layout[4 * k + 2] != 0 ? 1 : 0,
                   (x_layout[4 * k + 3] & 1) != 0 ? 1 : 0};
      RXMET_CHECK_ARG(static_cast<double>(T) * B * I < 4294967295.0 && xl.st >= 0 && xl.sb >= 0,
                      "strided x: T*B*I must be below 2^32 and the strides non-negative");
    }
    if (int rc = forward_prologue(training, T, B, I, H, dirs[k], xl, codes ? &codes[k] : nullptr,
                                  stream, &plans[k]))
      return rc;
  }
  bool stepped = false;
  for (int k = 0; k < ndir; ++k) stepped = stepped || plans[k].stepped;
  if (stepped) {
    for (int k = 0; k < ndir; ++k)
      if (int r = forward_recurrence_stepped(plans[k], *dirs[k].params, T, B, I, H, stream)) return r;
    return 0;
  }
  const int rc = forward_recurrence_clustered(plans, ndir, T, B, I, H, stream);
  if (rc < 0) return rc;
  if (rc == 1) return 0;
  RXMET_CHECK_ARG(H <= kMaxH,
                  "hidden_size above 256 needs the clustered recurrence (cooperative launch)");
  for (int k = 0; k < ndir; ++k)
    if (int r = forward_recurrence_tiles(plans[k], B, H, stream)) return r;
  return 0;
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int64_t rxmet_gru_forward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  if (T < 0 || B < 0 || I < 0 || H < 0) return 0;
  return static_cast<int64_t>(FwdWorkspace(T, B, I, H).total);
}

int rxmet_gru_forward_quant(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                            const float *W, const float *R, const float *bw, const float *br,
                            const float *x, const float *h0, const rxmet_gru_qparams *params,
                            float *h, float *v, float *W_q, float *R_q, float *bw_q, float *br_q,
                            float *x_q, uint8_t *x_mask, uint8_t *h0_mask, uint8_t *W_mask,
                            uint8_t *R_mask, uint8_t *bw_mask, uint8_t *br_mask, uint8_t *ih_mask,
                            uint8_t *hh_mask, uint8_t *gate_in_mask, uint8_t *gate_out_mask,
                            uint8_t *h_mask, void *workspace, void *stream_) {
  clear_error();
  const rxmet_gru_fwd_dir d = {W, R, bw, br, x, h0, params, h, v, W_q, R_q, bw_q, br_q, x_q,
                               x_mask, h0_mask, W_mask, R_mask, bw_mask, br_mask, ih_mask,
                               hh_mask, gate_in_mask, gate_out_mask, h_mask, workspace};
  return forward_dirs(1, is_training != 0, T, B, I, H, &d, nullptr, static_cast<hipStream_t>(stream_));
}

int rxmet_gru_forward_quant_dirs(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                 int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                 void *stream_) {
  clear_error();
  return forward_dirs(ndir, is_training != 0, T, B, I, H, dirs, nullptr,
                      static_cast<hipStream_t>(stream_));
}

int rxmet_gru_forward_quant_dirs_x(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                   int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                   const int64_t *x_layout, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(x_layout != nullptr, "x_layout must be non-null");
  return forward_dirs(ndir, is_training != 0, T, B, I, H, dirs, x_layout,
                      static_cast<hipStream_t>(stream_));
}

int rxmet_gru_forward_quant_dirs_codes(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                       int32_t I, int32_t H, const rxmet_gru_fwd_dir *dirs,
                                       const int64_t *x_layout, const rxmet_gru_saved_codes *codes,
                                       void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(codes != nullptr || !is_training, "codes must be non-null in training");
  return forward_dirs(ndir, is_training != 0, T, B, I, H, dirs, x_layout,
                      static_cast<hipStream_t>(stream_), is_training ? codes : nullptr);
}

}  // extern "C"
