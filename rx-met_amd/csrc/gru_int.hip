// gru_int.hip — MI355X QuantGRU forward on the int32 carrier, behind
// rxmet_gru_forward_quant_int (forward_quant_int_storage) and rxmet_gru_forward_int_io
// (forward_quantized_int_io).
//
// Reference path: quantGRUForwardInt / quantGRUForwardIntIO (operators/quant-gru/src/
// gru_interface.cc:384-627) over ForwardPassQuant (src/gru_forward_gpu_quant.cu): per-channel
// weight quantisation, x/h0 quantisation, one tiled int64 GEMM+bias kernel for the input
// projection, then a host loop of T steps each launching a tiled GEMM+bias kernel for R h and
// the integer pointwise kernel, and dequantisation passes over h and v.  Every value between
// the boundaries is an integer code; rescales are rshift_round(x M, shift) with a 16-bit
// mantissa M (or a pure shift in power-of-two mode) and activations are 16-segment PWL tables on
// codes.
//
// Here:
//   1. iq_weights : W/R/bw/br -> int32 codes + masks in one pass, plus the two bias terms
//      rescaled into each GEMM's accumulator scale;
//   2. iq_input   : x -> int32 codes + mask, h0 -> codes of row 0 (+ mask, + dequantised h[0]);
//   3. wx_gemm    : the time-parallel input projection summed exactly on int8 MFMA over
//      byte planes (exact_gemm.h, int32 operands), with the GEMM+bias rescale, clamp and mask
//      fused into the epilogue;
//   4. the recurrence, clustered (int_recurrence_cl; cluster.h) when R_q fits signed 8 bits,
//      H is a multiple of 16 and H <= 1024: one cooperative launch for all T steps, a batch
//      tile's hidden units split over a cluster of workgroups, R_q resident in VGPRs as int8
//      MFMA fragments, the h codes exchanged as byte planes each step, and the recurrent
//      linear's bias, rescale and clamp plus the integer gates fused in registers.  Otherwise
//      per step rh_gemm (the same GEMM for R_q (h - zp_h)) and int_point: the integer update,
//      reset and new gates, the hidden update, clamps and masks, the dequantised h and v.
#include <climits>
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
namespace {

// rshift_round (include/quantize_ops_helper.h:201-224): round(x / 2^n), ties to even, on |x|;
// a left shift for n <= 0.  Shifts lie in [-32, 62] (checked on the host).
__device__ __forceinline__ long long rshift_round(long long x, int n) {
  if (n <= 0) return static_cast<long long>(static_cast<unsigned long long>(x) << (-n));
  const bool neg = x < 0;
  const unsigned long long ax =
      neg ? 0ull - static_cast<unsigned long long>(x) : static_cast<unsigned long long>(x);
  const unsigned long long q = ax >> n, r = ax & ((1ull << n) - 1ull), half = 1ull << (n - 1);
  const unsigned long long res = r > half ? q + 1ull : (r < half ? q : q + (q & 1ull));
  return neg ? -static_cast<long long>(res) : static_cast<long long>(res);
}

__device__ __forceinline__ long long rescale(long long x, IRescale r) {
  return rshift_round(x * static_cast<long long>(r.mult), r.shift);
}

// int32 addition with two's-complement wrap (the reference adds int32 values).
__device__ __forceinline__ int32_t add32(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}

__device__ __forceinline__ int32_t clampi(int32_t v, IGrid g, uint8_t &keep) {
  keep = (v < g.lo || v > g.hi) ? 0 : 1;
  return v < g.lo ? g.lo : (v > g.hi ? g.hi : v);
}

// quantize(float, FixedPointScale, zp, bw) (quantize_ops_helper.h:356-364, 472-476): rint of
// the quotient in fp32, the zero point added in double, saturated before the conversion.
__device__ __forceinline__ int32_t quant_i(float v, float eff, int32_t zp, IGrid g,
                                           uint8_t &keep) {
  const double code = static_cast<double>(rintf(v / eff)) + static_cast<double>(zp);
  keep = (code < g.lo || code > g.hi) ? 0 : 1;
  return code < g.lo ? g.lo : (code > g.hi ? g.hi : static_cast<int32_t>(code));
}

// piecewise_linear_raw (quantize_ops_helper.h:503-535) over a table in LDS.
__device__ __forceinline__ int32_t pwl_i(int32_t q, const ILut &l) {
  int s = kSegments - 1;
#pragma unroll
  for (int i = kSegments - 1; i >= 0; --i)
    if (q < l.thr[i]) s = i;
  const long long bx = static_cast<long long>(l.qb[s]) *
                       static_cast<long long>(static_cast<int32_t>(static_cast<uint32_t>(q) -
                                                                   static_cast<uint32_t>(l.zp_x)));
  const int n = l.n[s];
  const int32_t term =
      n >= 0 ? static_cast<int32_t>(rshift_round(bx, n))
             : static_cast<int32_t>(static_cast<long long>(static_cast<unsigned long long>(bx) << (-n)));
  return add32(term, l.c[s]);
}

// ---------------------------------------------------------------------------------
// 1. weights
// ---------------------------------------------------------------------------------
struct IWeightArgs {
  const float *W, *R, *bw, *br;  // [I, 3H], [H, 3H], [3H], [3H]
  const float *eff;              // [4][3H] effective scales of W, R, bw, br
  const IRescale *rs;            // [4][3H] channel rescales (gemm_x, bw, gemm_h, br)
  IGrid gW, gR, gbw, gbr;
  int32_t *Wq, *Rq, *bwq, *brq;
  uint8_t *Wm, *Rm, *bwm, *brm;
  long long *bias;  // [2][3H]: bw and br in their GEMM's accumulator scale
};

__global__ __launch_bounds__(256) void iq_weights(int I, int H, IWeightArgs a) {
  const int C = 3 * H;
  const int64_t nW = static_cast<int64_t>(I) * C, nR = static_cast<int64_t>(H) * C;
  const int64_t total = nW + nR + C;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    uint8_t keep;
    if (i < nW) {
      const int c = static_cast<int>(i % C);
      a.Wq[i] = quant_i(a.W[i], a.eff[c], 0, a.gW, keep);
      if (a.Wm) a.Wm[i] = keep;
    } else if (i < nW + nR) {
      const int64_t j = i - nW;
      const int c = static_cast<int>(j % C);
      a.Rq[j] = quant_i(a.R[j], a.eff[C + c], 0, a.gR, keep);
      if (a.Rm) a.Rm[j] = keep;
    } else {
      const int c = static_cast<int>(i - nW - nR);
      const int32_t qb = quant_i(a.bw[c], a.eff[2 * C + c], 0, a.gbw, keep);
      a.bwq[c] = qb;
      if (a.bwm) a.bwm[c] = keep;
      const int32_t qr = quant_i(a.br[c], a.eff[3 * C + c], 0, a.gbr, keep);
      a.brq[c] = qr;
      if (a.brm) a.brm[c] = keep;
      a.bias[c] = rescale(qb, a.rs[C + c]);
      a.bias[C + c] = rescale(qr, a.rs[3 * C + c]);
    }
  }
}

// ---------------------------------------------------------------------------------
// 2. inputs
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void iq_input(int64_t nx, int64_t nh, const float *x,
                                                const float *h0, const int32_t *h0q,
                                                IntStepParams p, int32_t *xq, uint8_t *xm,
                                                int32_t *hq0, uint8_t *h0m, float *hout0) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nx + nh;
       i += stride) {
    uint8_t keep;
    if (i < nx) {
      xq[i] = quant_i(x[i], p.eff_x, p.zp_x, p.x, keep);
      if (xm) xm[i] = keep;
    } else {
      const int64_t j = i - nx;
      int32_t q = p.zp_h;
      if (h0q) {
        q = h0q[j];
      } else if (h0) {
        q = quant_i(h0[j], p.eff_h, p.zp_h, p.h, keep);
        if (h0m) h0m[j] = keep;
      }
      hq0[j] = q;
      if (hout0)
        hout0[j] = static_cast<float>(static_cast<int32_t>(static_cast<uint32_t>(q) -
                                                           static_cast<uint32_t>(p.zp_h))) *
                   p.eff_h;
    }
  }
}

// Codes outside [lo, hi] set *flag (int-IO inputs must lie on their grids).
__global__ __launch_bounds__(256) void check_codes(const int32_t *a, int64_t n, int32_t lo,
                                                   int32_t hi, int *flag) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  bool bad = false;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    bad = bad || a[i] < lo || a[i] > hi;
  if (bad) atomicOr(flag, 1);
}

// ---------------------------------------------------------------------------------
// 3./4a. GEMM + bias + rescale + clamp (quantizedGemmBiasFused,
//        src/gru_forward_gpu_quant.cu:112-176) on exact int8-MFMA sums
// ---------------------------------------------------------------------------------
// S(m, c) = sum_k (A(m, k) - zp) B(k, c) exactly; out(m, c) = clamp(int32(rescale(S + bias[c],
// rs[c])) + zp_out), mask (1 = kept) when non-null.
struct LinearOut {
  const long long *bias;
  const IRescale *rs;
  int32_t zp_out;
  IGrid g;
  int32_t *out;
  uint8_t *mask;
  int ld;  // row stride of out and mask
};

__device__ __forceinline__ void linear_store(const LinearOut &e, int m, int c, long long s) {
  uint8_t keep;
  const int32_t v = clampi(add32(static_cast<int32_t>(rescale(s + e.bias[c], e.rs[c])), e.zp_out),
                           e.g, keep);
  const size_t i = static_cast<size_t>(m) * e.ld + c;
  e.out[i] = v;
  if (e.mask) e.mask[i] = keep;
}

template <int PA, int PB>
__global__ __launch_bounds__(256) void linear_gemm(xgemm::OperandsT<int32_t, int32_t> o,
                                                   LinearOut e) {
  xgemm::block<PA, PB>(o, blockIdx.y * xgemm::kTile, blockIdx.x * xgemm::kTile,
                       [&](int m, int n, long long s) { linear_store(e, m, n, s); });
}

constexpr int kPackedMaxK = 256;
template <int PA, int PB>
__global__ __launch_bounds__(256) void linear_gemm_packed(xgemm::Packed p, LinearOut e) {
  xgemm::rows16<PA, PB>(p, 16 * blockIdx.x, threadIdx.x / 64, 4,
                        [&](int m, int n, const long long *s, int rows) {
#pragma unroll
                          for (int r = 0; r < 4; ++r)
                            if (r < rows) linear_store(e, m + r, n, s[r]);
                        });
}

// ---------------------------------------------------------------------------------
// 4b. pointwise step (PointwiseOperationsQuant, src/gru_forward_gpu_quant.cu:230-373, with
//     computeUpdateGate / ResetGate / NewGate / HiddenState, quantize_ops_helper.h:683-1023)
// ---------------------------------------------------------------------------------
struct IPointArgs {
  int T, B, H;
  const int32_t *wx;  // [T, B, 3H] weight_ih_linear codes
  const int32_t *rh;  // [B, 3H] weight_hh_linear codes of the step
  float *hout;        // [T+1, B, H] dequantised h, or null
  float *v;           // [T, B, 4H] dequantised (z, r, n, weight_hh_linear n), or null
  uint8_t *gin_m, *gout_m, *h_m;  // training masks, or null
};

__device__ __forceinline__ float dq(int32_t q, int32_t zp, float eff) {
  return static_cast<float>(add32(q, -zp)) * eff;
}

__global__ __launch_bounds__(256) void int_point(IPointArgs a, IntStepParams p, int t,
                                                 const int32_t *hq, int32_t *hq_next) {
  __shared__ ILut lut[3];
  for (int i = threadIdx.x; i < 3 * static_cast<int>(sizeof(ILut) / 4); i += blockDim.x)
    reinterpret_cast<int32_t *>(lut)[i] = reinterpret_cast<const int32_t *>(p.lut)[i];
  __syncthreads();
  const int H = a.H, C = 3 * H;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<int64_t>(a.B) * H) return;
  const int b = static_cast<int>(e / H), j = static_cast<int>(e % H);
  const size_t n = static_cast<size_t>(t) * a.B + b;
  const int32_t *wx = a.wx + n * C;
  const int32_t *rh = a.rh + static_cast<size_t>(b) * C;
  const int32_t wz = wx[j], wr = wx[H + j], wn = wx[2 * H + j];
  const int32_t hz = rh[j], hr = rh[H + j], hn = rh[2 * H + j];
  uint8_t k_zi, k_zo, k_ri, k_ro, k_ni, k_no, k_h;
  // update gate
  int32_t in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wz) - p.zp_wx, p.ih_zin)),
                           static_cast<int32_t>(rescale(static_cast<long long>(hz) - p.zp_rh, p.hh_zin))),
                     p.zp_zin);
  in = clampi(in, p.zin, k_zi);
  const int32_t z = clampi(pwl_i(in, lut[0]), p.zout, k_zo);
  // reset gate
  in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wr) - p.zp_wx, p.ih_rin)),
                   static_cast<int32_t>(rescale(static_cast<long long>(hr) - p.zp_rh, p.hh_rin))),
             p.zp_rin);
  in = clampi(in, p.rin, k_ri);
  const int32_t r = clampi(pwl_i(in, lut[1]), p.rout, k_ro);
  // new gate: r times the weight_hh_linear code of n, aligned to new_gate_input in one rescale
  const long long rmul = (static_cast<long long>(r) - p.zp_rout) * (static_cast<long long>(hn) - p.zp_rh);
  in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wn) - p.zp_wx, p.ih_nin)),
                   static_cast<int32_t>(rescale(rmul, p.rmul_nin))),
             p.zp_nin);
  in = clampi(in, p.nin, k_ni);
  const int32_t nn = clampi(pwl_i(in, lut[2]), p.nout, k_no);
  // hidden update: u h_old + (1 - u) n on the scale S_zout S_h, one rescale to h
  const int32_t hold = hq[e];
  const int32_t n_h = add32(static_cast<int32_t>(rescale(static_cast<long long>(nn) - p.zp_nout, p.nout_h)), p.zp_h);
  const long long oldc = (static_cast<long long>(z) - p.zp_zout) * (static_cast<long long>(hold) - p.zp_h);
  const long long newc = (static_cast<long long>(p.quant_one) - z) * (static_cast<long long>(n_h) - p.zp_h);
  const int32_t hnew = clampi(add32(static_cast<int32_t>(rescale(oldc + newc, p.old_h)), p.zp_h), p.h, k_h);
  hq_next[e] = hnew;
  const size_t NH = static_cast<size_t>(a.B) * H;
  if (a.hout) a.hout[(static_cast<size_t>(t) + 1) * NH + e] = dq(hnew, p.zp_h, p.eff_h);
  if (a.v) {
    float *vp = a.v + n * 4 * H + j;
    vp[0] = dq(z, p.zp_zout, p.eff_zout);
    vp[H] = dq(r, p.zp_rout, p.eff_rout);
    vp[2 * H] = dq(nn, p.zp_nout, p.eff_nout);
    vp[3 * H] = dq(hn, p.zp_rh, p.eff_rh);
  }
  if (a.gin_m) {
    const size_t mi = n * C + j;
    a.gin_m[mi] = k_zi;
    a.gin_m[mi + H] = k_ri;
    a.gin_m[mi + 2 * H] = k_ni;
    a.gout_m[mi] = k_zo;
    a.gout_m[mi + H] = k_ro;
    a.gout_m[mi + 2 * H] = k_no;
    a.h_m[static_cast<size_t>(t) * NH + e] = k_h;
  }
}

// ---------------------------------------------------------------------------------
// 4c. clustered recurrence: a batch tile's units split over G workgroups
// ---------------------------------------------------------------------------------
// Member m of a cluster owns UT unit tiles (16 units each) of one 16-sequence batch tile.
// Four waves per unit tile split the recurrent sum over the K-steps (wave q takes steps
// q, q+4, ...) with R_q fragments resident in VGPRs and add their partial sums through LDS;
// each lane then finishes one (sequence, unit) element: the three weight_hh_linear codes from
// the exact sums, the gates and the new h code.  The h codes are exchanged through global
// memory as byte planes (coherent accesses, double-buffered by step parity) and the members
// meet at a counter barrier once per step.
constexpr int kITile = 16;
constexpr int kIMaxKPerWave = 4;  // K-steps per wave: H <= 1024

// One direction of the clustered recurrence.
struct IClDir {
  int h_offset;                 // 0 (signed h grid) or 2^(bits-1) (unsigned): centred codes
  int gate_tab;                 // gate activations by table (every gate grid fits)
  const int32_t *wx;            // [T, B, 3H] weight_ih_linear codes
  const v4i *rfrag;             // R_q as int8 MFMA B fragments, [H/16][3][KS][64]
  const int32_t *rcol;          // [3H] column sums of R_q
  const long long *bias;        // [3H] br in the recurrent accumulator's scale
  const IRescale *rs;           // [3H] recurrent accumulator -> weight_hh_linear
  const int32_t *h0q;           // [B, H] h codes of row 0
  float *hout, *v;              // dequantised h [T+1, B, H] (row 0 written) and v, or null
  int32_t *hq;                  // h codes [T+1, B, H] (row 0 written), or null
  uint8_t *hh_m, *gin_m, *gout_m, *h_m;  // training masks, or null
  int8_t *hx;                   // [2][NPL][Bpad / 16][KS][16][64] exchanged h codes (see ihx_offset)
};

// The launch: clusters walk (direction, batch tile) pairs, so both directions of a
// bidirectional layer run in one launch and their sequential steps overlap.
struct IClArgs {
  int T, B, H, KS, Bpad;
  int G, UT, ncl, ntiles, ndir;
  unsigned *counters;           // [ncl], kCounterStride words apart
  int *timeout;
  unsigned spin_limit;  // polls before a wait gives up (cluster::spin_limit())
};

// Gate activations by table: a gate input is clamped to its grid, so when the grid has at most
// kIGateTabMax codes the recurrence tabulates clampi(pwl_i(lo + e), out grid) once per launch
// (value * 2 | keep of the output clamp per entry): one LDS read per gate and step.
constexpr int kIGateTabMax = 1024;

// R_q [H][3H] int32 codes -> int8 B fragments of v_mfma_i32_16x16x64_i8:
// frag[((ut * 3 + g) * KS + s) * 64 + lane] holds R[k][c] for c = g*H + 16*ut + lane % 16,
// k = 64*s + 16*(lane / 16) + 0..15 (zero beyond H).  Each lane also adds its 16 codes to the
// column sum rcol[c] (zeroed beforehand; integer atomics, so the sum is exact in any order).
__global__ __launch_bounds__(64) void pack_r_frags_i32(int H, int KS, const int32_t *__restrict__ Rq,
                                                       v4i *__restrict__ frag,
                                                       int32_t *__restrict__ rcol) {
  const int lane = threadIdx.x;
  const int idx = blockIdx.x;  // (ut * 3 + g) * KS + s
  const int s = idx % KS, g = (idx / KS) % 3, ut = idx / (3 * KS);
  const int C = 3 * H;
  const int c = g * H + 16 * ut + lane % 16;
  int wd[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int by[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 64 * s + 16 * (lane / 16) + 4 * q + e;
      by[e] = k < H ? Rq[static_cast<size_t>(k) * C + c] : 0;
      sum += by[e];
    }
    wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
  }
  frag[static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
  atomicAdd(rcol + c, sum);
}

// h codes as exchanged bytes: one plane (the centred code) or two (low byte - 128, high byte)
// Byte offset of (row b, unit j) in one plane of the exchange buffer: 1 KB blocks of 16 rows x
// 64 units, one per (batch tile, K-step), so that a wave reads an MFMA A fragment as contiguous
// bytes.
__device__ __forceinline__ unsigned ihx_offset(int b, int j, int KS) {
  return ((static_cast<unsigned>(b / kITile) * KS + j / 64) * kITile + b % kITile) * 64 + j % 64;
}

template <int NPL>
__device__ __forceinline__ void publish_h(int8_t *hx, unsigned plane_stride, int b, int KS, int j,
                                          int hcv) {
  unsigned char *dst = reinterpret_cast<unsigned char *>(hx) + ihx_offset(b, j, KS);
#pragma unroll
  for (int q = 0; q < NPL; ++q)
    cluster::store_bytes_coherent(dst + q * plane_stride,
                                  NPL == 1 ? hcv : (q == 0 ? (hcv & 255) - 128 : hcv >> 8));
}

// One (direction, batch tile) pair of the launch: the direction's LUT, gate tables and R_q
// fragments are loaded, then its T steps run.
template <int NPL>
__device__ __forceinline__ void int_cl_pair(const IClDir &a, const IntStepParams &p,
                                            const IClArgs &s, int tile, int member,
                                            unsigned *counter, unsigned &epoch, bool &alive,
                                            unsigned char *smem) {
  ILut *lut = reinterpret_cast<ILut *>(smem);
  v4i *red = reinterpret_cast<v4i *>(smem + (3 * sizeof(ILut) + 15) / 16 * 16);  // [UT][4][3][NPL][64]
  int32_t *gtab = reinterpret_cast<int32_t *>(red + static_cast<size_t>(s.UT) * 4 * 3 * NPL * 64);
  const int H = s.H, C = 3 * H, B = s.B, KS = s.KS;
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int utl = w / 4, kq = w % 4;
  const int ut = member * s.UT + utl;
  const int j = 16 * ut + l % 16;
  const int nr = 4 * (l / 16) + kq;  // batch row finished by this lane
  for (int i = tid; i < 3 * static_cast<int>(sizeof(ILut) / 4); i += blockDim.x)
    reinterpret_cast<int32_t *>(lut)[i] = reinterpret_cast<const int32_t *>(p.lut)[i];
  if (a.gate_tab) {
    __syncthreads();  // the LUT is in LDS; the tables are read after the first cluster barrier
    for (int i = tid; i < 3 * kIGateTabMax; i += blockDim.x) {
      const int g = i / kIGateTabMax, e = i % kIGateTabMax;
      // selected, not indexed: a local array indexed by g would live in scratch memory
      const IGrid gi = g == 0 ? p.zin : (g == 1 ? p.rin : p.nin);
      const IGrid go = g == 0 ? p.zout : (g == 1 ? p.rout : p.nout);
      if (e <= gi.hi - gi.lo) {
        uint8_t k = 0;
        const int32_t v = clampi(pwl_i(gi.lo + e, lut[g]), go, k);
        gtab[i] = v * 2 | k;
      }
    }
  }
  // gate g of input code q (clamped to its grid): output code and output-clamp keep flag
  auto gate = [&](int g, int32_t q, const IGrid &gi, const IGrid &go, uint8_t &keep) -> int32_t {
    if (a.gate_tab) {
      const int32_t e = gtab[g * kIGateTabMax + (q - gi.lo)];
      keep = static_cast<uint8_t>(e & 1);
      return e >> 1;
    }
    return clampi(pwl_i(q, lut[g]), go, keep);
  };
  v4i rfr[kIMaxKPerWave][3];
#pragma unroll
  for (int i = 0; i < kIMaxKPerWave; ++i) {
    const int ks = kq + 4 * i;
#pragma unroll
    for (int g = 0; g < 3; ++g)
      rfr[i][g] = ks < KS ? a.rfrag[((ut * 3 + g) * KS + ks) * 64 + l] : v4i{0, 0, 0, 0};
  }
  // S = sum_k R (h - zp_h) = (plane sums) + (centring - zp_h) colsum
  const long long centre = (NPL == 2 ? 128 : 0) + a.h_offset - p.zp_h;
  long long rc[3], bias[3];
  IRescale rs[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    const int c = g * H + j;
    rc[g] = centre * a.rcol[c];
    bias[g] = a.bias[c];
    rs[g] = a.rs[c];
  }
  const unsigned plane_stride = static_cast<unsigned>(s.Bpad) * KS * 64;
  // the exchange buffer, 2 NPL planes (32-bit byte offsets: checked by the launcher)
  const auto xr = cluster::buffer_rsrc(a.hx, 2u * NPL * plane_stride);
  const size_t NH = static_cast<size_t>(B) * H;
  v4i *myred = red + (static_cast<size_t>(utl) * 4 + kq) * 3 * NPL * 64;
  {
    const int b0 = tile * kITile, b = b0 + nr;
    const bool valid = b < B;
    int32_t hold = valid ? a.h0q[static_cast<size_t>(b) * H + j] : p.zp_h;
    publish_h<NPL>(a.hx, plane_stride, b, KS, j, hold - a.h_offset);
    int32_t wn_[3];
    auto load_wx = [&](int t) {
#pragma unroll
      for (int g = 0; g < 3; ++g)
        wn_[g] = valid ? a.wx[(static_cast<size_t>(t) * B + b) * C + g * H + j] : 0;
    };
    load_wx(0);
    alive = cluster::sync(counter, ++epoch * s.G, s.timeout, s.spin_limit);
    for (int t = 0; t < s.T && alive; ++t) {
      const int par = t & 1;
      const unsigned hin = par * NPL * plane_stride;  // byte offset of the step's planes
      int8_t *hnext = a.hx + (par ^ 1) * NPL * plane_stride;
      const int32_t wz = wn_[0], wr = wn_[1], wn = wn_[2];
      v4i acc[3][NPL];
#pragma unroll
      for (int g = 0; g < 3; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) acc[g][q] = v4i{0, 0, 0, 0};
      {
        // lane l: row l % 16, units 16 (l / 16) .. + 15 of K-step kq + 4 i
        const unsigned hrow = hin + static_cast<unsigned>(tile) * KS * 1024 + 64 * (l % 16) + 16 * (l / 16);
        v4i hfr[kIMaxKPerWave][NPL];
#pragma unroll
        for (int i = 0; i < kIMaxKPerWave; ++i)
#pragma unroll
          for (int q = 0; q < NPL; ++q)
            if (kq + 4 * i < KS) {
              const int4 v = cluster::load_coherent16(xr, hrow + q * plane_stride + 1024 * (kq + 4 * i));
              hfr[i][q] = v4i{v.x, v.y, v.z, v.w};
            }
#pragma unroll
        for (int i = 0; i < kIMaxKPerWave; ++i)
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
      // the three weight_hh_linear codes of (row b, unit j)
      int32_t rh[3];
      uint8_t k_hh[3];
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        long long ps[NPL];
#pragma unroll
        for (int q = 0; q < NPL; ++q) {
          int v = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int *src = reinterpret_cast<const int *>(
                red + ((static_cast<size_t>(utl) * 4 + k) * 3 * NPL + g * NPL + q) * 64 + l);
            v += src[kq];
          }
          ps[q] = v;
        }
        const long long S = (NPL == 2 ? 256 * ps[NPL - 1] + ps[0] : ps[0]) + rc[g];
        rh[g] = clampi(add32(static_cast<int32_t>(rescale(S + bias[g], rs[g])), p.zp_rh), p.rh,
                       k_hh[g]);
      }
      // gates and the hidden update (as int_point)
      uint8_t k_zi, k_zo, k_ri, k_ro, k_ni, k_no, k_h;
      int32_t in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wz) - p.zp_wx, p.ih_zin)),
                               static_cast<int32_t>(rescale(static_cast<long long>(rh[0]) - p.zp_rh, p.hh_zin))),
                         p.zp_zin);
      in = clampi(in, p.zin, k_zi);
      const int32_t z = gate(0, in, p.zin, p.zout, k_zo);
      in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wr) - p.zp_wx, p.ih_rin)),
                       static_cast<int32_t>(rescale(static_cast<long long>(rh[1]) - p.zp_rh, p.hh_rin))),
                 p.zp_rin);
      in = clampi(in, p.rin, k_ri);
      const int32_t r = gate(1, in, p.rin, p.rout, k_ro);
      const long long rmul = (static_cast<long long>(r) - p.zp_rout) * (static_cast<long long>(rh[2]) - p.zp_rh);
      in = add32(add32(static_cast<int32_t>(rescale(static_cast<long long>(wn) - p.zp_wx, p.ih_nin)),
                       static_cast<int32_t>(rescale(rmul, p.rmul_nin))),
                 p.zp_nin);
      in = clampi(in, p.nin, k_ni);
      const int32_t nn = gate(2, in, p.nin, p.nout, k_no);
      const int32_t n_h = add32(static_cast<int32_t>(rescale(static_cast<long long>(nn) - p.zp_nout, p.nout_h)), p.zp_h);
      const long long oldc = (static_cast<long long>(z) - p.zp_zout) * (static_cast<long long>(hold) - p.zp_h);
      const long long newc = (static_cast<long long>(p.quant_one) - z) * (static_cast<long long>(n_h) - p.zp_h);
      const int32_t hnew = clampi(add32(static_cast<int32_t>(rescale(oldc + newc, p.old_h)), p.zp_h), p.h, k_h);
      hold = hnew;
      publish_h<NPL>(hnext, plane_stride, b, KS, j, hnew - a.h_offset);
      // the other members only read the h codes: arrive now, store the outputs while waiting
      cluster::arrive(counter);
      ++epoch;
      if (valid) {
        const size_t e = static_cast<size_t>(b) * H + j;
        const size_t row = (static_cast<size_t>(t) + 1) * NH + e;
        if (a.hq) a.hq[row] = hnew;
        if (a.hout) a.hout[row] = dq(hnew, p.zp_h, p.eff_h);
        const size_t n = static_cast<size_t>(t) * B + b;
        if (a.v) {
          float *vp = a.v + n * 4 * H + j;
          vp[0] = dq(z, p.zp_zout, p.eff_zout);
          vp[H] = dq(r, p.zp_rout, p.eff_rout);
          vp[2 * H] = dq(nn, p.zp_nout, p.eff_nout);
          vp[3 * H] = dq(rh[2], p.zp_rh, p.eff_rh);
        }
        if (a.hh_m) {
          const size_t mi = n * C + j;
          a.hh_m[mi] = k_hh[0];
          a.hh_m[mi + H] = k_hh[1];
          a.hh_m[mi + 2 * H] = k_hh[2];
        }
        if (a.gin_m) {
          const size_t mi = n * C + j;
          a.gin_m[mi] = k_zi;
          a.gin_m[mi + H] = k_ri;
          a.gin_m[mi + 2 * H] = k_ni;
          a.gout_m[mi] = k_zo;
          a.gout_m[mi + H] = k_ro;
          a.gout_m[mi + 2 * H] = k_no;
          a.h_m[static_cast<size_t>(t) * NH + e] = k_h;
        }
      }
      if (t + 1 < s.T) load_wx(t + 1);
      alive = cluster::wait(counter, epoch * s.G, s.timeout, s.spin_limit);
    }
  }
}

template <int NPL>
__global__ __launch_bounds__(512) void int_recurrence_cl(IClDir a0, IClDir a1,
                                                         const IntStepParams *__restrict__ ps,
                                                         IClArgs s) {
  extern __shared__ __align__(16) unsigned char smem[];
  const cluster::Place pl = cluster::place(s.G, s.ncl);
  unsigned *counter = s.counters + cluster::kCounterStride * pl.cluster;
  unsigned epoch = 0;
  bool alive = true;
  for (int pair = pl.cluster; pair < s.ndir * s.ntiles && alive; pair += s.ncl) {
    const int d = pair / s.ntiles, tile = pair % s.ntiles;
    // the previous pair's readers of the LUT, the gate tables and the partial-sum buffer are
    // done
    __syncthreads();
    int_cl_pair<NPL>(d == 0 ? a0 : a1, ps[d], s, tile, pl.member, counter, epoch, alive, smem);
  }
}

// A launch whose cluster wait timed out: the int32 h codes are overwritten with INT32_MIN
// (outside every grid) so that no caller mistakes them for a result.
__global__ __launch_bounds__(256) void poison_codes(const int *timeout, int64_t n, int32_t *p) {
  if (*timeout == 0) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = INT32_MIN;
}

// ---------------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------------
struct IntWorkspace {
  size_t hostblk, bias, wx, rh, hq, xa, bfrag, colsum, flag, rfrag, rcol, hx, sync, sparams,
      total;
  IntWorkspace(int T, int B, int I, int H) {
    const size_t C = 3 * static_cast<size_t>(H);
    const size_t Kp = static_cast<size_t>(xgemm::pad_k(I));
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t o = 0;
    hostblk = o; o += al(4 * C * (sizeof(float) + sizeof(IRescale)));
    bias = o; o += al(2 * C * sizeof(long long));
    wx = o; o += al(sizeof(int32_t) * static_cast<size_t>(T) * B * C);
    rh = o; o += al(sizeof(int32_t) * static_cast<size_t>(B) * C);
    hq = o; o += al(sizeof(int32_t) * 2 * static_cast<size_t>(B) * H);
    const size_t ip = static_cast<size_t>(I) <= kPackedMaxK ? 1 : 0;
    xa = o; o += al(ip * 2 * static_cast<size_t>(T) * B * Kp);
    bfrag = o; o += al(ip * 2 * ((C + 15) / 16 * 16) * Kp);  // fragments of 16-column tiles
    colsum = o; o += al(ip * sizeof(long long) * C);
    flag = o; o += al(sizeof(int));
    // clustered recurrence: R_q fragments, R_q column sums, the exchanged h planes, counters
    const size_t KS = (static_cast<size_t>(H) + 63) / 64;
    const size_t Bpad = (static_cast<size_t>(B) + kITile - 1) / kITile * kITile;
    rfrag = o; o += al(sizeof(v4i) * 64 * (static_cast<size_t>(H) / 16) * 3 * KS);
    rcol = o; o += al(sizeof(int32_t) * C);
    hx = o; o += al(2 * 2 * Bpad * KS * 64);
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (2 * Bpad / kITile + 2));  // counters of up to 2 directions
    sparams = o; o += al(2 * sizeof(IntStepParams));
    total = o;
  }
};

// A(m, k) codes with base zp (A spans at most 16 bits), B(k, c) signed 16-bit codes.
static int launch_linear(const int32_t *A, int lda, int M, int K, float off, long long corr,
                         int pa, const int32_t *Bm, int sbk, int N, int pb, const LinearOut &e,
                         char *packed_ws, const IntWorkspace &ws, hipStream_t stream) {
  if (packed_ws != nullptr && K <= kPackedMaxK) {
    const int Kp = xgemm::pad_k(K);
    int8_t *xa = reinterpret_cast<int8_t *>(packed_ws + ws.xa);
    v4i *bf = reinterpret_cast<v4i *>(packed_ws + ws.bfrag);
    long long *cs = reinterpret_cast<long long *>(packed_ws + ws.colsum);
    if (int rc = xgemm::pack_a(A, lda, M, K, off, pa, xa, Kp, stream)) return rc;
    if (int rc = xgemm::pack_b(Bm, sbk, 1, K, N, pb, Kp, bf, cs, stream)) return rc;
    xgemm::Packed p;
    p.A = xa; p.aplane = static_cast<int64_t>(M) * Kp; p.Kp = Kp;
    p.B = bf; p.bplane = static_cast<int64_t>((N + 15) / 16) * (Kp / 64) * 64;
    p.colsum = cs; p.corr = corr; p.M = M; p.N = N;
    const dim3 grid((M + 15) / 16);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p, e); };
    if (pa == 1)
      pb == 1 ? go(linear_gemm_packed<1, 1>) : go(linear_gemm_packed<1, 2>);
    else
      pb == 1 ? go(linear_gemm_packed<2, 1>) : go(linear_gemm_packed<2, 2>);
  } else {
    xgemm::OperandsT<int32_t, int32_t> o;
    o.M = M; o.N = N; o.K = K;
    o.A = A; o.lda = lda;
    o.off = off; o.corr = corr;
    o.B = Bm; o.sbk = sbk; o.sbn = 1;
    const dim3 grid((N + xgemm::kTile - 1) / xgemm::kTile, (M + xgemm::kTile - 1) / xgemm::kTile);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, o, e); };
    if (pa == 1)
      pb == 1 ? go(linear_gemm<1, 1>) : go(linear_gemm<1, 2>);
    else
      pb == 1 ? go(linear_gemm<2, 1>) : go(linear_gemm<2, 2>);
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}

struct IntCall {
  bool training;
  int T, B, I, H;
  const float *W, *R, *bw, *br, *x, *h0;
  const int32_t *xq_in, *h0q_in;  // int-IO inputs (x, h0 unused then)
  const rxmet_gru_qparams *params;
  float *h, *v;                                   // dequantised outputs, or null
  int32_t *hq_out;                                // int-IO: h codes [T+1, B, H], or null
  int32_t *Wq, *Rq, *bwq, *brq, *xq;              // codes (xq null for int-IO)
  uint8_t *x_m, *h0_m, *W_m, *R_m, *bw_m, *br_m, *ih_m, *hh_m, *gin_m, *gout_m, *h_m;
  void *workspace;
};

// One direction's call after its prologue (weights and inputs quantised, the input
// projection done): what the recurrence reads and writes.
struct IntPlan {
  IntCall k;
  IntStepParams sp;
  IWeightArgs wa;
  long long *bias;
  IRescale *rs;
  int32_t *wx, *rh, *hqb, *hq0;
  char *wsb;
};

// The clustered recurrence for ndir directions in one launch, when R_q fits signed 8 bits,
// h spans at most 16 bits (the same plane count in every direction), H is a multiple of 16 up
// to 1024 and the grid can be resident at once; returns 1 when launched, 0 when the caller
// must step, negative on error.
static int int_recurrence_clustered(IntPlan *plans, int ndir, hipStream_t stream) {
  const IntCall &k0 = plans[0].k;
  const int T = k0.T, B = k0.B, H = k0.H, C = 3 * H;
  if (H % 16 != 0 || H > 1024 || std::getenv("RXMET_NO_CLUSTER") != nullptr) return 0;
  const int npl = k0.params->g[RXMET_GRU_H].bits <= 8 ? 1 : 2;
  for (int d = 0; d < ndir; ++d) {
    const IGrid &gR = plans[d].wa.gR;
    if (gR.lo < -128 || gR.hi > 127) return 0;
    if ((plans[d].k.params->g[RXMET_GRU_H].bits <= 8 ? 1 : 2) != npl) return 0;
  }
  // the exchange buffer (2 npl planes of Bpad KS 64 bytes) is addressed with 32-bit offsets
  if (2.0 * npl * ((B + kITile - 1) / kITile * kITile) * ((H + 63) / 64 * 64) >= 2147483648.0) return 0;
  const void *fn = npl == 1 ? reinterpret_cast<const void *>(&int_recurrence_cl<1>)
                            : reinterpret_cast<const void *>(&int_recurrence_cl<2>);
  int device = 0, ncu = 0;
  RXMET_CHECK_HIP(hipGetDevice(&device));
  RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
  IClArgs s{};
  s.T = T; s.B = B; s.H = H; s.KS = (H + 63) / 64;
  s.ndir = ndir;
  s.ntiles = (B + kITile - 1) / kITile;
  s.Bpad = s.ntiles * kITile;
  const int pairs = ndir * s.ntiles;
  // the smallest unit slice per workgroup whose grid fits one workgroup per CU, else two tiles
  s.UT = (H / 16) % 2 == 0 && static_cast<int64_t>(pairs) * (H / 16) > ncu ? 2 : 1;
  s.G = H / (16 * s.UT);
  const size_t lds = (3 * sizeof(ILut) + 15) / 16 * 16 +
                     sizeof(v4i) * static_cast<size_t>(s.UT) * 4 * 3 * npl * 64 +
                     sizeof(int32_t) * 3 * kIGateTabMax;
  RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
  int per_cu = 0;
  RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256 * s.UT, lds));
  int ncl = per_cu * ncu / s.G;
  if (ncl < 1) return 0;
  if (ncl > pairs) ncl = pairs;
  if (ncl >= 8) ncl -= ncl % 8;
  s.ncl = ncl;
  const IntWorkspace ws(T, B, k0.I, H);
  IClDir dirs[2]{};
  IntStepParams host_ps[2];
  for (int d = 0; d < ndir; ++d) {
    IntPlan &pl = plans[d];
    const IntCall &k = pl.k;
    const rxmet_grid &gh = k.params->g[RXMET_GRU_H];
    IClDir &a = dirs[d];
    a.h_offset = gh.bits < 32 && gh.is_unsigned ? 1 << (gh.bits - 1) : 0;
    a.gate_tab = 1;
    for (const IGrid &g : {pl.sp.zin, pl.sp.rin, pl.sp.nin})
      if (static_cast<int64_t>(g.hi) - g.lo >= kIGateTabMax) a.gate_tab = 0;
    v4i *rfrag = reinterpret_cast<v4i *>(pl.wsb + ws.rfrag);
    int32_t *rcol = reinterpret_cast<int32_t *>(pl.wsb + ws.rcol);
    hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream,
                       reinterpret_cast<unsigned *>(rcol), C);
    RXMET_CHECK_LAUNCH();
    hipLaunchKernelGGL(pack_r_frags_i32, dim3((H / 16) * 3 * s.KS), dim3(64), 0, stream, H, s.KS,
                       k.Rq, rfrag, rcol);
    RXMET_CHECK_LAUNCH();
    a.wx = pl.wx;
    a.rfrag = rfrag;
    a.rcol = rcol;
    a.bias = pl.wa.bias + C;
    a.rs = pl.wa.rs + 2 * C;
    a.h0q = pl.hq0;
    a.hout = k.h;
    a.v = k.v;
    a.hq = k.hq_out;
    a.hh_m = k.training ? k.hh_m : nullptr;
    a.gin_m = k.training ? k.gin_m : nullptr;
    a.gout_m = k.training ? k.gout_m : nullptr;
    a.h_m = k.training ? k.h_m : nullptr;
    if (a.gin_m && !(a.gout_m && a.h_m)) a.gin_m = nullptr;
    a.hx = reinterpret_cast<int8_t *>(pl.wsb + ws.hx);
    host_ps[d] = pl.sp;
  }
  if (ndir == 1) {
    dirs[1] = dirs[0];
    host_ps[1] = host_ps[0];
  }
  // both directions' step parameters in device memory (read with scalar loads)
  IntStepParams *ps = reinterpret_cast<IntStepParams *>(plans[0].wsb + ws.sparams);
  if (int rc = upload(ps, host_ps, sizeof(host_ps), stream)) return rc;
  s.counters = reinterpret_cast<unsigned *>(plans[0].wsb + ws.sync);
  s.timeout = reinterpret_cast<int *>(s.counters + cluster::kCounterStride * ncl);
  s.spin_limit = cluster::spin_limit();
  hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, s.counters,
                     cluster::kCounterStride * ncl + 1);
  RXMET_CHECK_LAUNCH();
  void *args[] = {&dirs[0], &dirs[1], &ps, &s};
  {
    rxmet::prof::Scope ps__("gru_int_recurrence", stream);
    RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * s.G), dim3(256 * s.UT), args,
                                    static_cast<unsigned>(lds), stream));
  }
  // a wait that timed out: every output after row 0 becomes NaN (codes: INT32_MIN)
  const size_t NH = static_cast<size_t>(B) * H;
  cluster::PoisonList pl{};
  for (int d = 0; d < ndir; ++d) {
    const IntCall &k = plans[d].k;
    if (k.h) {
      pl.p[pl.count] = k.h + NH;
      pl.n[pl.count++] = static_cast<int64_t>(T) * NH;
    }
    if (k.v) {
      pl.p[pl.count] = k.v;
      pl.n[pl.count++] = static_cast<int64_t>(T) * NH * 4;
    }
  }
  if (pl.count) {
    hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, s.timeout, pl);
    RXMET_CHECK_LAUNCH();
  }
  for (int d = 0; d < ndir; ++d)
    if (plans[d].k.hq_out) {
      hipLaunchKernelGGL(poison_codes, dim3(256), dim3(256), 0, stream, s.timeout,
                         static_cast<int64_t>(T) * NH, plans[d].k.hq_out + NH);
      RXMET_CHECK_LAUNCH();
    }
  return 1;
}

// Checks, parameters, weight and input quantisation and the input projection of one
// direction.
static int prologue_int(const IntCall &k, hipStream_t stream, IntPlan &plan) {
  const int T = k.T, B = k.B, I = k.I, H = k.H;
  RXMET_CHECK_ARG(k.params != nullptr && k.workspace != nullptr, "params and workspace must be non-null");
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(k.params->hidden == H, "params.hidden != hidden_size");
  RXMET_CHECK_ARG(k.W && k.R && k.bw && k.br && k.Wq && k.Rq && k.bwq && k.brq,
                  "required pointer is null");
  RXMET_CHECK_ARG(I < (1 << 17) && H < (1 << 17), "input_size and hidden_size must be below 131072");
  RXMET_CHECK_ARG(static_cast<double>(T) * B * 3 * H < 9.0e18, "tensor too large");
  const rxmet_gru_qparams &P = *k.params;
  const rxmet_grid *g = P.g;
  {
    const IGrid gx = igrid_of(g[RXMET_GRU_X].bits, g[RXMET_GRU_X].is_unsigned);
    const IGrid gh = igrid_of(g[RXMET_GRU_H].bits, g[RXMET_GRU_H].is_unsigned);
    const IGrid gw = igrid_of(P.chan_bits[RXMET_GRU_W], P.chan_unsigned[RXMET_GRU_W]);
    const IGrid gr = igrid_of(P.chan_bits[RXMET_GRU_R], P.chan_unsigned[RXMET_GRU_R]);
    RXMET_CHECK_ARG(xgemm::a_fits(gx.lo, gx.hi) && xgemm::a_fits(gh.lo, gh.hi),
                    "x and h grids must span at most 16 bits");
    RXMET_CHECK_ARG(xgemm::b_fits(gw.lo, gw.hi) && xgemm::b_fits(gr.lo, gr.hi),
                    "W and R codes must fit signed 16 bits");
  }
  const int C = 3 * H;
  const IntWorkspace ws(T, B, I, H);
  char *wsb = static_cast<char *>(k.workspace);
  float *eff = reinterpret_cast<float *>(wsb + ws.hostblk);
  IRescale *rs = reinterpret_cast<IRescale *>(wsb + ws.hostblk + 4 * static_cast<size_t>(C) * sizeof(float));
  long long *bias = reinterpret_cast<long long *>(wsb + ws.bias);
  int32_t *wx = reinterpret_cast<int32_t *>(wsb + ws.wx);

  IntStepParams &sp = plan.sp;
  std::vector<char> host(4 * static_cast<size_t>(C) * (sizeof(float) + sizeof(IRescale)));
  try {
    make_int_step_params(P, H, &sp);
    float *he = reinterpret_cast<float *>(host.data());
    for (int kk = 0; kk < 4; ++kk)
      for (int c = 0; c < C; ++c) he[kk * C + c] = effective_scale(P.chan_scale[kk][c], P.use_pot2 != 0);
    make_int_channel_rescales(P, H, reinterpret_cast<IRescale *>(host.data() + 4 * static_cast<size_t>(C) * sizeof(float)));
  } catch (const std::exception &ex) {
    set_error(ex.what());
    return -22;
  }

  // int-IO inputs must lie on the x / h grids: checked once, with one stream synchronisation
  if (k.xq_in != nullptr) {
    int *flag = reinterpret_cast<int *>(wsb + ws.flag);
    hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(64), 0, stream,
                       reinterpret_cast<unsigned *>(flag), 1);
    RXMET_CHECK_LAUNCH();
    const int64_t nx = static_cast<int64_t>(T) * B * I;
    hipLaunchKernelGGL(check_codes, dim3(static_cast<unsigned>(std::min<int64_t>((nx + 255) / 256, 4096))),
                       dim3(256), 0, stream, k.xq_in, nx, sp.x.lo, sp.x.hi, flag);
    RXMET_CHECK_LAUNCH();
    if (k.h0q_in) {
      const int64_t nh = static_cast<int64_t>(B) * H;
      hipLaunchKernelGGL(check_codes, dim3(static_cast<unsigned>(std::min<int64_t>((nh + 255) / 256, 4096))),
                         dim3(256), 0, stream, k.h0q_in, nh, sp.h.lo, sp.h.hi, flag);
      RXMET_CHECK_LAUNCH();
    }
    int bad = 0;
    RXMET_CHECK_HIP(hipMemcpyAsync(&bad, flag, sizeof(int), hipMemcpyDeviceToHost, stream));
    RXMET_CHECK_HIP(hipStreamSynchronize(stream));
    RXMET_CHECK_ARG(bad == 0, "x_q / h0_q hold codes outside the x / h grids");
  }

  if (int rc = upload(wsb + ws.hostblk, host.data(), host.size(), stream)) return rc;
  IWeightArgs &wa = plan.wa;
  wa.W = k.W; wa.R = k.R; wa.bw = k.bw; wa.br = k.br;
  wa.eff = eff; wa.rs = rs;
  wa.gW = igrid_of(P.chan_bits[RXMET_GRU_W], P.chan_unsigned[RXMET_GRU_W]);
  wa.gR = igrid_of(P.chan_bits[RXMET_GRU_R], P.chan_unsigned[RXMET_GRU_R]);
  wa.gbw = igrid_of(P.chan_bits[RXMET_GRU_BW], P.chan_unsigned[RXMET_GRU_BW]);
  wa.gbr = igrid_of(P.chan_bits[RXMET_GRU_BR], P.chan_unsigned[RXMET_GRU_BR]);
  wa.Wq = k.Wq; wa.Rq = k.Rq; wa.bwq = k.bwq; wa.brq = k.brq;
  wa.Wm = k.training ? k.W_m : nullptr;
  wa.Rm = k.training ? k.R_m : nullptr;
  wa.bwm = k.training ? k.bw_m : nullptr;
  wa.brm = k.training ? k.br_m : nullptr;
  wa.bias = bias;
  {
    rxmet::prof::Scope ps__("gru_int_quant_weights", stream);
    const int64_t total = static_cast<int64_t>(I + H + 1) * C;
    hipLaunchKernelGGL(iq_weights, dim3(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 8192))),
                       dim3(256), 0, stream, I, H, wa);
  }
  RXMET_CHECK_LAUNCH();

  const int64_t nx = k.xq_in ? 0 : static_cast<int64_t>(T) * B * I, nh = static_cast<int64_t>(B) * H;
  plan.hqb = reinterpret_cast<int32_t *>(wsb + ws.hq);
  int32_t *hq0 = k.hq_out ? k.hq_out : plan.hqb;
  {
    rxmet::prof::Scope ps__("gru_int_quant_input", stream);
    const int64_t blocks = std::min<int64_t>((nx + nh + 255) / 256, 8192);
    hipLaunchKernelGGL(iq_input, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, nx, nh,
                       k.x, k.h0, k.h0q_in, sp, k.xq, k.training ? k.x_m : nullptr, hq0,
                       k.training ? k.h0_m : nullptr, k.h);
  }
  RXMET_CHECK_LAUNCH();

  // input projection: weight_ih_linear codes of every step
  const int32_t *xq = k.xq_in ? k.xq_in : k.xq;
  {
    const double xlo = sp.x.lo, xhi = sp.x.hi;
    const float off = xgemm::a_shift(xlo, xhi);
    const int pa = xgemm::a_planes(xlo, xhi), pb = xgemm::b_planes(wa.gW.lo, wa.gW.hi);
    LinearOut e{bias, rs, sp.zp_wx, sp.wx, wx, k.training ? k.ih_m : nullptr, C};
    rxmet::prof::Scope ps__("gru_int_input_gemm", stream);
    if (int rc = launch_linear(xq, I, T * B, I, off, static_cast<long long>(off) - sp.zp_x, pa,
                               k.Wq, C, C, pb, e, wsb, ws, stream))
      return rc;
  }
  plan.k = k;
  plan.bias = bias;
  plan.rs = rs;
  plan.wx = wx;
  plan.rh = reinterpret_cast<int32_t *>(wsb + ws.rh);
  plan.hq0 = hq0;
  plan.wsb = wsb;
  return 0;
}

// The stepped recurrence of one direction: per step R_q (h - zp_h) + br -> weight_hh_linear
// codes, then the gates.
static int stepped_int(const IntPlan &plan, hipStream_t stream) {
  const IntCall &k = plan.k;
  const IntStepParams &sp = plan.sp;
  const int T = k.T, B = k.B, I = k.I, H = k.H, C = 3 * H;
  const IntWorkspace ws(T, B, I, H);
  const int64_t nh = static_cast<int64_t>(B) * H;
  const double hlo = sp.h.lo, hhi = sp.h.hi;
  const float hoff = xgemm::a_shift(hlo, hhi);
  const int hpa = xgemm::a_planes(hlo, hhi), rpb = xgemm::b_planes(plan.wa.gR.lo, plan.wa.gR.hi);
  IPointArgs pa;
  pa.T = T; pa.B = B; pa.H = H;
  pa.wx = plan.wx; pa.rh = plan.rh; pa.hout = k.h; pa.v = k.v;
  pa.gin_m = k.training ? k.gin_m : nullptr;
  pa.gout_m = k.training ? k.gout_m : nullptr;
  pa.h_m = k.training ? k.h_m : nullptr;
  if (pa.gin_m && !(pa.gout_m && pa.h_m)) pa.gin_m = nullptr;
  const dim3 pgrid(static_cast<unsigned>((nh + 255) / 256));
  rxmet::prof::Scope ps__("gru_int_recurrence", stream);
  const int32_t *hcur = plan.hq0;
  for (int t = 0; t < T; ++t) {
    int32_t *hnext = k.hq_out ? k.hq_out + (static_cast<size_t>(t) + 1) * nh
                              : plan.hqb + static_cast<size_t>((t + 1) & 1) * nh;
    LinearOut e{plan.bias + C, plan.rs + 2 * C, sp.zp_rh, sp.rh, plan.rh,
                k.training && k.hh_m ? k.hh_m + static_cast<size_t>(t) * B * C : nullptr, C};
    if (int rc = launch_linear(hcur, H, B, H, hoff, static_cast<long long>(hoff) - sp.zp_h, hpa,
                               k.Rq, C, C, rpb, e, nullptr, ws, stream))
      return rc;
    hipLaunchKernelGGL(int_point, pgrid, dim3(256), 0, stream, pa, sp, t, hcur, hnext);
    RXMET_CHECK_LAUNCH();
    hcur = hnext;
  }
  return 0;
}

// ndir directions with the same shapes (each with its own workspace): the prologues, then
// one clustered launch for all of them, or each direction stepped.
static int forward_int_dirs(const IntCall *calls, int ndir, hipStream_t stream) {
  RXMET_CHECK_ARG(ndir == 1 || ndir == 2, "ndir must be 1 or 2");
  IntPlan plans[2];
  for (int d = 0; d < ndir; ++d) {
    if (d > 0)
      RXMET_CHECK_ARG(calls[d].T == calls[0].T && calls[d].B == calls[0].B &&
                          calls[d].I == calls[0].I && calls[d].H == calls[0].H &&
                          calls[d].training == calls[0].training,
                      "the directions must have the same shapes and mode");
    if (int rc = prologue_int(calls[d], stream, plans[d])) return rc;
  }
  const int rc = int_recurrence_clustered(plans, ndir, stream);
  if (rc < 0) return rc;
  if (rc == 1) return 0;
  for (int d = 0; d < ndir; ++d)
    if (int r = stepped_int(plans[d], stream)) return r;
  return 0;
}

static int forward_int(const IntCall &k, hipStream_t stream) {
  return forward_int_dirs(&k, 1, stream);
}

}  // namespace
}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int64_t rxmet_gru_forward_int_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  if (T < 1 || B < 1 || I < 1 || H < 1) return -22;
  return static_cast<int64_t>(IntWorkspace(T, B, I, H).total);
}

int rxmet_gru_forward_quant_int(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                                const float *W, const float *R, const float *bw, const float *br,
                                const float *x, const float *h0, const rxmet_gru_qparams *params,
                                float *h, float *v, int32_t *W_q, int32_t *R_q, int32_t *bw_q,
                                int32_t *br_q, int32_t *x_q, uint8_t *x_mask, uint8_t *h0_mask,
                                uint8_t *W_mask, uint8_t *R_mask, uint8_t *bw_mask,
                                uint8_t *br_mask, uint8_t *ih_mask, uint8_t *hh_mask,
                                uint8_t *gate_in_mask, uint8_t *gate_out_mask, uint8_t *h_mask,
                                void *workspace, void *stream) {
  clear_error();
  RXMET_CHECK_ARG(x && h && x_q, "x, h and x_q must be non-null");
  if (is_training)
    RXMET_CHECK_ARG(v && x_mask && W_mask && R_mask && bw_mask && br_mask && ih_mask && hh_mask &&
                        gate_in_mask && gate_out_mask && h_mask && (h0 == nullptr || h0_mask),
                    "training needs v and every mask output");
  IntCall k{};
  k.training = is_training != 0;
  k.T = T; k.B = B; k.I = I; k.H = H;
  k.W = W; k.R = R; k.bw = bw; k.br = br; k.x = x; k.h0 = h0;
  k.params = params;
  k.h = h; k.v = v;
  k.Wq = W_q; k.Rq = R_q; k.bwq = bw_q; k.brq = br_q; k.xq = x_q;
  k.x_m = x_mask; k.h0_m = h0_mask; k.W_m = W_mask; k.R_m = R_mask; k.bw_m = bw_mask;
  k.br_m = br_mask; k.ih_m = ih_mask; k.hh_m = hh_mask; k.gin_m = gate_in_mask;
  k.gout_m = gate_out_mask; k.h_m = h_mask;
  k.workspace = workspace;
  return forward_int(k, static_cast<hipStream_t>(stream));
}

int rxmet_gru_forward_quant_int_dirs(int32_t ndir, int32_t is_training, int32_t T, int32_t B,
                                     int32_t I, int32_t H, const rxmet_gru_int_dir *dirs,
                                     void *stream) {
  clear_error();
  RXMET_CHECK_ARG(ndir == 1 || ndir == 2, "ndir must be 1 or 2");
  RXMET_CHECK_ARG(dirs != nullptr, "dirs must be non-null");
  IntCall calls[2]{};
  const bool io = dirs[0].x_q_in != nullptr;
  for (int d = 0; d < ndir; ++d) {
    const rxmet_gru_int_dir &a = dirs[d];
    RXMET_CHECK_ARG((a.x_q_in != nullptr) == io, "both directions must be int-IO or neither");
    IntCall &k = calls[d];
    k.T = T; k.B = B; k.I = I; k.H = H;
    k.W = a.W; k.R = a.R; k.bw = a.bw; k.br = a.br;
    k.params = a.params;
    k.Wq = a.W_q; k.Rq = a.R_q; k.bwq = a.bw_q; k.brq = a.br_q;
    k.workspace = a.workspace;
    if (io) {
      RXMET_CHECK_ARG(!is_training, "int-IO directions run without training outputs");
      RXMET_CHECK_ARG(a.h_q != nullptr, "x_q_in and h_q must be non-null");
      k.training = false;
      k.xq_in = a.x_q_in; k.h0q_in = a.h0_q_in;
      k.hq_out = a.h_q;
    } else {
      RXMET_CHECK_ARG(a.x && a.h && a.x_q, "x, h and x_q must be non-null");
      if (is_training)
        RXMET_CHECK_ARG(a.v && a.x_mask && a.W_mask && a.R_mask && a.bw_mask && a.br_mask &&
                            a.ih_mask && a.hh_mask && a.gate_in_mask && a.gate_out_mask &&
                            a.h_mask && (a.h0 == nullptr || a.h0_mask),
                        "training needs v and every mask output");
      k.training = is_training != 0;
      k.x = a.x; k.h0 = a.h0;
      k.h = a.h; k.v = a.v; k.xq = a.x_q;
      k.x_m = a.x_mask; k.h0_m = a.h0_mask; k.W_m = a.W_mask; k.R_m = a.R_mask;
      k.bw_m = a.bw_mask; k.br_m = a.br_mask; k.ih_m = a.ih_mask; k.hh_m = a.hh_mask;
      k.gin_m = a.gate_in_mask; k.gout_m = a.gate_out_mask; k.h_m = a.h_mask;
    }
  }
  return forward_int_dirs(calls, ndir, static_cast<hipStream_t>(stream));
}

int rxmet_gru_forward_int_io(int32_t T, int32_t B, int32_t I, int32_t H, const float *W,
                             const float *R, const float *bw, const float *br,
                             const int32_t *x_q, const int32_t *h0_q,
                             const rxmet_gru_qparams *params, int32_t *h_q, int32_t *W_q,
                             int32_t *R_q, int32_t *bw_q, int32_t *br_q, void *workspace,
                             void *stream) {
  clear_error();
  RXMET_CHECK_ARG(x_q && h_q, "x_q and h_q must be non-null");
  IntCall k{};
  k.training = false;
  k.T = T; k.B = B; k.I = I; k.H = H;
  k.W = W; k.R = R; k.bw = bw; k.br = br;
  k.xq_in = x_q; k.h0q_in = h0_q;
  k.params = params;
  k.hq_out = h_q;
  k.Wq = W_q; k.Rq = R_q; k.bwq = bw_q; k.brq = br_q;
  k.workspace = workspace;
  return forward_int(k, static_cast<hipStream_t>(stream));
}

}  // extern "C"
