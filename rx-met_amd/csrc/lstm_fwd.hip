// lstm_fwd.hip — MI355X QuantLSTM FP32 q-carrier forward, behind rxmet_lstm_forward_quant.
//
// Reference path: lstm_forward_quantized (pytorch/lib/lstm_interface_binding.cc:643-806) ->
// lstmForwardQuantizedFpCuda (src/lstm/forward_quantized_fp_cuda.cu): boundary quantisation
// kernels (:580-660), one SGEMM for the input linear of all steps, then per step an SGEMM for
// the recurrent linear and fusedLstmPointwiseKernel (:690-880).  Numerics follow the CPU
// q-carrier reference that specifies that path (src/lstm/forward_quantized_fp_cpu.cc:20-197).
//
// Here:
//   1. lstm_quant_weights : one wave per gate channel quantises its W_ih / W_hh rows and
//      biases (codes + clamp masks), sums the W_hh codes and rescales the bias codes to the
//      accumulator grids;
//   2. lstm_quant_inputs  : x, h0, c0 codes and masks;
//   3. lstm_pack_whh      : W_hh codes -> int8 MFMA B fragments;
//   4. lstm_input_gemm    : the input linear of all T steps as an exact integer GEMM with
//      the whole input branch fused in its epilogue (bias, rescale, clamp + mask, and the
//      rescale to each gate-input grid), so the recurrence only adds the recurrent branch;
//   5. lstm_recurrence_cl : (H a multiple of 64) a cluster of H/64 workgroups per 16-sequence
//      batch tile in one cooperative launch.  Each member keeps the W_hh fragments of its 64
//      units resident in LDS, computes the recurrent linear on v_mfma_i32_16x16x64_i8, the
//      gates through precomputed activation tables (exact: the activation is a function of
//      the integer gate-input code), the cell and hidden update, every clamp mask and the
//      checkpoints; the new h codes are exchanged through global memory and the members meet
//      at a counter barrier once per step (cluster.h);
//   5'. lstm_recurrence   : otherwise, one persistent workgroup per 16 sequences walks the T
//      steps with h in LDS and W_hh fragments streamed from L2.
//
// Activations: sigmoid keeps the reference's float op order around exp, with exp and tanh
// evaluated in double and rounded once to float.
#include <cmath>
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "cluster.h"
#include "exact_gemm.h"
#include "lstm_internal.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_lstm.h"

namespace rxmet {
namespace lstm {

constexpr int kBT = 16;       // sequences per recurrent workgroup (MFMA N)
constexpr int kMaxH = 512;    // 8 waves x 4 unit tiles x 16 units
constexpr int kTilesPerWave = 4;

// Per-channel constants uploaded from the host.
struct ChanHost {
  float w_ih_s, w_hh_s, b_ih_s, b_hh_s;
  float ih_mult, hh_mult, ih_bmult, hh_bmult;
  int32_t ih_shift, hh_shift, ih_bshift, hh_bshift;
};

// Per-channel constants produced on the device for the two linears.
struct ChanRun {
  float ih_bacc;   // rescaled centred bias of the input linear (0 without bias)
  float hh_bacc;
  int32_t hh_k;    // integer correction of the recurrent MFMA sum (zero points, plane offsets)
  int32_t hh_k_hi; // its upper 32 bits (the correction exceeds int32 only with 16-bit W_hh)
};

__device__ __forceinline__ float rescale(float v, float mult, int shift) {
  return rintf(ldexpf(v * mult, -shift));
}

__device__ __forceinline__ float clamp_grid(double v, const Grid &g, uint8_t &clamped) {
  clamped = (v < g.dlo || v > g.dhi) ? 1 : 0;
  return v <= g.dflo ? g.flo : (v >= g.dfhi ? g.fhi : static_cast<float>(v));
}

__device__ __forceinline__ float quantize(float v, float s, int32_t zp, const Grid &g,
                                          uint8_t &clamped) {
  const double r = rint(static_cast<double>(v) / static_cast<double>(s)) + static_cast<double>(zp);
  return clamp_grid(r, g, clamped);
}

__device__ __forceinline__ float dequant(float q, float s, int32_t zp) {
  return static_cast<float>((static_cast<double>(q) - zp) * static_cast<double>(s));
}

__device__ __forceinline__ float center(float v, int32_t zp) {
  return static_cast<float>(static_cast<double>(v) - zp);
}

// Float-domain forms of clamp_grid / center / dequant for grids whose codes lie within
// +-2^24 (at most 24 bits): every in-range sum or difference of integer-valued floats is then
// exact in float, a rounded out-of-range sum stays beyond the same endpoint, and the product
// of a code difference and a float scale is exact in double, so its float rounding equals the
// fp32 product.  The results equal the double-domain forms bit for bit.
__device__ __forceinline__ float clamp_grid_f(float v, const Grid &g, uint8_t &clamped) {
  const float s = v + static_cast<float>(g.zp);
  clamped = (s < g.flo || s > g.fhi) ? 1 : 0;
  return s <= g.flo ? g.flo : (s >= g.fhi ? g.fhi : s);
}

__device__ __forceinline__ float center_f(float v, int32_t zp) { return v - static_cast<float>(zp); }

__device__ __forceinline__ float dequant_f(float q, float s, int32_t zp) {
  return (q - static_cast<float>(zp)) * s;
}

inline bool fits_f32(const Grid &g) { return g.lo > -(1 << 24) && g.hi < (1 << 24); }

__device__ __forceinline__ float act_sigmoid(float x) {
  if (x >= 0.0f) {
    const float e = static_cast<float>(exp(-static_cast<double>(x)));
    return 1.0f / (1.0f + e);
  }
  const float e = static_cast<float>(exp(static_cast<double>(x)));
  return e / (1.0f + e);
}

__device__ __forceinline__ float act_tanh(float x) {
  return static_cast<float>(tanh(static_cast<double>(x)));
}

// Real activation boundary: dequantise, activate in fp32, quantise to the output grid.
// Activation k (gates 0..3, 4 = tanh of the cell) then takes the reference CPU core's result
// at the few input codes where its C-library expf / tanhf lead to another output code than
// the double evaluation (sp.exc_*, listed on the host; none on most grids).
// EXC = false skips the lookup (launches whose parameters have no exception codes).
template <bool EXC = true>
__device__ __forceinline__ float real_act(float q, const Grid &in, const Grid &out, bool is_tanh,
                                          const StepParams &sp, int k, uint8_t &clamped) {
  const float x = static_cast<float>((static_cast<double>(q) - in.dzp) * in.dscale);
  const float a = is_tanh ? act_tanh(x) : act_sigmoid(x);
  const double t = rint(static_cast<double>(a) / out.dscale) + out.dzp;
  float v = clamp_grid(t, out, clamped);
  const int n = EXC ? sp.exc_n[k] : 0;
  if (n > 0) {
    const int32_t key = static_cast<int32_t>(q);
    const int32_t *ks = sp.exc_key + sp.exc_off[k];
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (ks[mid] < key)
        lo = mid + 1;
      else
        hi = mid;
    }
    if (lo < n && ks[lo] == key) {
      const uint32_t e = sp.exc_val[sp.exc_off[k] + lo];
      clamped = static_cast<uint8_t>(e & 1u);
      v = static_cast<float>(static_cast<int64_t>(e >> 1) + out.lo);
    }
  }
  return v;
}

// Element r of an MFMA accumulator without dynamic register indexing.
__device__ __forceinline__ int pick(const v4i &v, int r) {
  return r == 0 ? v[0] : (r == 1 ? v[1] : (r == 2 ? v[2] : v[3]));
}

__device__ __forceinline__ float cell_scale(float p, const StepParams &sp, int k) {
  return sp.cell_fp[k]
             ? static_cast<float>(ldexp(static_cast<double>(p) * sp.cell_mant[k], sp.cell_exp[k]))
             : p * sp.cell_ratio[k];
}

// ---------------------------------------------------------------------------------
// 1-3. quantisation prologue
// ---------------------------------------------------------------------------------
struct WeightArgs {
  int I, H, bias, npl;
  const float *W_ih, *W_hh, *b_ih, *b_hh;
  const ChanHost *ch;
  float *wq_ih, *wq_hh, *bq_ih, *bq_hh;
  uint8_t *wm_ih, *wm_hh, *bm_ih, *bm_hh;
  ChanRun *run;
  int32_t hh_k_factor;  // h_offset - zp_h (+128 with two planes)
};

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ __launch_bounds__(64) void lstm_quant_weights(WeightArgs a, Grid gw_ih, Grid gw_hh,
                                                         Grid gb_ih, Grid gb_hh) {
  const int c = blockIdx.x, l = threadIdx.x;
  const ChanHost ch = a.ch[c];
  uint8_t m;
  for (int k = l; k < a.I; k += 64) {
    const size_t i = static_cast<size_t>(c) * a.I + k;
    const float q = quantize(a.W_ih[i], ch.w_ih_s, 0, gw_ih, m);
    a.wq_ih[i] = q;
    if (a.wm_ih) a.wm_ih[i] = m;
  }
  int s = 0;  // |sum| <= 2^15 * H: int32 for H < 2^16
  for (int k = l; k < a.H; k += 64) {
    const size_t i = static_cast<size_t>(c) * a.H + k;
    const float q = quantize(a.W_hh[i], ch.w_hh_s, 0, gw_hh, m);
    a.wq_hh[i] = q;
    if (a.wm_hh) a.wm_hh[i] = m;
    s += static_cast<int>(q);
  }
  s = wave_sum_int(s);
  if (l == 0) {
    ChanRun r;
    r.ih_bacc = 0.0f;
    r.hh_bacc = 0.0f;
    if (a.bias) {
      const float qi = quantize(a.b_ih[c], ch.b_ih_s, 0, gb_ih, m);
      a.bq_ih[c] = qi;
      if (a.bm_ih) a.bm_ih[c] = m;
      const float qh = quantize(a.b_hh[c], ch.b_hh_s, 0, gb_hh, m);
      a.bq_hh[c] = qh;
      if (a.bm_hh) a.bm_hh[c] = m;
      r.ih_bacc = rescale(center(qi, 0), ch.ih_bmult, ch.ih_bshift);
      r.hh_bacc = rescale(center(qh, 0), ch.hh_bmult, ch.hh_bshift);
    }
    const int64_t k64 = static_cast<int64_t>(s) * a.hh_k_factor;
    r.hh_k = static_cast<int32_t>(k64);
    r.hh_k_hi = static_cast<int32_t>(k64 >> 32);
    a.run[c] = r;
  }
}

__global__ __launch_bounds__(256) void lstm_quant_inputs(int64_t nx, int64_t nh, const float *x,
                                                         const float *h0, const float *c0,
                                                         StepParams sp, float *xq, uint8_t *xm,
                                                         float *hq, uint8_t *hm, float *cq,
                                                         uint8_t *cm) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nx + nh;
       i += stride) {
    uint8_t m = 0;
    if (i < nx) {
      xq[i] = quantize(x[i], sp.x.scale, sp.x.zp, sp.x, m);
      if (xm) xm[i] = m;
    } else {
      const int64_t j = i - nx;
      uint8_t m2 = 0;
      hq[j] = quantize(h0 ? h0[j] : 0.0f, sp.h.scale, sp.h.zp, sp.h, m);
      cq[j] = quantize(c0 ? c0[j] : 0.0f, sp.c.scale, sp.c.zp, sp.c, m2);
      if (hm) hm[j] = h0 ? m : 0;
      if (cm) cm[j] = c0 ? m2 : 0;
    }
  }
}

// W_hh codes [4H][H] -> B fragments of D[b][c] = sum_k h[b][k] W[c][k]:
// frag[(ct * KS + s) * 64 + lane] = W[16 ct + lane % 16][64 s + 16 (lane / 16) + 0..15].
// With pw = 2 planes (W_hh wider than 8 bits, at most 16) W = 256 bh + bl + 128 with bl, bh
// signed bytes: bl's fragments first, then bh's, plane_stride fragments apart.
__global__ __launch_bounds__(64) void lstm_pack_whh(int H, int KS, int pw, size_t plane_stride,
                                                    const float *__restrict__ wq,
                                                    v4i *__restrict__ frag) {
  const int lane = threadIdx.x, idx = blockIdx.x;
  const int s = idx % KS, ct = idx / KS;
  const int c = 16 * ct + lane % 16;
  for (int p = 0; p < pw; ++p) {
    int wd[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int by[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = 64 * s + 16 * (lane / 16) + 4 * q + e;
        int w = k < H ? static_cast<int>(wq[static_cast<size_t>(c) * H + k]) : 0;
        if (pw == 2) {  // (the two-plane recurrence needs H a multiple of 64: no padded k)
          const int u = w + 32768;
          w = p == 0 ? (u & 255) - 128 : (u >> 8) - 128;
        }
        by[e] = w;
      }
      wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
    }
    frag[p * plane_stride + static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
  }
}

// ---------------------------------------------------------------------------------
// 4. input linear of all steps, exact, with the input branch fused in the epilogue
// ---------------------------------------------------------------------------------
template <int PA, int PB>
__global__ __launch_bounds__(256) void lstm_input_gemm(xgemm::Operands o, int H,
                                                       const ChanHost *__restrict__ ch,
                                                       const ChanRun *__restrict__ run,
                                                       StepParams sp, float *__restrict__ lhs,
                                                       uint8_t *__restrict__ lin_mask) {
  const int C = o.N;
  xgemm::block<PA, PB>(o, blockIdx.y * xgemm::kTile, blockIdx.x * xgemm::kTile,
                       [&](int m, int c, long long s) {
                         const int g = c / H;
                         const float accf = static_cast<float>(s) + run[c].ih_bacc;
                         uint8_t clamped;
                         const float lin = clamp_grid(
                             static_cast<double>(rescale(accf, ch[c].ih_mult, ch[c].ih_shift)) +
                                 sp.ih_lin.dzp,
                             sp.ih_lin, clamped);
                         const size_t oi = static_cast<size_t>(m) * C + c;
                         lhs[oi] = rescale(center(lin, sp.ih_lin.zp), sp.ih_to_gate[g].mult,
                                           sp.ih_to_gate[g].shift);
                         if (lin_mask) lin_mask[oi] = clamped;
                       });
}

// Pre-packed variant (I <= kPackedMaxK): one wave per 16 rows and every fourth channel tile,
// the same input-branch epilogue (in float when the linear grid fits 24 bits, where the float
// clamp and centring are exact).
constexpr int kPackedMaxK = 256;
template <int PA, int PB, bool F32>
__global__ __launch_bounds__(256) void lstm_input_gemm_packed(xgemm::Packed p, int H,
                                                              const ChanHost *__restrict__ ch,
                                                              const ChanRun *__restrict__ run,
                                                              StepParams sp, float *__restrict__ lhs,
                                                              uint8_t *__restrict__ lin_mask) {
  const int C = p.N;
  xgemm::rows16<PA, PB>(
      p, 16 * blockIdx.x, threadIdx.x / 64, 4, [&](int m, int c, const long long *s, int rows) {
        // the channel's constants once for its (up to) four rows
        const int g = c / H;
        const float bacc = run[c].ih_bacc, mult = ch[c].ih_mult;
        const int32_t shift = ch[c].ih_shift;
        const Rescale tg = g == 0 ? sp.ih_to_gate[0]
                           : g == 1 ? sp.ih_to_gate[1]
                           : g == 2 ? sp.ih_to_gate[2]
                                    : sp.ih_to_gate[3];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r >= rows) break;
          const float accf = static_cast<float>(s[r]) + bacc;
          uint8_t clamped;
          const float x = rescale(accf, mult, shift);
          const float lin = F32 ? clamp_grid_f(x, sp.ih_lin, clamped)
                                : clamp_grid(static_cast<double>(x) + sp.ih_lin.dzp, sp.ih_lin, clamped);
          const size_t oi = static_cast<size_t>(m + r) * C + c;
          const float cl = F32 ? center_f(lin, sp.ih_lin.zp) : center(lin, sp.ih_lin.zp);
          lhs[oi] = rescale(cl, tg.mult, tg.shift);
          if (lin_mask) lin_mask[oi] = clamped;
        }
      });
}

// ---------------------------------------------------------------------------------
// 5. recurrence
// ---------------------------------------------------------------------------------
struct RecArgs {
  int T, B, H, KS, UT;
  float h_offset;          // 2^(bits-1) for an unsigned h grid (codes centred into int8/int16)
  const float *lhs;        // [T, B, 4H] input branch on the gate-input grids
  const v4i *frag;         // W_hh fragments
  const ChanHost *ch;
  const ChanRun *run;
  const float *h0q, *c0q;  // [B, H]
  float *output;           // [T, B, H] dequantised
  float *h_n, *c_n;        // [B, H] dequantised
  // checkpoints (null in inference)
  float *gate_out, *cell, *cell_tanh, *hidden;
  uint8_t *hh_lin_m, *gate_in_m, *gate_out_m, *cell_m, *cell_tanh_m, *hidden_m;
  // saved state as codes (training; instead of gate_out, cell, cell_tanh and the six masks
  // above): the blocks and the cell codes of lck_block
  uint8_t *ckb;
  uint16_t *cellc;
  int wide_out;  // clustered path: outputs 16-byte aligned, stored as 16-byte rows through LDS
};

// A saved code as its offset from the grid's minimum (grids of at most 16 bits).
__device__ __forceinline__ uint32_t lck_u16(float code, int32_t lo) {
  return static_cast<uint32_t>(static_cast<int32_t>(code) - lo) & 0xFFFFu;
}

// One gate output of (step t, sequence b, unit j) and its three gate masks into its block.
__device__ __forceinline__ void lck_store_gate(const RecArgs &a, int t, int b, int j, int g,
                                               float go, int32_t lo, uint32_t bits) {
  uint8_t *blk = a.ckb + static_cast<size_t>(lck_block(t, b, j, a.B, a.H)) * kLckBlock;
  const int R = b % 16, e = j % 16;
  reinterpret_cast<uint16_t *>(blk)[(R * 4 + g) * 16 + e] = static_cast<uint16_t>(lck_u16(go, lo));
  blk[kLckGm + (g * 16 + R) * 16 + e] = static_cast<uint8_t>(bits);
}

// The cell-phase codes of (step t, sequence b, unit j): tanh(c) and the three masks into the
// step's block, the cell into the cell codes at step t + 1.
__device__ __forceinline__ void lck_store_cell(const RecArgs &a, const StepParams &sp, int t, int b,
                                               int j, float cn, float ct, uint32_t bits) {
  const uint32_t k = lck_block(t, b, j, a.B, a.H);
  uint8_t *blk = a.ckb + static_cast<size_t>(k) * kLckBlock;
  const int R = b % 16, e = j % 16;
  reinterpret_cast<uint16_t *>(blk + kLckTanh)[R * 16 + e] =
      static_cast<uint16_t>(lck_u16(ct, sp.tanh_c.lo));
  blk[kLckCm + R * 16 + e] = static_cast<uint8_t>(bits);
  a.cellc[static_cast<size_t>(lck_block(t + 1, b, j, a.B, a.H)) * kLcellBlock + R * 16 + e] =
      static_cast<uint16_t>(lck_u16(cn, sp.c.lo));
}

// One (sequence, unit) step of the q-carrier (forward_quantized_fp_cpu.cc:18-44, 116-190): per
// gate the recurrent linear from its exact centred sum plus the rescaled bias (accf), its
// rescale and clamp, the gate input with the input branch (lhs), the real activation; then the
// cell (two contributions, one rounding) and the hidden update, with every clamp mask
// (1 = clamped).
struct LstmPoint {
  float gout[4], cn, ct, hv;
  uint8_t m_hl[4], m_gi[4], m_go[4], m_c, m_t, m_h;
};

__device__ __forceinline__ LstmPoint lstm_point(const float accf[4], const float mult[4],
                                                const int shift[4], const float lhs[4],
                                                float c_old, const StepParams &sp) {
  LstmPoint o;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float lin = clamp_grid(static_cast<double>(rescale(accf[g], mult[g], shift[g])) +
                                     sp.hh_lin.dzp,
                                 sp.hh_lin, o.m_hl[g]);
    const float rhs = rescale(center(lin, sp.hh_lin.zp), sp.hh_to_gate[g].mult,
                              sp.hh_to_gate[g].shift);
    const float gi = clamp_grid(static_cast<double>(lhs[g] + rhs) + sp.gin[g].dzp, sp.gin[g],
                                o.m_gi[g]);
    o.gout[g] = real_act(gi, sp.gin[g], sp.gout[g], g == 2, sp, g, o.m_go[g]);
  }
  const float pf = center(o.gout[1], sp.gout[1].zp) * center(c_old, sp.c.zp);
  const float pi = center(o.gout[0], sp.gout[0].zp) * center(o.gout[2], sp.gout[2].zp);
  const float sum = cell_scale(pf, sp, 0) + cell_scale(pi, sp, 1);
  o.cn = clamp_grid(static_cast<double>(rintf(sum)) + sp.c.dzp, sp.c, o.m_c);
  o.ct = real_act(o.cn, sp.c, sp.tanh_c, true, sp, 4, o.m_t);
  const float raw = center(o.gout[3], sp.gout[3].zp) * center(o.ct, sp.tanh_c.zp);
  o.hv = clamp_grid(static_cast<double>(rescale(raw, sp.hidden.mult, sp.hidden.shift)) + sp.h.dzp,
                    sp.h, o.m_h);
  return o;
}

// The outputs of one (step t, sequence b, unit j): dequantised output, the checkpoints and
// masks in training, h_n / c_n at the last step.
__device__ __forceinline__ void lstm_store(const RecArgs &a, const StepParams &sp, int t, int b,
                                           int j, const LstmPoint &o) {
  const uint32_t H = static_cast<uint32_t>(a.H), C = 4u * H;
  const uint32_t row = static_cast<uint32_t>(t) * a.B + b;
  const uint32_t oh = row * H + j;
  a.output[oh] = dequant(o.hv, sp.h.scale, sp.h.zp);
  if (a.hidden != nullptr && a.ckb != nullptr) {
    a.hidden[oh] = o.hv;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      lck_store_gate(a, t, b, j, g, o.gout[g], sp.gout[g].lo,
                     o.m_hl[g] | (o.m_gi[g] << 1) | (o.m_go[g] << 2));
    lck_store_cell(a, sp, t, b, j, o.cn, o.ct, o.m_c | (o.m_t << 1) | (o.m_h << 2));
  } else if (a.hidden != nullptr) {
    a.cell[oh] = o.cn;
    a.cell_tanh[oh] = o.ct;
    a.hidden[oh] = o.hv;
    a.cell_m[oh] = o.m_c;
    a.cell_tanh_m[oh] = o.m_t;
    a.hidden_m[oh] = o.m_h;
    const uint32_t oc = row * C + j;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      a.gate_out[oc + g * H] = o.gout[g];
      a.hh_lin_m[oc + g * H] = o.m_hl[g];
      a.gate_in_m[oc + g * H] = o.m_gi[g];
      a.gate_out_m[oc + g * H] = o.m_go[g];
    }
  }
  if (t == a.T - 1) {
    const uint32_t os = static_cast<uint32_t>(b) * H + j;
    a.h_n[os] = dequant(o.hv, sp.h.scale, sp.h.zp);
    a.c_n[os] = dequant(o.cn, sp.c.scale, sp.c.zp);
  }
}

template <int NPL>
__global__ __launch_bounds__(512) void lstm_recurrence(RecArgs a, StepParams sp) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 4 * H, B = a.B, KS = a.KS;
  const int ROW = KS * 64 + 16;  // plane row stride in bytes
  float4 *chan = reinterpret_cast<float4 *>(smem);                       // [4H]: mult, bacc, k, shift
  float *cstate = reinterpret_cast<float *>(chan + C);                   // [16][H] cell codes
  int8_t *plane = reinterpret_cast<int8_t *>(cstate + kBT * H);          // [2][NPL][16][ROW]
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int b0 = blockIdx.x * kBT;
  for (int c = tid; c < C; c += blockDim.x) {
    const ChanRun r = a.run[c];
    const ChanHost h = a.ch[c];
    chan[c] = make_float4(h.hh_mult, r.hh_bacc, __int_as_float(r.hh_k), __int_as_float(h.hh_shift));
  }
  for (int i = tid; i < 2 * NPL * kBT * ROW / 4; i += blockDim.x)
    reinterpret_cast<int *>(plane)[i] = 0;
  __syncthreads();
  // initial h planes
  for (int i = tid; i < kBT * H; i += blockDim.x) {
    const int n = i / H, j = i % H, b = b0 + n;
    const float q = b < B ? a.h0q[static_cast<size_t>(b) * H + j] : static_cast<float>(sp.h.zp);
    const int hc = static_cast<int>(q - a.h_offset);
    if (NPL == 1) {
      plane[n * ROW + j] = static_cast<int8_t>(hc);
    } else {
      plane[n * ROW + j] = static_cast<int8_t>((hc & 255) - 128);
      plane[(kBT + n) * ROW + j] = static_cast<int8_t>(hc >> 8);
    }
  }
  // each (row, unit) cell code is read and written by one lane only
  for (int i = tid; i < kBT * H; i += blockDim.x) {
    const int n = i / H, j = i % H, b = b0 + n;
    cstate[i] = b < B ? a.c0q[static_cast<size_t>(b) * H + j] : static_cast<float>(sp.c.zp);
  }
  const int nrow0 = 4 * (l / 16);
  __syncthreads();

  for (int t = 0; t < a.T; ++t) {
    const int cur = t & 1, nxt = cur ^ 1;
    const int8_t *pc = plane + cur * NPL * kBT * ROW;
    int8_t *pn = plane + nxt * NPL * kBT * ROW;
#pragma unroll 1
    for (int u = 0; u < kTilesPerWave; ++u) {
      const int ut = kTilesPerWave * w + u;
      if (ut >= a.UT) continue;
      const int j = 16 * ut + l % 16;
      __builtin_amdgcn_sched_barrier(0);
      v4i acc[4][NPL];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < NPL; ++q) acc[g][q] = v4i{0, 0, 0, 0};
      for (int s = 0; s < KS; ++s) {
        v4i hfr[NPL];
#pragma unroll
        for (int q = 0; q < NPL; ++q)
          hfr[q] = *reinterpret_cast<const v4i *>(pc + (q * kBT + l % 16) * ROW + 64 * s + 16 * (l / 16));
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const v4i bf = a.frag[(static_cast<uint32_t>(g * a.UT + ut) * KS + s) * 64 + l];
#pragma unroll
          for (int q = 0; q < NPL; ++q) acc[g][q] = mfma_i8(hfr[q], bf, acc[g][q]);
        }
      }
      float4 cc[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) cc[g] = chan[g * H + j];
#pragma unroll 1
      for (int r = 0; r < 4; ++r) {
        const int nr = nrow0 + r, b = b0 + nr;
        const bool valid = b < B;
        const uint32_t row = static_cast<uint32_t>(t) * B + b;  // (t, b)
        float accf[4], mult[4], lhs[4];
        int shift[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int v = pick(acc[g][0], r);
          if (NPL == 2) v += 256 * pick(acc[g][1], r);
          v += __float_as_int(cc[g].z);
          accf[g] = static_cast<float>(v) + cc[g].y;
          mult[g] = cc[g].x;
          shift[g] = __float_as_int(cc[g].w);
          lhs[g] = valid ? a.lhs[static_cast<size_t>(row) * C + g * H + j] : 0.0f;
        }
        float &cref = cstate[nr * H + j];
        const LstmPoint o = lstm_point(accf, mult, shift, lhs, cref, sp);
        cref = o.cn;
        const float hv = o.hv;
        if (valid) lstm_store(a, sp, t, b, j, o);
        const int hc = static_cast<int>(hv - a.h_offset);
        if (NPL == 1) {
          pn[nr * ROW + j] = static_cast<int8_t>(hc);
        } else {
          pn[nr * ROW + j] = static_cast<int8_t>((hc & 255) - 128);
          pn[(kBT + nr) * ROW + j] = static_cast<int8_t>(hc >> 8);
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------
// 5'. stepped recurrence (W_hh wider than 8 bits, H above 512, or recurrent sums beyond int32)
// ---------------------------------------------------------------------------------
// Per step one exact GEMM of the centred h codes against the W_hh codes (xgemm::block: byte
// planes on int8 MFMA, combined in int64, rounded once to fp32) and one pointwise launch over
// all (sequence, unit) pairs; h codes in two fp32 [B, H] buffers, the cell codes in one.
template <int PA, int PB>
__global__ __launch_bounds__(256) void lstm_step_gemm(xgemm::Operands o, float *ghh) {
  xgemm::block<PA, PB>(o, blockIdx.x * xgemm::kTile, blockIdx.y * xgemm::kTile,
                       [&](int m, int n, long long sum) {
                         ghh[static_cast<size_t>(m) * o.N + n] = static_cast<float>(sum);
                       });
}

__global__ __launch_bounds__(256) void lstm_step_point(RecArgs a, StepParams sp, int t,
                                                       const float *ghh, const float *cin,
                                                       float *cout, float *hnext) {
  const int H = a.H, C = 4 * H;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<int64_t>(a.B) * H) return;
  const int b = static_cast<int>(e / H), j = static_cast<int>(e % H);
  float accf[4], mult[4], lhs[4];
  int shift[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int c = g * H + j;
    accf[g] = ghh[static_cast<size_t>(b) * C + c] + a.run[c].hh_bacc;
    mult[g] = a.ch[c].hh_mult;
    shift[g] = a.ch[c].hh_shift;
    lhs[g] = a.lhs[(static_cast<size_t>(t) * a.B + b) * C + c];
  }
  const LstmPoint o = lstm_point(accf, mult, shift, lhs, cin[e], sp);
  cout[e] = o.cn;
  hnext[e] = o.hv;
  lstm_store(a, sp, t, b, j, o);
}

// ---------------------------------------------------------------------------------
// 5b. clustered recurrence: a batch tile's units split over G = H / 64 workgroups
// ---------------------------------------------------------------------------------
// Member m of a cluster owns units [64 m, 64 m + 64) for all four gates and keeps their W_hh
// fragments (256 channels x H int8) resident in LDS for the whole launch.  Wave w computes
// unit tile w % 4 for the gate pair w / 4 (i, f or g, o) over the full K; the gate outputs
// meet in LDS and each wave then finishes the cell and hidden update of two of the lane's
// four rows.  The new h codes go to a global exchange buffer, double-buffered by step
// parity, and the members meet at a cluster barrier once per step.
constexpr int kClUnits = 64;
constexpr int kLutMaxEntries = 4096;  // activation tables kept in LDS up to 16 KB each

// The real activation of a gate is a function of the gate-input code alone, and the cell's
// tanh a function of the cell code: on grids of at most kLutMaxEntries codes the clustered
// recurrence reads precomputed results (same device function, evaluated once per code) from
// LDS.  Grids of up to kGlobalLutMaxCodes codes that LDS cannot hold have their tables in
// global memory (L2-resident, 256 KB per 16-bit grid) when that saves work on the step's
// dependent chain: the four gates (eight evaluations per lane and step, one gather instead),
// and the cell's tanh when its grid has exception codes (a lookup instead of the evaluation
// and the search of the exception list).  Entry = (output code - output grid lo) << 1 | mask.
constexpr int kGlobalLutMaxCodes = 1 << 16;
struct ActLut {
  const uint32_t *table;  // gate tables [off[g] .. off[g] + n[g]), then the tanh table
  int off[4], n[4];       // n = 0: no gate tables (computed in place)
  int tanh_off, tanh_n;   // tanh_n = 0: computed in place
  int total;
  // tables read from global memory, laid out the same way
  const uint32_t *gtable;
  int goff[4], gn[4], gtanh_off, gtanh_n, gtotal;
};

__global__ __launch_bounds__(256) void lstm_build_act_lut(StepParams sp, ActLut lut,
                                                          uint32_t *table) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= lut.total) return;
  uint8_t m;
  float v;
  int lo;
  // the double evaluation only: lstm_act_lut_exceptions then writes the exception entries.
  // Every StepParams member is named with a constant index (a run-time index into the
  // kernel-argument struct would copy the whole struct to scratch memory per thread).
  auto gate = [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    v = real_act<false>(static_cast<float>(sp.gin[k].lo + (i - lut.off[k])), sp.gin[k],
                        sp.gout[k], k == 2, sp, k, m);
    lo = sp.gout[k].lo;
  };
  if (lut.tanh_n > 0 && i >= lut.tanh_off) {
    v = real_act<false>(static_cast<float>(sp.c.lo + (i - lut.tanh_off)), sp.c, sp.tanh_c, true,
                        sp, 4, m);
    lo = sp.tanh_c.lo;
  } else if (i < lut.off[1]) {
    gate(std::integral_constant<int, 0>{});
  } else if (i < lut.off[2]) {
    gate(std::integral_constant<int, 1>{});
  } else if (i < lut.off[3]) {
    gate(std::integral_constant<int, 2>{});
  } else {
    gate(std::integral_constant<int, 3>{});
  }
  table[i] = (static_cast<uint32_t>(static_cast<int>(v) - lo) << 1) | m;
}

// The reference's entries at the exception codes of the activations a table holds (one thread
// per listed code; launched after lstm_build_act_lut on the same stream).
__global__ __launch_bounds__(256) void lstm_act_lut_exceptions(StepParams sp, ActLut lut,
                                                               uint32_t *table) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    if (i < sp.exc_n[k]) {
      const bool have = k < 4 ? lut.n[k] > 0 : lut.tanh_n > 0;
      if (!have) return;
      const int lo_in = k < 4 ? sp.gin[k].lo : sp.c.lo;
      const int base = k < 4 ? lut.off[k] : lut.tanh_off;
      table[base + (sp.exc_key[sp.exc_off[k] + i] - lo_in)] = sp.exc_val[sp.exc_off[k] + i];
      return;
    }
    i -= sp.exc_n[k];
  }
}


__device__ __forceinline__ float lut_code(const uint32_t *t, int idx, int out_lo, uint8_t &m) {
  const uint32_t e = t[idx];
  m = static_cast<uint8_t>(e & 1u);
  return static_cast<float>(static_cast<int>(e >> 1) + out_lo);
}

struct ClusterArgs {
  int ncl, G, ntiles, Bpad;
  int8_t *hx;          // [2][NPL][Bpad][H] centred h codes as int8 planes
  unsigned *counters;  // [ncl] barrier arrivals, kCounterStride words apart
  int *timeout;        // set by a member whose barrier wait gave up
  unsigned spin_limit; // polls before a wait gives up (cluster::spin_limit())
  ActLut lut;
};

// Bits k of sixteen packed mask bytes as sixteen 0/1 bytes.
__device__ __forceinline__ uint4 mask_bits(const uint4 v, int k) {
  return make_uint4((v.x >> k) & 0x01010101u, (v.y >> k) & 0x01010101u, (v.z >> k) & 0x01010101u,
                    (v.w >> k) & 0x01010101u);
}

// One float array [T, B, H] of the member's 64 units for the tile's 16 rows from the staging
// rows src ([16][64] in LDS), as 16-byte stores (deq: dequantise h codes on the way).
__device__ __forceinline__ void flush_rows(float *dst, const float *src, int t, int b0, int B, int H,
                                           int u0, int c0, int nthr, bool deq, float scale, int32_t zp) {
  for (int c = c0; c < 16 * 16; c += nthr) {
    const int row = c / 16, q = c % 16, b = b0 + row;
    if (b >= B) continue;
    float4 v = *reinterpret_cast<const float4 *>(src + row * kClUnits + 4 * q);
    if (deq) {
      v.x = dequant_f(v.x, scale, zp);
      v.y = dequant_f(v.y, scale, zp);
      v.z = dequant_f(v.z, scale, zp);
      v.w = dequant_f(v.w, scale, zp);
    }
    *reinterpret_cast<float4 *>(dst + (static_cast<size_t>(t) * B + b) * H + u0 + 4 * q) = v;
  }
}

// Stores of one step's outputs and checkpoints for the member's units, after the arrival:
// the gate outputs straight from the gate exchange xg, the mask bytes from their packed bits,
// and the cell-phase values staged through xg once every wave has finished reading it.
// Every thread of the workgroup calls it; (srow, su) is the lane's first staging row and unit.
__device__ __forceinline__ void flush_step(const RecArgs &a, const StepParams &sp, int t, int b0,
                                           int u0, bool train, float *xg, const uint8_t *gm,
                                           const uint8_t *cm, const float (&hvs)[2],
                                           const float (&cst)[2], const float (&cts)[2], int srow,
                                           int su) {
  const int H = a.H, C = 4 * H, B = a.B, tid = threadIdx.x, nthr = blockDim.x;
  if (train) {
    for (int c = tid; c < 4 * 16 * 16; c += nthr) {
      const int k = c % 4, ut = (c / 4) % 4, row = (c / 16) % 16, g = c / 256, b = b0 + row;
      if (b >= B) continue;
      *reinterpret_cast<float4 *>(a.gate_out + (static_cast<size_t>(t) * B + b) * C + g * H + u0 +
                                  16 * ut + 4 * k) =
          *reinterpret_cast<const float4 *>(xg + ((ut * 4 + g) * 16 + row) * 16 + 4 * k);
    }
    for (int c = (tid + nthr - 256 % nthr) % nthr; c < 4 * 16 * 4; c += nthr) {
      const int q = c % 4, row = (c / 4) % 16, g = c / 64, b = b0 + row;
      if (b >= B) continue;
      const uint4 v = *reinterpret_cast<const uint4 *>(gm + (g * 16 + row) * kClUnits + 16 * q);
      const size_t o = (static_cast<size_t>(t) * B + b) * C + g * H + u0 + 16 * q;
      *reinterpret_cast<uint4 *>(a.hh_lin_m + o) = mask_bits(v, 0);
      *reinterpret_cast<uint4 *>(a.gate_in_m + o) = mask_bits(v, 1);
      *reinterpret_cast<uint4 *>(a.gate_out_m + o) = mask_bits(v, 2);
    }
  }
  __syncthreads();  // every read of xg is done
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    float *d = xg + (srow + rr) * kClUnits + su;
    d[0] = hvs[rr];
    d[16 * kClUnits] = cst[rr];
    d[32 * kClUnits] = cts[rr];
  }
  __syncthreads();
  flush_rows(a.output, xg, t, b0, B, H, u0, tid, nthr, true, sp.h.scale, sp.h.zp);
  if (train) {
    flush_rows(a.hidden, xg, t, b0, B, H, u0, (tid + nthr - 256 % nthr) % nthr, nthr, false, 0.f, 0);
    flush_rows(a.cell, xg + 16 * kClUnits, t, b0, B, H, u0, tid, nthr, false, 0.f, 0);
    flush_rows(a.cell_tanh, xg + 32 * kClUnits, t, b0, B, H, u0, (tid + nthr - 256 % nthr) % nthr,
               nthr, false, 0.f, 0);
    for (int c = tid; c < 16 * 4; c += nthr) {
      const int q = c % 4, row = c / 4, b = b0 + row;
      if (b >= B) continue;
      const uint4 v = *reinterpret_cast<const uint4 *>(cm + row * kClUnits + 16 * q);
      const size_t o = (static_cast<size_t>(t) * B + b) * H + u0 + 16 * q;
      *reinterpret_cast<uint4 *>(a.cell_m + o) = mask_bits(v, 0);
      *reinterpret_cast<uint4 *>(a.cell_tanh_m + o) = mask_bits(v, 1);
      *reinterpret_cast<uint4 *>(a.hidden_m + o) = mask_bits(v, 2);
    }
  }
}

// Two codes as one word: code - lo of each, low half first.
__device__ __forceinline__ uint32_t lck_pair(float a, float b, int32_t lo) {
  return lck_u16(a, lo) | (lck_u16(b, lo) << 16);
}

// flush_step for the saved codes: the member's four blocks of the step (one contiguous run)
// and its four cell-code blocks of step t + 1, besides the output and the hidden codes.
__device__ __forceinline__ void flush_step_codes(const RecArgs &a, const StepParams &sp, int t,
                                                 int tile, int b0, int u0, float *xg,
                                                 const uint8_t *gm, const uint8_t *cm,
                                                 const float (&hvs)[2], const float (&cst)[2],
                                                 const float (&cts)[2], int srow, int su) {
  const int H = a.H, B = a.B, tid = threadIdx.x, nthr = blockDim.x;
  const size_t nt = static_cast<size_t>(B + 15) / 16;
  uint8_t *blk = a.ckb + ((static_cast<size_t>(t) * nt + tile) * (H / 16) + u0 / 16) * kLckBlock;
  uint16_t *cel = a.cellc + ((static_cast<size_t>(t + 1) * nt + tile) * (H / 16) + u0 / 16) * kLcellBlock;
  // gate codes [ut][16 rows][4 gates][16 units] from xg [(ut * 4 + g) * 16 + row][16], four
  // codes (8 bytes) per store
  for (int c = tid; c < 1024; c += nthr) {
    const int ut = c >> 8, R = (c >> 4) & 15, g = (c >> 2) & 3, qq = c & 3;
    // selected, not indexed: a kernel-argument array indexed at run time goes through scratch
    const int32_t lo = g == 0 ? sp.gout[0].lo : g == 1 ? sp.gout[1].lo : g == 2 ? sp.gout[2].lo
                                                                            : sp.gout[3].lo;
    const float4 v = *reinterpret_cast<const float4 *>(xg + ((ut * 4 + g) * 16 + R) * 16 + 4 * qq);
    *reinterpret_cast<uint2 *>(blk + ut * kLckBlock + ((R * 4 + g) * 16 + 4 * qq) * 2) =
        make_uint2(lck_pair(v.x, v.y, lo), lck_pair(v.z, v.w, lo));
  }
  // gate masks [ut][4 gates][16 rows][16 units], cell-phase masks [ut][16 rows][16 units]
  for (int c = (tid + nthr - 1024 % nthr) % nthr; c < 256 + 64; c += nthr) {
    if (c < 256) {
      const int ut = c >> 6, g = (c >> 4) & 3, R = c & 15;
      *reinterpret_cast<uint4 *>(blk + ut * kLckBlock + kLckGm + (g * 16 + R) * 16) =
          *reinterpret_cast<const uint4 *>(gm + (g * 16 + R) * kClUnits + 16 * ut);
    } else {
      const int ut = (c - 256) >> 4, R = (c - 256) & 15;
      *reinterpret_cast<uint4 *>(blk + ut * kLckBlock + kLckCm + R * 16) =
          *reinterpret_cast<const uint4 *>(cm + R * kClUnits + 16 * ut);
    }
  }
  __syncthreads();  // every read of xg is done
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    float *d = xg + (srow + rr) * kClUnits + su;
    d[0] = hvs[rr];
    d[16 * kClUnits] = cst[rr];
    d[32 * kClUnits] = cts[rr];
  }
  __syncthreads();
  flush_rows(a.output, xg, t, b0, B, H, u0, tid, nthr, true, sp.h.scale, sp.h.zp);
  flush_rows(a.hidden, xg, t, b0, B, H, u0, (tid + nthr - 256 % nthr) % nthr, nthr, false, 0.f, 0);
  // tanh(c) codes into the blocks, the cell codes into step t + 1's cell blocks
  for (int c = tid; c < 512; c += nthr) {
    const int k = c >> 8, ut = (c >> 6) & 3, R = (c >> 2) & 15, qq = c & 3;
    const float4 v = *reinterpret_cast<const float4 *>(xg + (k == 0 ? 32 : 16) * kClUnits +
                                                       R * kClUnits + 16 * ut + 4 * qq);
    const int32_t lo = k == 0 ? sp.tanh_c.lo : sp.c.lo;
    uint2 *dst = k == 0 ? reinterpret_cast<uint2 *>(blk + ut * kLckBlock + kLckTanh + (R * 16 + 4 * qq) * 2)
                        : reinterpret_cast<uint2 *>(cel + ut * kLcellBlock + R * 16 + 4 * qq);
    *dst = make_uint2(lck_pair(v.x, v.y, lo), lck_pair(v.z, v.w, lo));
  }
}

// The cell codes of c0 (step 0 of the cell-code array) from the c0 codes [B, H].
__global__ __launch_bounds__(256) void lstm_c0_codes(int B, int H, const float *__restrict__ c0q,
                                                     int32_t c_lo, uint16_t *__restrict__ cellc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(B) * H) return;
  const int b = static_cast<int>(i / H), j = static_cast<int>(i % H);
  cellc[static_cast<size_t>(lck_block(0, b, j, B, H)) * kLcellBlock + (b % 16) * 16 + j % 16] =
      static_cast<uint16_t>(lck_u16(c0q[i], c_lo));
}

// PW = 2: W_hh of up to 16 bits as two int8 planes, W = 256 bh + bl + 128 (lstm_pack_whh), so
// sum_k W y = 256 sum bh y + sum bl y + 128 sum_k y for each h plane y; the row sums sum_k y come
// from one more MFMA against a fragment of ones, and the planes are recombined in int64.
template <int NPL, int PW, bool EXC, bool CK>
__global__ __launch_bounds__(512) void lstm_recurrence_cl(RecArgs a, StepParams sp,
                                                          ClusterArgs cl) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 4 * H, B = a.B, KS = a.KS;
  v4i *wl = reinterpret_cast<v4i *>(smem);                       // [PW][4 gates][4 tiles][KS][64]
  float *xg = reinterpret_cast<float *>(wl + PW * 16 * KS * 64);  // [4 tiles][4 gates][16][16]
  // mask bits of a step (bit 0..2): gate phase [4 gates][16][64] (hh linear, gate in, gate out),
  // cell phase [16][64] (cell, cell tanh, hidden)
  uint8_t *gm = reinterpret_cast<uint8_t *>(xg + 4 * 4 * 16 * 16);
  uint8_t *cm = gm + 4 * 16 * kClUnits;
  uint32_t *lut = reinterpret_cast<uint32_t *>(cm + 16 * kClUnits);  // [cl.lut.total]
  for (int i = threadIdx.x; i < cl.lut.total; i += blockDim.x) lut[i] = cl.lut.table[i];
  const bool gate_lut = cl.lut.n[0] > 0, tanh_lut = cl.lut.tanh_n > 0;
  const bool gate_glut = cl.lut.gn[0] > 0, tanh_glut = cl.lut.gtanh_n > 0;
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int ut = w & 3, gp = w >> 2;
  const cluster::Place pl = cluster::place(cl.G, cl.ncl);
  const int u0 = pl.member * kClUnits;
  const int j = u0 + 16 * ut + l % 16;
  const int nrow0 = 4 * (l / 16);
  const size_t frag_plane = static_cast<size_t>(C / 16) * KS * 64;
  for (int i = tid; i < PW * 16 * KS * 64; i += blockDim.x) {
    const int pw = i / (16 * KS * 64), i1 = i % (16 * KS * 64);
    const int lane = i1 % 64, rest = i1 / 64, s = rest % KS, gt = rest / KS;
    const int ct = (gt / 4) * a.UT + u0 / 16 + gt % 4;
    wl[i] = a.frag[pw * frag_plane + (static_cast<size_t>(ct) * KS + s) * 64 + lane];
  }
  float4 cc[2];
  int64_t hk64[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = (2 * gp + q) * H + j;
    const ChanRun r = a.run[c];
    const ChanHost h = a.ch[c];
    cc[q] = make_float4(h.hh_mult, r.hh_bacc, __int_as_float(r.hh_k), __int_as_float(h.hh_shift));
    hk64[q] = (static_cast<int64_t>(r.hh_k_hi) << 32) | static_cast<uint32_t>(r.hh_k);
  }
  const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};
  unsigned *counter = cl.counters + cluster::kCounterStride * pl.cluster;
  unsigned epoch = 0;
  bool alive = true;
  const bool train = a.hidden != nullptr;
  const unsigned plane_stride = static_cast<unsigned>(cl.Bpad) * H;
  // the exchange buffer, 2 NPL planes (32-bit byte offsets: checked by the launcher)
  const auto xr = cluster::buffer_rsrc(cl.hx, 2u * NPL * plane_stride);

  for (int tile = pl.cluster; tile < cl.ntiles && alive; tile += cl.ncl) {
    const int b0 = tile * 16;
    float cst[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int b = b0 + nrow0 + 2 * gp + rr;
      const float q = b < B ? a.h0q[static_cast<size_t>(b) * H + j] : static_cast<float>(sp.h.zp);
      const int hc = static_cast<int>(q - a.h_offset);
      unsigned char *dst = reinterpret_cast<unsigned char *>(cl.hx) + static_cast<size_t>(b) * H + j;
#pragma unroll
      for (int p = 0; p < NPL; ++p)
        cluster::store_bytes_coherent(dst + p * plane_stride,
                                      NPL == 1 ? hc : (p == 0 ? (hc & 255) - 128 : hc >> 8));
      cst[rr] = b < B ? a.c0q[static_cast<size_t>(b) * H + j] : static_cast<float>(sp.c.zp);
    }
    // input branch of my two gates for my four rows, loaded one step ahead
    float lh[2][4];
    auto load_lhs = [&](int t) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int b = b0 + nrow0 + r;
          lh[q][r] = b < B ? a.lhs[(static_cast<size_t>(t) * B + b) * C + (2 * gp + q) * H + j]
                           : 0.0f;
        }
    };
    load_lhs(0);
    alive = cluster::sync(counter, ++epoch * cl.G, cl.timeout, cl.spin_limit);

    for (int t = 0; t < a.T && alive; ++t) {
      const int par = t & 1;
      const unsigned hin_off = par * NPL * plane_stride;  // byte offset of the step's planes
      int8_t *hout = cl.hx + static_cast<size_t>(par ^ 1) * NPL * plane_stride;
      v4i acc[2][PW][NPL], rs[NPL];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int pw = 0; pw < PW; ++pw)
#pragma unroll
          for (int p = 0; p < NPL; ++p) acc[q][pw][p] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < NPL; ++p) rs[p] = v4i{0, 0, 0, 0};
      if (NPL == 1 && kBT * (H + 16) <= static_cast<int>(sizeof(float)) * 4 * 4 * 16 * 16) {
        // The tile's h codes are read from the exchange buffer once per workgroup (one 16-byte
        // coherent load per thread and plane-chunk) into the gate exchange area, which is free
        // until the gate phase; the waves then take their A fragments from LDS.
        int8_t *hs = reinterpret_cast<int8_t *>(xg);
        const int rst = H + 16, cpr = H / 16, n = NPL * kBT * cpr;
        int4 hv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e0 = tid + 512 * i, e = e0 < n ? e0 : 0;
          const int p = e / (kBT * cpr), r = (e / cpr) % kBT, c = e % cpr;
          hv[i] = cluster::load_coherent16(xr, hin_off + p * plane_stride + (b0 + r) * H + 16 * c);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e = tid + 512 * i;
          if (e < n) {
            const int p = e / (kBT * cpr), r = (e / cpr) % kBT, c = e % cpr;
            *reinterpret_cast<int4 *>(hs + (p * kBT + r) * rst + 16 * c) = hv[i];
          }
        }
        __syncthreads();
        const int8_t *arow = hs + (l % 16) * rst + 16 * (l / 16);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if (s < KS) {
            v4i af[NPL];
#pragma unroll
            for (int p = 0; p < NPL; ++p)
              af[p] = *reinterpret_cast<const v4i *>(arow + p * kBT * rst + 64 * s);
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int pw = 0; pw < PW; ++pw) {
                const v4i bf = wl[((pw * 16 + (2 * gp + q) * 4 + ut) * KS + s) * 64 + l];
#pragma unroll
                for (int p = 0; p < NPL; ++p) acc[q][pw][p] = mfma_i8(af[p], bf, acc[q][pw][p]);
              }
            if constexpr (PW == 2) {
#pragma unroll
              for (int p = 0; p < NPL; ++p) rs[p] = mfma_i8(af[p], ones, rs[p]);
            }
          }
        }
        __syncthreads();  // the gate phase rewrites the area
      } else {
        // all of the step's h fragments in flight at once (KS <= 8; <= 4 with two W planes)
        constexpr int kKS = PW == 2 ? 4 : 8;
        v4i hfr[kKS][NPL];
#pragma unroll
        for (int s = 0; s < kKS; ++s)
#pragma unroll
          for (int p = 0; p < NPL; ++p)
            if (s < KS) {
              const int4 v = cluster::load_coherent16(
                  xr, hin_off + (b0 + l % 16) * H + 16 * (l / 16) + p * plane_stride + 64 * s);
              hfr[s][p] = v4i{v.x, v.y, v.z, v.w};
            }
#pragma unroll
        for (int s = 0; s < kKS; ++s) {
          if (s < KS) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
              for (int pw = 0; pw < PW; ++pw) {
                const v4i bf = wl[((pw * 16 + (2 * gp + q) * 4 + ut) * KS + s) * 64 + l];
#pragma unroll
                for (int p = 0; p < NPL; ++p)
                  acc[q][pw][p] = mfma_i8(hfr[s][p], bf, acc[q][pw][p]);
              }
            if constexpr (PW == 2) {
#pragma unroll
              for (int p = 0; p < NPL; ++p) rs[p] = mfma_i8(hfr[s][p], ones, rs[p]);
            }
          }
        }
      }
      // gate phase: two gates x four rows; the gate pair is a compile-time constant so the
      // per-gate parameters are static kernel-argument reads
      auto gate_phase = [&](auto gpc) {
        constexpr int GP = decltype(gpc)::value;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int nr = nrow0 + r, b = b0 + nr;
          const bool valid = b < B;
          const uint32_t oc = (static_cast<uint32_t>(t) * B + b) * static_cast<uint32_t>(C) + j;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            constexpr int g0 = 2 * GP;
            const int g = g0 + q;
            const Grid &gin = q == 0 ? sp.gin[g0] : sp.gin[g0 + 1];
            const Grid &gout = q == 0 ? sp.gout[g0] : sp.gout[g0 + 1];
            const Rescale &h2g = q == 0 ? sp.hh_to_gate[g0] : sp.hh_to_gate[g0 + 1];
            float accf;
            if constexpr (PW == 1) {
              int v = pick(acc[q][0][0], r);
              if constexpr (NPL == 2) v += 256 * pick(acc[q][0][NPL - 1], r);
              v += __float_as_int(cc[q].z);
              accf = static_cast<float>(v) + cc[q].y;
            } else {
              int64_t v = hk64[q];
#pragma unroll
              for (int p = 0; p < NPL; ++p) {
                const int64_t sp_ = 256 * static_cast<int64_t>(pick(acc[q][1][p], r)) +
                                    pick(acc[q][0][p], r) + 128 * static_cast<int64_t>(pick(rs[p], r));
                v += p == 0 ? sp_ : 256 * sp_;
              }
              accf = static_cast<float>(v) + cc[q].y;
            }
            uint8_t m_hl, m_gi, m_go;
            const float lin = clamp_grid_f(rescale(accf, cc[q].x, __float_as_int(cc[q].w)),
                                           sp.hh_lin, m_hl);
            const float rhs = rescale(center_f(lin, sp.hh_lin.zp), h2g.mult, h2g.shift);
            const float gi = clamp_grid_f(lh[q][r] + rhs, gin, m_gi);
            const float go =
                gate_lut
                    ? lut_code(lut + (q == 0 ? cl.lut.off[g0] : cl.lut.off[g0 + 1]),
                               static_cast<int>(gi) - gin.lo, gout.lo, m_go)
                    : (gate_glut
                           ? lut_code(cl.lut.gtable + (q == 0 ? cl.lut.goff[g0] : cl.lut.goff[g0 + 1]),
                                      static_cast<int>(gi) - gin.lo, gout.lo, m_go)
                           : real_act<EXC>(gi, gin, gout, g == 2, sp, g, m_go));
            xg[((ut * 4 + g) * 16 + nr) * 16 + l % 16] = go;
            // (the codes kernel always stages: the launcher runs it only with wide_out set)
            if (CK || a.wide_out) {
              if (train)
                gm[(g * 16 + nr) * kClUnits + 16 * ut + l % 16] =
                    static_cast<uint8_t>(m_hl | (m_gi << 1) | (m_go << 2));
            } else if (train && valid) {
              a.gate_out[oc + g * H] = go;
              a.hh_lin_m[oc + g * H] = m_hl;
              a.gate_in_m[oc + g * H] = m_gi;
              a.gate_out_m[oc + g * H] = m_go;
            }
          }
        }
      };
      if (gp == 0)
        gate_phase(std::integral_constant<int, 0>{});
      else
        gate_phase(std::integral_constant<int, 1>{});
      if (t + 1 < a.T) load_lhs(t + 1);
      __syncthreads();
      // cell phase: rows 2 gp, 2 gp + 1 of the lane's four
      float hvs[2], cts[2];
      uint8_t mcs[2], mts[2], mhs[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int nr = nrow0 + 2 * gp + rr, b = b0 + nr;
        float gout[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) gout[g] = xg[((ut * 4 + g) * 16 + nr) * 16 + l % 16];
        const float pf = center_f(gout[1], sp.gout[1].zp) * center_f(cst[rr], sp.c.zp);
        const float pi = center_f(gout[0], sp.gout[0].zp) * center_f(gout[2], sp.gout[2].zp);
        const float sum = cell_scale(pf, sp, 0) + cell_scale(pi, sp, 1);
        const float cn = clamp_grid_f(rintf(sum), sp.c, mcs[rr]);
        cst[rr] = cn;
        cts[rr] =
            tanh_lut ? lut_code(lut + cl.lut.tanh_off, static_cast<int>(cn) - sp.c.lo,
                                sp.tanh_c.lo, mts[rr])
                     : (tanh_glut ? lut_code(cl.lut.gtable + cl.lut.gtanh_off,
                                             static_cast<int>(cn) - sp.c.lo, sp.tanh_c.lo, mts[rr])
                                  : real_act<EXC>(cn, sp.c, sp.tanh_c, true, sp, 4, mts[rr]));
        const float raw = center_f(gout[3], sp.gout[3].zp) * center_f(cts[rr], sp.tanh_c.zp);
        hvs[rr] = clamp_grid_f(rescale(raw, sp.hidden.mult, sp.hidden.shift), sp.h, mhs[rr]);
        if ((CK || a.wide_out) && train)
          cm[nr * kClUnits + 16 * ut + l % 16] =
              static_cast<uint8_t>(mcs[rr] | (mts[rr] << 1) | (mhs[rr] << 2));
        const int hc = static_cast<int>(hvs[rr] - a.h_offset);
        unsigned char *dst = reinterpret_cast<unsigned char *>(hout) + static_cast<size_t>(b) * H + j;
#pragma unroll
        for (int p = 0; p < NPL; ++p)
          cluster::store_bytes_coherent(dst + p * plane_stride,
                                        NPL == 1 ? hc : (p == 0 ? (hc & 255) - 128 : hc >> 8));
      }
      // the other members only read the h codes: arrive, then store outputs while waiting
      cluster::arrive(counter);
      ++epoch;
      if (CK || a.wide_out) {
        if constexpr (CK)
          flush_step_codes(a, sp, t, tile, b0, u0, xg, gm, cm, hvs, cst, cts, nrow0 + 2 * gp,
                           16 * ut + l % 16);
        else
          flush_step(a, sp, t, b0, u0, train, xg, gm, cm, hvs, cst, cts, nrow0 + 2 * gp,
                     16 * ut + l % 16);
        if (t == a.T - 1) {
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const int b = b0 + nrow0 + 2 * gp + rr;
            if (b >= B) continue;
            const uint32_t os = static_cast<uint32_t>(b) * H + j;
            a.h_n[os] = dequant_f(hvs[rr], sp.h.scale, sp.h.zp);
            a.c_n[os] = dequant_f(cst[rr], sp.c.scale, sp.c.zp);
          }
        }
      } else {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int b = b0 + nrow0 + 2 * gp + rr;
        if (b >= B) continue;
        const float hv = hvs[rr], cn = cst[rr];
        const uint32_t oh = (static_cast<uint32_t>(t) * B + b) * static_cast<uint32_t>(H) + j;
        a.output[oh] = dequant_f(hv, sp.h.scale, sp.h.zp);
        if (train) {
          a.cell[oh] = cn;
          a.cell_tanh[oh] = cts[rr];
          a.hidden[oh] = hv;
          a.cell_m[oh] = mcs[rr];
          a.cell_tanh_m[oh] = mts[rr];
          a.hidden_m[oh] = mhs[rr];
        }
        if (t == a.T - 1) {
          const uint32_t os = static_cast<uint32_t>(b) * H + j;
          a.h_n[os] = dequant_f(hv, sp.h.scale, sp.h.zp);
          a.c_n[os] = dequant_f(cn, sp.c.scale, sp.c.zp);
        }
      }
      }
      alive = cluster::wait(counter, epoch * cl.G, cl.timeout, cl.spin_limit);
    }
  }
}

size_t recurrence_cl_lds(int KS, int pw, int lut_entries) {
  return sizeof(v4i) * pw * 16 * static_cast<size_t>(KS) * 64 + sizeof(float) * 4 * 4 * 16 * 16 +
         5 * 16 * kClUnits + sizeof(uint32_t) * static_cast<size_t>(lut_entries);
}

// Outputs of a launch whose cluster wait timed out are not trustworthy: overwrite them with NaN.
__global__ __launch_bounds__(256) void lstm_poison_on_timeout(const int *timeout, int64_t n_out,
                                                              float *output, int64_t n_state,
                                                              float *h_n, float *c_n) {
  if (*timeout == 0) return;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_out; i += stride)
    output[i] = NAN;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_state;
       i += stride) {
    h_n[i] = NAN;
    c_n[i] = NAN;
  }
}

size_t recurrence_lds(int H, int KS, int npl) {
  return sizeof(float4) * 4 * static_cast<size_t>(H) + sizeof(float) * kBT * static_cast<size_t>(H) +
         static_cast<size_t>(2) * npl * kBT * (KS * 64 + 16);
}

struct FwdWorkspace {
  size_t chost, run, frag, lhs, xq, wih, whh, bih, bhh, h0q, c0q, hx, sync, lut, glut, exc, xa,
      bfrag, colsum, sh, sc, sg, total;
  FwdWorkspace(int T, int B, int I, int H) {
    const size_t C = 4 * static_cast<size_t>(H), KS = (H + 63) / 64;
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t o = 0;
    chost = o; o += al(sizeof(ChanHost) * C);
    run = o; o += al(sizeof(ChanRun) * C);
    frag = o; o += al(sizeof(v4i) * 64 * (C / 16) * KS * 2);  // up to two W_hh planes
    lhs = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * C);
    // codes used internally when the caller keeps no checkpoints
    xq = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * I);
    wih = o; o += al(sizeof(float) * C * I);
    whh = o; o += al(sizeof(float) * C * H);
    bih = o; o += al(sizeof(float) * C);
    bhh = o; o += al(sizeof(float) * C);
    h0q = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    c0q = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    // clustered recurrence: h exchange planes (two parities, up to two planes) and counters
    const size_t Bpad = (static_cast<size_t>(B) + 15) / 16 * 16;
    hx = o; o += al(2 * 2 * Bpad * H);
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (Bpad / 16 + 1));
    lut = o; o += al(sizeof(uint32_t) * 2 * kLutMaxEntries);
    glut = o; o += al(sizeof(uint32_t) * 5 * static_cast<size_t>(kGlobalLutMaxCodes));
    // reference activation exceptions: keys, then entries, of at most 5 full 16-bit grids
    exc = o; o += al(sizeof(int32_t) * 2 * 5 * static_cast<size_t>(kActExcMaxCodes));
    // packed operands of the input linear (I <= 256): x planes, W_ih fragments, column sums
    const size_t Kp = static_cast<size_t>(xgemm::pad_k(I));
    const size_t ip = static_cast<size_t>(I) <= kPackedMaxK ? 1 : 0;
    xa = o; o += al(ip * 2 * static_cast<size_t>(T) * B * Kp);
    bfrag = o; o += al(ip * 2 * ((C + 15) / 16 * 16) * Kp);  // fragments of 16-column tiles
    colsum = o; o += al(ip * sizeof(long long) * C);
    // stepped recurrence: two h code buffers, the cell codes [B, H] and the sums [B, 4H]
    sh = o; o += al(sizeof(float) * 2 * static_cast<size_t>(B) * H);
    sc = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    sg = o; o += al(sizeof(float) * static_cast<size_t>(B) * C);
    total = o;
  }
};

}  // namespace lstm
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::lstm;

extern "C" {

int64_t rxmet_lstm_forward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  if (T < 1 || B < 1 || I < 1 || H < 1) return 0;
  return static_cast<int64_t>(FwdWorkspace(T, B, I, H).total);
}

static int lstm_forward_impl(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0,
                             const rxmet_lstm_params *params, float *output, float *h_n,
                             float *c_n, const rxmet_lstm_saved *saved,
                             const rxmet_lstm_saved_codes *codes, void *workspace, void *stream_) {
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H % 16 == 0, "hidden_size must be a multiple of 16");
  RXMET_CHECK_ARG(W_ih && W_hh && x && params && output && h_n && c_n && workspace,
                  "required pointer is null");
  RXMET_CHECK_ARG((h0 == nullptr) == (c0 == nullptr), "h0 and c0 must be given together");
  RXMET_CHECK_ARG(params->hidden == H, "params hidden size does not match");
  const bool bias = params->bias_enabled != 0;
  RXMET_CHECK_ARG(!bias || (b_ih && b_hh), "bias enabled but bias pointers are null");
  const rxmet_lstm_op_config &h_t = params->config.op[RXMET_LSTM_OUTPUT];
  RXMET_CHECK_ARG(h_t.bits <= 16, "output (h) wider than 16 bits is not supported");
  RXMET_CHECK_ARG(static_cast<double>(T) * B * 4 * H < 4294967295.0,
                  "T*B*4H too large for 32-bit element offsets");
  if (saved && codes) {
    RXMET_CHECK_ARG(saved->x_q && saved->w_ih_q && saved->w_hh_q && saved->h0_q && saved->c0_q &&
                        saved->x_m && saved->w_ih_m && saved->w_hh_m && saved->h0_m &&
                        saved->c0_m && saved->hidden && saved->ih_linear_m && codes->blocks &&
                        codes->cell_codes,
                    "training forward needs the masters, hidden, ih_linear_m and the codes");
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    RXMET_CHECK_ARG(a16(codes->blocks) && a16(codes->cell_codes),
                    "the saved codes must be 16-byte aligned");
  } else if (saved) {
    RXMET_CHECK_ARG(saved->x_q && saved->w_ih_q && saved->w_hh_q && saved->h0_q && saved->c0_q &&
                        saved->x_m && saved->w_ih_m && saved->w_hh_m && saved->h0_m &&
                        saved->c0_m && saved->gate_out && saved->cell && saved->cell_tanh &&
                        saved->hidden && saved->ih_linear_m && saved->hh_linear_m &&
                        saved->gate_in_m && saved->gate_out_m && saved->cell_m &&
                        saved->cell_tanh_m && saved->hidden_m,
                    "training forward needs every saved tensor");
    RXMET_CHECK_ARG(!bias || (saved->b_ih_q && saved->b_hh_q && saved->b_ih_m && saved->b_hh_m),
                    "training forward with bias needs the saved bias codes and masks");
  }
  StepParams sp;
  ChannelParams cp;
  if (int rc = derive(*params, &sp, &cp)) return rc;
  if (saved && codes) {
    bool fit = sp.c.hi - sp.c.lo <= 65535 && sp.tanh_c.hi - sp.tanh_c.lo <= 65535;
    for (int g = 0; g < 4; ++g) fit = fit && sp.gout[g].hi - sp.gout[g].lo <= 65535;
    RXMET_CHECK_ARG(fit, "saved codes need gate-output, cell and tanh grids of at most 16 bits");
  }
  const int C = 4 * H, KS = (H + 63) / 64, UT = H / 16;
  // the input branch is an exact byte-plane GEMM; the recurrent MFMA sum must fit int32
  RXMET_CHECK_ARG(I < (1 << 17), "input_size must be below 131072 for the exact input GEMM");
  RXMET_CHECK_ARG(xgemm::a_fits(sp.x.lo, sp.x.hi), "input codes must span at most 16 bits");
  const Grid gwh_t = grid_of(params->config.op[RXMET_LSTM_W_HH], 1.0f, 0);
  RXMET_CHECK_ARG(xgemm::b_fits(gwh_t.lo, gwh_t.hi), "W_hh codes must fit signed 16 bits");
  RXMET_CHECK_ARG(xgemm::a_fits(sp.h.lo, sp.h.hi), "h codes must span at most 16 bits");
  // the MFMA recurrences hold W_hh as int8 fragments and keep at most 512 units per batch tile;
  // one W_hh plane sums in int32; two planes (W_hh of 9-16 bits) only in the clustered
  // recurrence, for H a multiple of 64 up to 256 (both planes resident in LDS), summed in int64;
  // anything else steps
  const int pw = xgemm::b_planes(gwh_t.lo, gwh_t.hi);
  bool f32_grids = fits_f32(sp.hh_lin) && fits_f32(sp.c) && fits_f32(sp.tanh_c) && fits_f32(sp.h);
  for (int g = 0; g < 4; ++g) f32_grids = f32_grids && fits_f32(sp.gin[g]) && fits_f32(sp.gout[g]);
  const bool may_cluster = H % kClUnits == 0 && f32_grids &&
                           std::getenv("RXMET_NO_CLUSTER") == nullptr;
  const bool stepped = (pw > 1 && !(may_cluster && H <= 256)) || H > kMaxH ||
                       (pw == 1 && !(std::ldexp(1.0, h_t.bits) * 128.0 * H < 2147483647.0)) ||
                       std::getenv("RXMET_LSTM_STEPPED") != nullptr;

  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const FwdWorkspace ws(T, B, I, H);
  char *wsb = static_cast<char *>(workspace);
  const ActExceptions exc = act_exceptions(sp);
  if (!exc.key.empty()) {
    int32_t *ek = reinterpret_cast<int32_t *>(wsb + ws.exc);
    uint32_t *ev = reinterpret_cast<uint32_t *>(ek + 5 * static_cast<size_t>(kActExcMaxCodes));
    if (int rc = upload(ek, exc.key.data(), sizeof(int32_t) * exc.key.size(), stream)) return rc;
    if (int rc = upload(ev, exc.val.data(), sizeof(uint32_t) * exc.val.size(), stream)) return rc;
    sp.exc_key = ek;
    sp.exc_val = ev;
    for (int k = 0; k < 5; ++k) {
      sp.exc_off[k] = exc.off[k];
      sp.exc_n[k] = exc.n[k];
    }
  }
  std::vector<ChanHost> hostc(C);
  for (int c = 0; c < C; ++c) {
    ChanHost &h = hostc[c];
    h.w_ih_s = cp.w_ih_scale[c];
    h.w_hh_s = cp.w_hh_scale[c];
    h.b_ih_s = bias ? cp.b_ih_scale[c] : 1.0f;
    h.b_hh_s = bias ? cp.b_hh_scale[c] : 1.0f;
    h.ih_mult = cp.ih_acc_to_lin[c].mult;
    h.ih_shift = cp.ih_acc_to_lin[c].shift;
    h.hh_mult = cp.hh_acc_to_lin[c].mult;
    h.hh_shift = cp.hh_acc_to_lin[c].shift;
    h.ih_bmult = cp.ih_bias_to_acc[c].mult;
    h.ih_bshift = cp.ih_bias_to_acc[c].shift;
    h.hh_bmult = cp.hh_bias_to_acc[c].mult;
    h.hh_bshift = cp.hh_bias_to_acc[c].shift;
  }
  ChanHost *chost = reinterpret_cast<ChanHost *>(wsb + ws.chost);
  ChanRun *run = reinterpret_cast<ChanRun *>(wsb + ws.run);
  v4i *frag = reinterpret_cast<v4i *>(wsb + ws.frag);
  float *lhs = reinterpret_cast<float *>(wsb + ws.lhs);
  if (int rc = upload(chost, hostc.data(), sizeof(ChanHost) * C, stream)) return rc;
  const rxmet_lstm_saved sv = saved ? *saved : rxmet_lstm_saved{};
  float *xq = saved ? sv.x_q : reinterpret_cast<float *>(wsb + ws.xq);
  float *wih = saved ? sv.w_ih_q : reinterpret_cast<float *>(wsb + ws.wih);
  float *whh = saved ? sv.w_hh_q : reinterpret_cast<float *>(wsb + ws.whh);
  float *bih = (saved && bias) ? sv.b_ih_q : reinterpret_cast<float *>(wsb + ws.bih);
  float *bhh = (saved && bias) ? sv.b_hh_q : reinterpret_cast<float *>(wsb + ws.bhh);
  float *h0q = saved ? sv.h0_q : reinterpret_cast<float *>(wsb + ws.h0q);
  float *c0q = saved ? sv.c0_q : reinterpret_cast<float *>(wsb + ws.c0q);

  const int npl = h_t.bits <= 8 ? 1 : 2;
  const float h_offset = (h_t.is_unsigned && h_t.bits < 32) ? std::ldexp(1.0f, h_t.bits - 1) : 0.0f;
  WeightArgs wa;
  wa.I = I; wa.H = H; wa.bias = bias ? 1 : 0; wa.npl = npl;
  wa.W_ih = W_ih; wa.W_hh = W_hh; wa.b_ih = b_ih; wa.b_hh = b_hh; wa.ch = chost;
  wa.wq_ih = wih; wa.wq_hh = whh; wa.bq_ih = bih; wa.bq_hh = bhh;
  wa.wm_ih = sv.w_ih_m; wa.wm_hh = sv.w_hh_m; wa.bm_ih = sv.b_ih_m; wa.bm_hh = sv.b_hh_m;
  wa.run = run;
  wa.hh_k_factor = static_cast<int32_t>(h_offset) - sp.h.zp + (npl == 2 ? 128 : 0);
  const rxmet_lstm_op_config *oc = params->config.op;
  const Grid gwi = grid_of(oc[RXMET_LSTM_W_IH], 1.0f, 0), gwh = grid_of(oc[RXMET_LSTM_W_HH], 1.0f, 0);
  const Grid gbi = grid_of(oc[RXMET_LSTM_B_IH], 1.0f, 0), gbh = grid_of(oc[RXMET_LSTM_B_HH], 1.0f, 0);
  {
    rxmet::prof::Scope ps__("lstm_fwd_quant_weights", stream);
    hipLaunchKernelGGL(lstm_quant_weights, dim3(C), dim3(64), 0, stream, wa, gwi, gwh, gbi, gbh);
  }
  RXMET_CHECK_LAUNCH();
  const int64_t nx = static_cast<int64_t>(T) * B * I, nh = static_cast<int64_t>(B) * H;
  int64_t blocks = (nx + nh + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(lstm_quant_inputs, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     nx, nh, x, h0, c0, sp, xq, sv.x_m, h0q, sv.h0_m, c0q, sv.c0_m);
  RXMET_CHECK_LAUNCH();
  if (!stepped) {
    hipLaunchKernelGGL(lstm_pack_whh, dim3((C / 16) * KS), dim3(64), 0, stream, H, KS, pw,
                       static_cast<size_t>(C / 16) * KS * 64, whh, frag);
    RXMET_CHECK_LAUNCH();
  }
  const int M = T * B;
  {
    RXMET_CHECK_ARG(xgemm::b_fits(gwi.lo, gwi.hi), "W_ih codes must be signed 16-bit at most");
    const float off = xgemm::a_shift(sp.x.lo, sp.x.hi);
    const int pa = xgemm::a_planes(sp.x.lo, sp.x.hi), pb = xgemm::b_planes(gwi.lo, gwi.hi);
    rxmet::prof::Scope ps__("lstm_fwd_input_gemm", stream);
    if (I <= kPackedMaxK) {
      const int Kp = xgemm::pad_k(I);
      int8_t *xa = reinterpret_cast<int8_t *>(wsb + ws.xa);
      v4i *bf = reinterpret_cast<v4i *>(wsb + ws.bfrag);
      long long *cs = reinterpret_cast<long long *>(wsb + ws.colsum);
      if (int rc = xgemm::pack_a(xq, I, M, I, off, pa, xa, Kp, stream)) return rc;
      if (int rc = xgemm::pack_b(wih, 1, I, I, C, pb, Kp, bf, cs, stream)) return rc;
      xgemm::Packed p;
      p.A = xa; p.aplane = static_cast<int64_t>(M) * Kp; p.Kp = Kp;
      p.B = bf; p.bplane = static_cast<int64_t>((C + 15) / 16) * (Kp / 64) * 64;
      p.colsum = cs; p.corr = static_cast<long long>(off) - sp.x.zp; p.M = M; p.N = C;
      const dim3 grid((M + 15) / 16);
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, p, H, chost, run, sp, lhs,
                           sv.ih_linear_m);
      };
      const bool f32 = fits_f32(sp.ih_lin);
      if (pa == 1 && pb == 1)
        f32 ? go(lstm_input_gemm_packed<1, 1, true>) : go(lstm_input_gemm_packed<1, 1, false>);
      else if (pa == 1)
        f32 ? go(lstm_input_gemm_packed<1, 2, true>) : go(lstm_input_gemm_packed<1, 2, false>);
      else if (pb == 1)
        f32 ? go(lstm_input_gemm_packed<2, 1, true>) : go(lstm_input_gemm_packed<2, 1, false>);
      else
        f32 ? go(lstm_input_gemm_packed<2, 2, true>) : go(lstm_input_gemm_packed<2, 2, false>);
    } else {
      xgemm::Operands o;
      o.M = M; o.N = C; o.K = I;
      o.A = xq; o.lda = I;
      o.off = off;
      o.corr = static_cast<long long>(o.off) - sp.x.zp;
      o.B = wih; o.sbk = 1; o.sbn = I;  // W_ih codes [4H][I]
      const dim3 grid((C + 63) / 64, (M + 63) / 64);
      if (pa == 1 && pb == 1)
        hipLaunchKernelGGL((lstm_input_gemm<1, 1>), grid, dim3(256), 0, stream, o, H, chost, run, sp,
                           lhs, sv.ih_linear_m);
      else if (pa == 1)
        hipLaunchKernelGGL((lstm_input_gemm<1, 2>), grid, dim3(256), 0, stream, o, H, chost, run, sp,
                           lhs, sv.ih_linear_m);
      else if (pb == 1)
        hipLaunchKernelGGL((lstm_input_gemm<2, 1>), grid, dim3(256), 0, stream, o, H, chost, run, sp,
                           lhs, sv.ih_linear_m);
      else
        hipLaunchKernelGGL((lstm_input_gemm<2, 2>), grid, dim3(256), 0, stream, o, H, chost, run, sp,
                           lhs, sv.ih_linear_m);
    }
  }
  RXMET_CHECK_LAUNCH();

  RecArgs ra;
  ra.T = T; ra.B = B; ra.H = H; ra.KS = KS; ra.UT = UT; ra.h_offset = h_offset;
  ra.lhs = lhs; ra.frag = frag; ra.ch = chost; ra.run = run; ra.h0q = h0q; ra.c0q = c0q;
  ra.output = output; ra.h_n = h_n; ra.c_n = c_n;
  ra.gate_out = sv.gate_out; ra.cell = sv.cell; ra.cell_tanh = sv.cell_tanh; ra.hidden = sv.hidden;
  ra.hh_lin_m = sv.hh_linear_m; ra.gate_in_m = sv.gate_in_m; ra.gate_out_m = sv.gate_out_m;
  ra.cell_m = sv.cell_m; ra.cell_tanh_m = sv.cell_tanh_m; ra.hidden_m = sv.hidden_m;
  ra.ckb = nullptr; ra.cellc = nullptr;
  if (saved && codes) {
    ra.gate_out = ra.cell = ra.cell_tanh = nullptr;
    ra.hh_lin_m = ra.gate_in_m = ra.gate_out_m = ra.cell_m = ra.cell_tanh_m = ra.hidden_m = nullptr;
    ra.ckb = codes->blocks;
    ra.cellc = codes->cell_codes;
    const int64_t n = static_cast<int64_t>(B) * H;
    hipLaunchKernelGGL(lstm_c0_codes, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       stream, B, H, c0q, sp.c.lo, ra.cellc);
    RXMET_CHECK_LAUNCH();
  }
  {
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    bool wide = H % 16 == 0 && a16(ra.output);
    if (ra.ckb != nullptr)
      wide = wide && a16(ra.hidden);
    else if (ra.hidden != nullptr)
      wide = wide && a16(ra.gate_out) && a16(ra.cell) && a16(ra.cell_tanh) && a16(ra.hidden) &&
             a16(ra.hh_lin_m) && a16(ra.gate_in_m) && a16(ra.gate_out_m) && a16(ra.cell_m) &&
             a16(ra.cell_tanh_m) && a16(ra.hidden_m);
    ra.wide_out = wide ? 1 : 0;
  }
  auto run_stepped = [&]() -> int {
    float *hb = reinterpret_cast<float *>(wsb + ws.sh);
    float *cs = reinterpret_cast<float *>(wsb + ws.sc);
    float *ghh = reinterpret_cast<float *>(wsb + ws.sg);
    const int pa = xgemm::a_planes(sp.h.lo, sp.h.hi), pb = xgemm::b_planes(gwh_t.lo, gwh_t.hi);
    xgemm::Operands o{};
    o.M = B; o.N = C; o.K = H;
    o.lda = H;
    o.off = xgemm::a_shift(sp.h.lo, sp.h.hi);
    o.corr = static_cast<long long>(o.off) - sp.h.zp;  // sums of (h - zp_h) W_hh
    o.B = whh; o.sbk = 1; o.sbn = H;                    // W_hh codes [4H][H]
    const dim3 ggrid((B + xgemm::kTile - 1) / xgemm::kTile, (C + xgemm::kTile - 1) / xgemm::kTile);
    const int64_t n = static_cast<int64_t>(B) * H;
    const dim3 pgrid(static_cast<unsigned>((n + 255) / 256));
    rxmet::prof::Scope ps__("lstm_fwd_recurrence", stream);
    const float *hcur = h0q, *cin = c0q;
    for (int t = 0; t < T; ++t) {
      float *hnext = hb + static_cast<size_t>(t & 1) * n;
      o.A = hcur;
      if (pa == 1 && pb == 1)
        hipLaunchKernelGGL((lstm_step_gemm<1, 1>), ggrid, dim3(256), 0, stream, o, ghh);
      else if (pa == 1)
        hipLaunchKernelGGL((lstm_step_gemm<1, 2>), ggrid, dim3(256), 0, stream, o, ghh);
      else if (pb == 1)
        hipLaunchKernelGGL((lstm_step_gemm<2, 1>), ggrid, dim3(256), 0, stream, o, ghh);
      else
        hipLaunchKernelGGL((lstm_step_gemm<2, 2>), ggrid, dim3(256), 0, stream, o, ghh);
      RXMET_CHECK_LAUNCH();
      hipLaunchKernelGGL(lstm_step_point, pgrid, dim3(256), 0, stream, ra, sp, t, ghh, cin, cs,
                         hnext);
      RXMET_CHECK_LAUNCH();
      hcur = hnext;
      cin = cs;
    }
    return 0;
  };
  if (stepped) return run_stepped();
  if (may_cluster) {
    // clustered path when the whole grid can be resident at once
    const bool has_exc = !exc.key.empty();
#define RXMET_LSTM_CL(N, P, E)                                                         \
  {reinterpret_cast<const void *>(&lstm_recurrence_cl<N, P, E, false>),              \
   reinterpret_cast<const void *>(&lstm_recurrence_cl<N, P, E, true>)}
    const void *fns[2][2][2][2] = {
        {{RXMET_LSTM_CL(1, 1, false), RXMET_LSTM_CL(1, 1, true)},
         {RXMET_LSTM_CL(1, 2, false), RXMET_LSTM_CL(1, 2, true)}},
        {{RXMET_LSTM_CL(2, 1, false), RXMET_LSTM_CL(2, 1, true)},
         {RXMET_LSTM_CL(2, 2, false), RXMET_LSTM_CL(2, 2, true)}}};
#undef RXMET_LSTM_CL
    const void *fn = fns[npl - 1][pw - 1][has_exc ? 1 : 0][ra.ckb != nullptr ? 1 : 0];
    ActLut lut{};
    uint32_t *lut_table = reinterpret_cast<uint32_t *>(wsb + ws.lut);
    int dev_lds = 0;
    {
      int dev = 0;
      RXMET_CHECK_HIP(hipGetDevice(&dev));
      RXMET_CHECK_HIP(hipDeviceGetAttribute(&dev_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
      // table entries that fit beside the resident weights and the gate exchange
      const int64_t room = (static_cast<int64_t>(dev_lds) -
                            static_cast<int64_t>(recurrence_cl_lds(KS, pw, 0))) / 4;
      int64_t n[4], tot = 0;
      for (int g = 0; g < 4; ++g) {
        n[g] = static_cast<int64_t>(sp.gin[g].hi) - sp.gin[g].lo + 1;
        tot += n[g];
      }
      if (tot <= kLutMaxEntries && tot <= room) {
        for (int g = 0, o = 0; g < 4; ++g) {
          lut.off[g] = o;
          lut.n[g] = static_cast<int>(n[g]);
          o += lut.n[g];
        }
        lut.total = static_cast<int>(tot);
      }
      const int64_t nc = static_cast<int64_t>(sp.c.hi) - sp.c.lo + 1;
      if (nc <= kLutMaxEntries && lut.total + nc <= room) {
        lut.tanh_off = lut.total;
        lut.tanh_n = static_cast<int>(nc);
        lut.total += lut.tanh_n;
      }
      lut.table = lut_table;
      // global tables for what LDS does not hold
      bool gates_fit = lut.n[0] == 0;
      for (int g = 0; g < 4; ++g) gates_fit = gates_fit && n[g] <= kGlobalLutMaxCodes;
      if (gates_fit) {
        for (int g = 0, o = 0; g < 4; ++g) {
          lut.goff[g] = o;
          lut.gn[g] = static_cast<int>(n[g]);
          o += lut.gn[g];
        }
        lut.gtotal = static_cast<int>(tot);
      }
      if (lut.tanh_n == 0 && nc <= kGlobalLutMaxCodes && exc.n[4] > 0) {
        lut.gtanh_off = lut.gtotal;
        lut.gtanh_n = static_cast<int>(nc);
        lut.gtotal += lut.gtanh_n;
      }
      lut.gtable = reinterpret_cast<uint32_t *>(wsb + ws.glut);
    }
    const size_t lds_cl = recurrence_cl_lds(KS, pw, lut.total);
    if (static_cast<int64_t>(lds_cl) > dev_lds) {
      RXMET_CHECK_ARG(pw == 2, "clustered recurrence does not fit in LDS");
      return run_stepped();  // the two W_hh planes do not fit beside the exchange areas
    }
    int device = 0, ncu = 0, per_cu = 0;
    RXMET_CHECK_HIP(hipGetDevice(&device));
    RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
    RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds_cl)));
    RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 512, lds_cl));
    ClusterArgs cl;
    cl.G = H / kClUnits;
    cl.ntiles = (B + kBT - 1) / kBT;
    cl.Bpad = cl.ntiles * kBT;
    int ncl = per_cu * ncu / cl.G;
    if (ncl > cl.ntiles) ncl = cl.ntiles;
    if (ncl >= 8) ncl -= ncl % 8;
    // (the exchange buffer, 2 npl planes of Bpad H bytes, is addressed with 32-bit offsets)
    if (ncl >= 1 && 4.0 * cl.Bpad * H < 2147483648.0 && std::getenv("RXMET_NO_CLUSTER") == nullptr &&
        (ra.ckb == nullptr || ra.wide_out)) {
      cl.ncl = ncl;
      cl.hx = reinterpret_cast<int8_t *>(wsb + ws.hx);
      cl.counters = reinterpret_cast<unsigned *>(wsb + ws.sync);
      cl.timeout = reinterpret_cast<int *>(cl.counters + cluster::kCounterStride * ncl);
      cl.spin_limit = cluster::spin_limit();
      cl.lut = lut;
      hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, cl.counters,
                     cluster::kCounterStride * ncl + 1);
      RXMET_CHECK_LAUNCH();
      const int n_exc = static_cast<int>(exc.key.size());
      if (lut.total > 0) {
        hipLaunchKernelGGL(lstm_build_act_lut, dim3((lut.total + 255) / 256), dim3(256), 0, stream,
                           sp, lut, lut_table);
        RXMET_CHECK_LAUNCH();
        if (n_exc > 0) {
          hipLaunchKernelGGL(lstm_act_lut_exceptions, dim3((n_exc + 255) / 256), dim3(256), 0,
                             stream, sp, lut, lut_table);
          RXMET_CHECK_LAUNCH();
        }
      }
      if (lut.gtotal > 0) {  // the builder on the global tables' layout
        ActLut gl{};
        for (int g = 0; g < 4; ++g) {
          gl.off[g] = lut.goff[g];
          gl.n[g] = lut.gn[g];
        }
        gl.tanh_off = lut.gtanh_off;
        gl.tanh_n = lut.gtanh_n;
        gl.total = lut.gtotal;
        uint32_t *gt = reinterpret_cast<uint32_t *>(wsb + ws.glut);
        hipLaunchKernelGGL(lstm_build_act_lut, dim3((gl.total + 255) / 256), dim3(256), 0, stream,
                           sp, gl, gt);
        RXMET_CHECK_LAUNCH();
        if (n_exc > 0) {
          hipLaunchKernelGGL(lstm_act_lut_exceptions, dim3((n_exc + 255) / 256), dim3(256), 0,
                             stream, sp, gl, gt);
          RXMET_CHECK_LAUNCH();
        }
      }
      void *args[] = {&ra, &sp, &cl};
      {
        rxmet::prof::Scope ps__("lstm_fwd_recurrence", stream);
        RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * cl.G), dim3(512), args,
                                                   static_cast<unsigned>(lds_cl), stream));
      }
      const int64_t n_out = static_cast<int64_t>(T) * B * H, n_state = static_cast<int64_t>(B) * H;
      hipLaunchKernelGGL(lstm_poison_on_timeout, dim3(64), dim3(256), 0, stream, cl.timeout, n_out,
                         output, n_state, h_n, c_n);
      RXMET_CHECK_LAUNCH();
      return 0;
    }
  }
  if (pw == 2) return run_stepped();  // the per-tile recurrence holds one W_hh plane
  const size_t lds = recurrence_lds(H, KS, npl);
  const dim3 grid((B + kBT - 1) / kBT), block(64 * ((UT + kTilesPerWave - 1) / kTilesPerWave));
  {
    rxmet::prof::Scope ps__("lstm_fwd_recurrence", stream);
    if (npl == 1) {
      RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&lstm_recurrence<1>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          static_cast<int>(lds)));
      hipLaunchKernelGGL(lstm_recurrence<1>, grid, block, lds, stream, ra, sp);
    } else {
      RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&lstm_recurrence<2>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          static_cast<int>(lds)));
      hipLaunchKernelGGL(lstm_recurrence<2>, grid, block, lds, stream, ra, sp);
    }
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_lstm_forward_quant(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0,
                             const rxmet_lstm_params *params, float *output, float *h_n,
                             float *c_n, const rxmet_lstm_saved *saved, void *workspace,
                             void *stream_) {
  clear_error();
  return lstm_forward_impl(T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, params, output, h_n,
                           c_n, saved, nullptr, workspace, stream_);
}

int rxmet_lstm_forward_quant_codes(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                                   const float *W_hh, const float *b_ih, const float *b_hh,
                                   const float *x, const float *h0, const float *c0,
                                   const rxmet_lstm_params *params, float *output, float *h_n,
                                   float *c_n, const rxmet_lstm_saved *saved,
                                   const rxmet_lstm_saved_codes *codes, void *workspace,
                                   void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(saved == nullptr || codes != nullptr, "codes must be non-null with saved");
  return lstm_forward_impl(T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, params, output, h_n,
                           c_n, saved, saved ? codes : nullptr, workspace, stream_);
}

}  // extern "C"
