// gru_bwd.hip — MI355X QuantGRU backward (STE), behind rxmet_gru_backward_quant.
//
// Reference path: backward_quant_float_storage_wrapper (pytorch/lib/
// gru_interface_binding.cc:789-920) dequantises the saved codes in place, transposes
// x/W/R with torch copies, then BackwardPassQuant::Run (src/gru_backward_gpu_quant.cu:
// 379-493) loops over t = T-1..0 from the host, launching PointwiseOperationsQuant
// (:93-266, atomicAdd bias gradients) and an SGEMM dh += R dq per step, followed by three
// SGEMMs (dx, dR, dW) and four mask passes.
//
// Here:
//   1. prologue    : x, h_prev and W codes as bf16 operand planes for the weight-gradient
//                    GEMMs (h codes recovered exactly from the dequantised h);
//   2. recurrence  : both directions walk t = T-1..0 in one clustered launch
//                    (bwd_recurrence_cl: a batch tile's hidden units split over a cluster of
//                    workgroups, dq * scale_R exchanged through global memory each step and
//                    dh += R_deq dq summed on bf16 MFMA, dq split exactly into three bf16
//                    terms against the R codes resident in VGPRs);
//                    the per-tile fallback (bwd_recurrence) keeps one workgroup per 16
//                    sequences, each lane owning one hidden unit for four sequences, with
//                    dh += R_deq dq on int8 MFMA over 22-bit block-fixed-point dq (three int8
//                    planes against the resident int8 R_q, recombined in fp64; error <= 2^-22
//                    of the row maximum per term).  Both fuse the STE pointwise (all mask
//                    families), write dp/dq for the GEMMs and keep fp64 bias partials;
//                    For H > 256 the stepped path (bwd_step_point + a K-split dh GEMM per
//                    step) replaces both;
//   3. bias fold   : per-workgroup fp64 partials summed in a fixed order (deterministic);
//   4. dx, dW, dR  : bf16-MFMA GEMMs with the gradients split exactly into three bf16 terms
//                    (wgrad_gemm.h; dW and dR split over the long T*B reduction and summed in
//                    a fixed order), then one mask pass.

#include <algorithm>

#include "cluster.h"
#include "gru_internal.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_gru.h"
#include "wgrad_gemm.h"

namespace rxmet {
namespace gru {

constexpr int kBTile = 16;

// ---------------------------------------------------------------------------------
// 1. prologue
// ---------------------------------------------------------------------------------

// R_q [H][3H] -> B fragments of D[b][k] = sum_c A[b][c] R[k][c]:
// frag[((ut * KS2) + s) * 64 + lane] holds R_q[k][c] for k = 16*ut + lane % 16,
// c = 64*s + 16*(lane / 16) + 0..15 (zero beyond 3H).  rowsum[k] = sum_c R_q[k][c].
__global__ __launch_bounds__(64) void pack_rt_frags(int H, int KS2, const float *__restrict__ Rq,
                                                    v4i *__restrict__ frag,
                                                    float *__restrict__ rowsum) {
  const int lane = threadIdx.x;
  const int idx = blockIdx.x;
  const int s = idx % KS2, ut = idx / KS2;
  const int C = 3 * H;
  const int k = 16 * ut + lane % 16;
  int wd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int by[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 64 * s + 16 * (lane / 16) + 4 * q + e;
      by[e] = (c < C && k < H) ? static_cast<int>(Rq[static_cast<size_t>(k) * C + c]) : 0;
    }
    wd[q] = pack4_i8(by[0], by[1], by[2], by[3]);
  }
  frag[static_cast<size_t>(idx) * 64 + lane] = v4i{wd[0], wd[1], wd[2], wd[3]};
  if (s == 0 && lane < 16 && k < H) {
    int sum = 0;
    for (int c = 0; c < C; ++c) sum += static_cast<int>(Rq[static_cast<size_t>(k) * C + c]);
    rowsum[k] = static_cast<float>(sum);
  }
}

// ---------------------------------------------------------------------------------
// 2. backward recurrence
// ---------------------------------------------------------------------------------
struct BwdArgs {
  int T, B, H, KS2;
  const float *dh_new;       // [T+1, B, H]
  const float *h;            // [T+1, B, H] dequantised
  const float *v;            // [T, B, 4H] dequantised
  const uint8_t *ih_m, *hh_m, *gin_m, *gout_m, *h_m;  // may be null
  const uint8_t *bw_m, *br_m, *h0_m;                  // may be null
  const v4i *rfrag;          // packed R_q fragments
  const float *rowsum;       // [H]
  const float *eff_r;        // [3H] effective per-channel scales of R
  float *dp, *dq;            // [T, B, 3H]
  double *bias_partial;      // [numWG][2][3H]
  float *dh0;                // [B, H]
  float *xch;                // clustered path: [2][Bpad][KP] exchanged dq * scale_R
  const uint4 *rt;           // clustered path: packed R_q codes, see pack_rt_bf16
  // saved state as codes (instead of v and the five per-step masks; the per-tile kernel
  // does not read them): v_codes [T, B, 4H] and mask_bits [T, B, H] of the forward; field q
  // of v is (v_codes - vzl[q]) * veff[q], vzl = zero point - grid minimum
  const uint16_t *vc, *mb;
  // dh_new read in place from the layer's output gradient (rxmet_gru_grad_view), when gv_on
  const float *gv, *gv_hn;
  int64_t gv_t, gv_b, gv_k;
  int gv_col0, gv_rev, gv_on;
  float vzl[4], veff[4];
};

constexpr int kPlanes = 3;

__global__ __launch_bounds__(512) void bwd_recurrence(BwdArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 3 * H, B = a.B;
  const int CP = a.KS2 * 64;          // padded channel count
  const int ROW = CP + 16;            // plane row stride in bytes
  float *dqs = reinterpret_cast<float *>(smem);                  // [16][CP] dq * scale_R
  unsigned *rowmax = reinterpret_cast<unsigned *>(dqs + kBTile * CP);  // [16] |max| bits
  int *rowexp = reinterpret_cast<int *>(rowmax + kBTile);              // [16]
  int8_t *plane = reinterpret_cast<int8_t *>(rowexp + kBTile);          // [3][16][ROW]

  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int w = tid / 64, l = tid % 64;
  const int b0 = blockIdx.x * kBTile;

  for (int i = tid; i < kBTile * CP; i += nthreads) dqs[i] = 0.0f;
  for (int i = tid; i < kPlanes * kBTile * ROW / 4; i += nthreads) reinterpret_cast<int *>(plane)[i] = 0;
  if (tid < kBTile) rowmax[tid] = 0u;

  v4i rfr[2][12];
  float rsum[2], effr[2][3];
  uint8_t mbw[2][3], mbr[2][3];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ut = 2 * w + u;
    const int j = 16 * ut + l % 16;
#pragma unroll
    for (int s = 0; s < 12; ++s)
      rfr[u][s] = (s < a.KS2 && 16 * ut < H) ? a.rfrag[(static_cast<size_t>(ut) * a.KS2 + s) * 64 + l]
                                           : v4i{0, 0, 0, 0};
    rsum[u] = j < H ? a.rowsum[j] : 0.0f;
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      effr[u][g] = j < H ? a.eff_r[g * H + j] : 0.0f;
      mbw[u][g] = (j < H && a.bw_m) ? a.bw_m[g * H + j] : 1;
      mbr[u][g] = (j < H && a.br_m) ? a.br_m[g * H + j] : 1;
    }
  }
  float dh[2][4];
  double sbw[2][3], sbr[2][3];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int r = 0; r < 4; ++r) dh[u][r] = 0.0f;
#pragma unroll
    for (int g = 0; g < 3; ++g) sbw[u][g] = sbr[u][g] = 0.0;
  }
  __syncthreads();

  const int nrow0 = 4 * (l / 16);
  const uint32_t BH = static_cast<uint32_t>(B) * H;

  for (int t = a.T - 1; t >= 0; --t) {
    // ---- pointwise STE backward (reference order of operations) ----
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = 16 * (2 * w + u) + l % 16;
      if (16 * (2 * w + u) >= H) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nr = nrow0 + r, b = b0 + nr;
        float dpv[3] = {0.f, 0.f, 0.f}, dqv[3] = {0.f, 0.f, 0.f};
        if (b < B) {
          const uint32_t oH = static_cast<uint32_t>(b) * H + j;
          const uint32_t oC = 3u * static_cast<uint32_t>(b) * H + j;
          const uint32_t tH = static_cast<uint32_t>(t) * BH;
          const uint32_t tC = 3u * tH, v0 = 4u * tH + 4u * static_cast<uint32_t>(b) * H + j;
          float dht = a.dh_new[tH + BH + oH] + dh[u][r];
          if (a.h_m) dht *= static_cast<float>(a.h_m[tH + oH]);
          const float z = a.v[v0], rr = a.v[v0 + H], g = a.v[v0 + 2 * H], qg = a.v[v0 + 3 * H];
          dh[u][r] = z * dht;
          const float dg = (1.0f - z) * dht;
          const float dz = (a.h[tH + oH] - g) * dht;
          const uint32_t m = tC + oC;
          float dpg = (1.0f - g * g) * dg;
          if (a.gout_m) dpg *= static_cast<float>(a.gout_m[m + 2 * H]);
          if (a.gin_m) dpg *= static_cast<float>(a.gin_m[m + 2 * H]);
          float dqg = dpg * rr;
          const float dr = dpg * qg;
          float dpr = rr * (1.0f - rr) * dr, dqr = dpr;
          float dpz = z * (1.0f - z) * dz, dqz = dpz;
          if (a.gout_m) {
            const float mz = static_cast<float>(a.gout_m[m]), mr = static_cast<float>(a.gout_m[m + H]);
            dpz *= mz; dqz *= mz; dpr *= mr; dqr *= mr;
          }
          if (a.gin_m) {
            const float mz = static_cast<float>(a.gin_m[m]), mr = static_cast<float>(a.gin_m[m + H]);
            dpz *= mz; dqz *= mz; dpr *= mr; dqr *= mr;
          }
          if (a.hh_m) {
            dqz *= static_cast<float>(a.hh_m[m]);
            dqr *= static_cast<float>(a.hh_m[m + H]);
            dqg *= static_cast<float>(a.hh_m[m + 2 * H]);
          }
          if (a.ih_m) {
            dpz *= static_cast<float>(a.ih_m[m]);
            dpr *= static_cast<float>(a.ih_m[m + H]);
            dpg *= static_cast<float>(a.ih_m[m + 2 * H]);
          }
          dpv[0] = dpz; dpv[1] = dpr; dpv[2] = dpg;
          dqv[0] = dqz; dqv[1] = dqr; dqv[2] = dqg;
#pragma unroll
          for (int gg = 0; gg < 3; ++gg) {
            a.dp[m + gg * H] = dpv[gg];
            a.dq[m + gg * H] = dqv[gg];
            sbw[u][gg] += static_cast<double>(dpv[gg] * static_cast<float>(mbw[u][gg]));
            sbr[u][gg] += static_cast<double>(dqv[gg] * static_cast<float>(mbr[u][gg]));
          }
        }
        // dq scaled by the per-channel dequantisation scale of R, staged for the GEMM
        float mx = 0.0f;
#pragma unroll
        for (int gg = 0; gg < 3; ++gg) {
          const float sv = dqv[gg] * effr[u][gg];
          dqs[nr * CP + gg * H + j] = sv;
          const float as = fabsf(sv);
          mx = (as > mx || as != as) ? as : mx;  // keeps NaN
        }
        if (!(mx <= 3.0e38f)) mx = INFINITY;  // NaN/inf rows propagate below
        atomicMax(&rowmax[nr], __float_as_uint(mx));
      }
    }
    __syncthreads();
    // ---- block fixed point: 22-bit integers split into three int8 planes ----
    if (tid < kBTile) {
      const float m = __uint_as_float(rowmax[tid]);
      int ex = 0;
      if (m > 0.0f && m <= 3.0e38f) frexpf(m, &ex);
      rowexp[tid] = (m > 0.0f && m <= 3.0e38f) ? 22 - ex : (m == 0.0f ? 0 : 1000);
    }
    __syncthreads();
    for (int i = tid; i < kBTile * CP; i += nthreads) {
      const int nr = i / CP, c = i % CP;
      const int e = rowexp[nr];
      int q = 0;
      if (e != 1000) q = static_cast<int>(rintf(ldexpf(dqs[i], e)));
      const int uq = q + (1 << 23);
      plane[(0 * kBTile + nr) * ROW + c] = static_cast<int8_t>((uq & 255) - 128);
      plane[(1 * kBTile + nr) * ROW + c] = static_cast<int8_t>(((uq >> 8) & 255) - 128);
      plane[(2 * kBTile + nr) * ROW + c] = static_cast<int8_t>((uq >> 16) - 128);
    }
    __syncthreads();
    if (tid < kBTile) rowmax[tid] = 0u;
    // ---- dh += R_deq dq on MFMA ----
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (16 * (2 * w + u) >= H) continue;
      v4i acc[kPlanes];
#pragma unroll
      for (int q = 0; q < kPlanes; ++q) acc[q] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < 12; ++s) {
        if (s < a.KS2) {
#pragma unroll
          for (int q = 0; q < kPlanes; ++q) {
            const v4i afr = *reinterpret_cast<const v4i *>(plane + (q * kBTile + l % 16) * ROW +
                                                           64 * s + 16 * (l / 16));
            acc[q] = mfma_i8(afr, rfr[u][s], acc[q]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = rowexp[nrow0 + r];
        const double comb = 65536.0 * acc[2][r] + 256.0 * acc[1][r] + static_cast<double>(acc[0][r]) +
                            32896.0 * static_cast<double>(rsum[u]);
        const float add = e == 1000 ? NAN : static_cast<float>(ldexp(comb, -e));
        dh[u][r] = dh[u][r] + add;
      }
    }
    __syncthreads();
  }
  // dh0 and bias partials
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = 16 * (2 * w + u) + l % 16;
    if (16 * (2 * w + u) >= H) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int b = b0 + nrow0 + r;
      if (b < B) {
        const uint32_t o = static_cast<uint32_t>(b) * H + j;
        a.dh0[o] = a.h0_m ? dh[u][r] * static_cast<float>(a.h0_m[o]) : dh[u][r];
      }
    }
    // sum the four row groups (lanes l, l^16, l^32, l^48 share the unit)
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      double x = sbw[u][gg], y = sbr[u][gg];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      y += __shfl_xor(y, 16, 64);
      y += __shfl_xor(y, 32, 64);
      if (l < 16) {
        double *p = a.bias_partial + static_cast<size_t>(blockIdx.x) * 2 * C;
        p[gg * H + j] = x;
        p[C + gg * H + j] = y;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// 2b. clustered backward recurrence
// ---------------------------------------------------------------------------------
// Member m of a cluster owns UT unit tiles (16 units) of one 16-sequence batch tile.  Per step
// each lane finishes the STE pointwise of one (sequence, unit), writes dq * scale_R of its
// three channels to a global exchange buffer (coherent stores), and after the cluster barrier
// the four waves of a unit tile compute dh += R_deq dq for that tile on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16), each over a quarter of the 3H channels: the exchanged values
// split exactly into three bf16 terms against the R_q codes (resident in VGPRs as one bf16
// plane, or two for codes beyond +-256: the RNE bf16 of the code and the exact residual), fp32
// accumulation; the four partial sums are added through LDS in a fixed order.
constexpr int kBwMaxKS2 = 12;  // 3H <= 768
constexpr int kBwMaxKB = (kBwMaxKS2 + 1) / 2;  // 32-channel MFMA blocks per wave
constexpr int kMaxHStepped = 1024;
constexpr int kStepMaxSplit = 8;  // K splits of the stepped dh GEMM

struct BwdClArgs {
  int ncl, G, UT, ntiles, Bpad, KP, ndir;  // KP = 3H padded to a multiple of 64
  unsigned *counters;
  int *timeout;
  unsigned spin_limit;  // polls before a wait gives up (cluster::spin_limit())
};

// R_q [H][3H] -> per (unit tile ut, wave q, 32-channel block kb, lane l) the bf16 B fragment
// R_q[j][k + e], e = 0..7, with j = 16 ut + l % 16 and k = 16 q KS2 + 32 kb + 8 (l / 16): wave q
// contracts channels [16 q KS2, 16 (q + 1) KS2), zero beyond them and beyond 3H.  Plane 0 holds
// the RNE bf16 of each code; with two planes plane 1 (at rt + nfrag * 64, nfrag = gridDim.x)
// holds the residual code - plane 0, exact in bf16 for |code| < 2^16.
__global__ __launch_bounds__(64) void pack_rt_bf16(int H, int KS2, int nplanes, const float *__restrict__ Rq,
                                                   uint4 *__restrict__ rt) {
  const int l = threadIdx.x, idx = blockIdx.x;  // idx = (ut * 4 + q) * nkb + kb
  const int nkb = (KS2 + 1) / 2;
  const int kb = idx % nkb, q = (idx / nkb) % 4, ut = idx / (4 * nkb);
  const int j = 16 * ut + l % 16;
  const int k0 = 16 * q * KS2 + 32 * kb + 8 * (l / 16), kend = min(16 * (q + 1) * KS2, 3 * H);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = k0 + e < kend ? Rq[static_cast<size_t>(j) * 3 * H + k0 + e] : 0.0f;
  unsigned w[4], r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const v2f x = v2f{v[2 * e], v[2 * e + 1]};
    w[e] = pack_bf16x2(x);
    r[e] = pack_bf16x2(x - unpack_bf16x2(w[e]));
  }
  rt[static_cast<size_t>(idx) * 64 + l] = make_uint4(w[0], w[1], w[2], w[3]);
  if (nplanes == 2)
    rt[(static_cast<size_t>(gridDim.x) + idx) * 64 + l] = make_uint4(r[0], r[1], r[2], r[3]);
}

// A mask that may be absent.  The load is unconditional (an absent mask reads the same index
// of `fallback`, a buffer at least as large as any mask: the saved activations v, [T, B, 4H]
// floats) and the value is replaced by 1 afterwards, so the step's loads need no branch;
// multiplying by 1.0f leaves every value, NaN and -0 included, as it was.
struct MaskRef {
  const uint8_t *p;
  bool on;
  __device__ __forceinline__ float at(uint32_t i) const {
    const float v = static_cast<float>(p[i]);
    return on ? v : 1.0f;
  }
};
__device__ __forceinline__ MaskRef mask_ref(const uint8_t *p, const void *fallback) {
  return p ? MaskRef{p, true} : MaskRef{static_cast<const uint8_t *>(fallback), false};
}

// The step inputs of one lane (sequence b, unit j) at time t: dh_new, h, the four saved gate
// values and the 13 mask values (absent masks read 1).
constexpr int kBwRaw = 19;
struct BwdMasks {
  MaskRef h, go, gi, hh, ih;
};
__device__ __forceinline__ void bwd_load_step(const BwdArgs &a, const BwdMasks &mk, int t, int b,
                                              int j, float (&r)[kBwRaw]) {
  const int H = a.H;
  const uint32_t BH = static_cast<uint32_t>(a.B) * H;
  const uint32_t oH = static_cast<uint32_t>(b) * H + j;
  const uint32_t tH = static_cast<uint32_t>(t) * BH;
  const uint32_t m = 3u * tH + 3u * static_cast<uint32_t>(b) * H + j;
  const uint32_t v0 = 4u * tH + 4u * static_cast<uint32_t>(b) * H + j;
  if (a.gv_on) {
    float g = 0.0f;
    if (a.gv) {
      const int64_t tt = a.gv_rev ? a.T - 1 - t : t;
      g = a.gv[tt * a.gv_t + b * a.gv_b + (a.gv_col0 + j) * a.gv_k];
    }
    if (t == a.T - 1 && a.gv_hn) g += a.gv_hn[oH];
    r[0] = g;
  } else {
    r[0] = a.dh_new[tH + BH + oH];
  }
  r[1] = a.h[tH + oH];
  if (a.vc) {
    // blocked codes: block ((t ceil(B/16) + b / 16) H/16 + j / 16) of 16 rows x 16 units, v as
    // [16][4][16], mask bits as [16][16]; the forward's (code - zero point) * effective scale,
    // from code - minimum: the same fp32 operations on the same values
    const uint32_t nt = static_cast<uint32_t>(a.B + 15) / 16;
    const uint32_t row = ((static_cast<uint32_t>(t) * nt + static_cast<uint32_t>(b) / 16) *
                              (static_cast<uint32_t>(H) / 16) + static_cast<uint32_t>(j) / 16) * 16 +
                         static_cast<uint32_t>(b) % 16;
    const uint32_t e = static_cast<uint32_t>(j) % 16;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      r[2 + q] = (static_cast<float>(a.vc[64 * row + 16 * q + e]) - a.vzl[q]) * a.veff[q];
    const unsigned bits = a.mb[16 * row + e];
    auto bit = [&](int k) { return static_cast<float>((bits >> k) & 1u); };
    r[6] = bit(12);
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      r[7 + gg] = bit(9 + gg);
      r[10 + gg] = bit(6 + gg);
      r[13 + gg] = bit(3 + gg);
      r[16 + gg] = bit(gg);
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) r[2 + q] = a.v[v0 + q * H];
  r[6] = mk.h.at(tH + oH);
#pragma unroll
  for (int gg = 0; gg < 3; ++gg) {
    r[7 + gg] = mk.go.at(m + gg * H);
    r[10 + gg] = mk.gi.at(m + gg * H);
    r[13 + gg] = mk.hh.at(m + gg * H);
    r[16 + gg] = mk.ih.at(m + gg * H);
  }
}

// STE pointwise of one (sequence, unit) at one step: from the step inputs and the carried
// gradient dhc, the pre-activation gradients dp (input branch) and dq (recurrent branch) of
// the three gates; returns the part of dh_{t-1} that does not pass through R (z dh_t).
__device__ __forceinline__ float bwd_point(const float (&cur)[kBwRaw], float dhc, float (&dpv)[3],
                                           float (&dqv)[3]) {
  const float z = cur[2], rr = cur[3], g = cur[4], qg = cur[5];
  const float dht = (cur[0] + dhc) * cur[6];
  const float dg = (1.0f - z) * dht;
  const float dz = (cur[1] - g) * dht;
  float dpg = (1.0f - g * g) * dg;
  dpg *= cur[7 + 2];
  dpg *= cur[10 + 2];
  float dqg = dpg * rr;
  const float dr = dpg * qg;
  float dpr = rr * (1.0f - rr) * dr, dqr = dpr;
  float dpz = z * (1.0f - z) * dz, dqz = dpz;
  dpz *= cur[7]; dqz *= cur[7]; dpr *= cur[8]; dqr *= cur[8];
  dpz *= cur[10]; dqz *= cur[10]; dpr *= cur[11]; dqr *= cur[11];
  dqz *= cur[13]; dqr *= cur[14]; dqg *= cur[15];
  dpz *= cur[16]; dpr *= cur[17]; dpg *= cur[18];
  dpv[0] = dpz; dpv[1] = dpr; dpv[2] = dpg;
  dqv[0] = dqz; dqv[1] = dqr; dqv[2] = dqg;
  return z * dht;
}

// LDS of the clustered backward: partial sums, bias partials, the staged exchange rows.
constexpr size_t kBwRedBytes = 16 * 1024, kBwBredBytes = sizeof(double) * 2 * 4 * 16 * 6;
__host__ __device__ constexpr size_t bwd_cl_lds(int KP) {
  return kBwRedBytes + kBwBredBytes + sizeof(float) * kBTile * static_cast<size_t>(KP + 4);
}

// One (direction, batch tile) pair, run by one member of UT unit tiles; writes the pair's
// bias partials.
template <int UT, int NPL>
__device__ __forceinline__ void bwd_cl_pair(const BwdArgs &a, const BwdClArgs &cl, int tile,
                                            int member, unsigned *counter, unsigned &epoch,
                                            bool &alive) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int H = a.H, C = 3 * H, B = a.B, KS2 = a.KS2, KP = cl.KP;
  v4f *red = reinterpret_cast<v4f *>(smem);                          // [UT][4][64]
  double *bred = reinterpret_cast<double *>(smem + kBwRedBytes);     // [UT][4][16][6]
  float *xs = reinterpret_cast<float *>(smem + kBwRedBytes + kBwBredBytes);  // [16][KP + 4]
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int utl = w / 4, kq = w % 4;
  const int ut = member * UT + utl;
  // staging of the exchange rows: thread -> row tid / (16 UT), 16-byte chunks
  // tid % (16 UT) + 16 UT q for q < ceil(KS2 / UT)
  constexpr int kQ = (kBwMaxKS2 + UT - 1) / UT;
  const int srow = tid / (16 * UT), sc0 = tid % (16 * UT), sqn = (KS2 + UT - 1) / UT;
  const int j = 16 * ut + l % 16;
  const int nr = 4 * (l / 16) + kq;
  const int nkb = (KS2 + 1) / 2;
  const size_t nfrag = static_cast<size_t>(H / 16) * 4 * nkb;
  v8bf rtb[NPL][kBwMaxKB];
#pragma unroll
  for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
    for (int i = 0; i < kBwMaxKB; ++i)
      rtb[pl][i] = __builtin_bit_cast(
          v8bf, i < nkb ? a.rt[(pl * nfrag + (static_cast<size_t>(ut) * 4 + kq) * nkb + i) * 64 + l]
                        : make_uint4(0, 0, 0, 0));
  float effr[3];
  float mbw[3], mbr[3];
#pragma unroll
  for (int g = 0; g < 3; ++g) {
    effr[g] = a.eff_r[g * H + j];
    mbw[g] = a.bw_m ? static_cast<float>(a.bw_m[g * H + j]) : 1.0f;
    mbr[g] = a.br_m ? static_cast<float>(a.br_m[g * H + j]) : 1.0f;
  }
  double sbw[3] = {0.0, 0.0, 0.0}, sbr[3] = {0.0, 0.0, 0.0};
  const uint32_t BH = static_cast<uint32_t>(B) * H;
  v4f *myred = red + (static_cast<size_t>(utl) * 4 + kq) * 64;
  // the exchange buffer, [2][Bpad][KP] floats (32-bit byte offsets: checked by the launcher)
  const auto xr = cluster::buffer_rsrc(a.xch, 8u * cl.Bpad * KP);
  const BwdMasks mk = {mask_ref(a.h_m, a.v), mask_ref(a.gout_m, a.v), mask_ref(a.gin_m, a.v),
                       mask_ref(a.hh_m, a.v), mask_ref(a.ih_m, a.v)};

  {
    const int b0 = tile * kBTile, b = b0 + nr;
    const bool valid = b < B;
    float dhc = 0.0f;
    // step inputs are loaded one step ahead: the next step's loads are in flight during the
    // cluster wait
    float cur[kBwRaw];
    if (valid) bwd_load_step(a, mk, a.T - 1, b, j, cur);
    for (int t = a.T - 1; t >= 0 && alive; --t) {
      const int par = t & 1;
      float dqv[3] = {0.f, 0.f, 0.f}, dpv[3] = {0.f, 0.f, 0.f};
      uint32_t m = 0;
      float dhl = 0.0f;
      if (valid) {
        m = 3u * static_cast<uint32_t>(t) * BH + 3u * static_cast<uint32_t>(b) * H + j;
        dhl = bwd_point(cur, dhc, dpv, dqv);
#pragma unroll
        for (int gg = 0; gg < 3; ++gg) {
          sbw[gg] += static_cast<double>(dpv[gg] * mbw[gg]);
          sbr[gg] += static_cast<double>(dqv[gg] * mbr[gg]);
        }
      }
      float *xrow = a.xch + (static_cast<size_t>(par) * cl.Bpad + b) * KP;
#pragma unroll
      for (int gg = 0; gg < 3; ++gg)
        cluster::store_coherent(reinterpret_cast<unsigned *>(xrow + gg * H + j),
                                __float_as_uint(dqv[gg] * effr[gg]));
      // the other members only read the exchange: arrive, then store dp / dq while waiting
      cluster::arrive(counter);
      ++epoch;
      if (valid) {
#pragma unroll
        for (int gg = 0; gg < 3; ++gg) {
          a.dp[m + gg * H] = dpv[gg];
          a.dq[m + gg * H] = dqv[gg];
        }
      }
      if (valid && t > 0) bwd_load_step(a, mk, t - 1, b, j, cur);
      alive = cluster::wait(counter, epoch * cl.G, cl.timeout, cl.spin_limit);
      if (!alive) break;
      // stage the tile's exchange rows in LDS (all loads in flight; a q past the row re-reads
      // q = 0 and is not stored), then dh += R_deq dq over this wave's quarter of the channels
      {
        const unsigned src = 4u * ((static_cast<unsigned>(par) * cl.Bpad + b0 + srow) * KP + 4 * sc0);
        float *dst = xs + srow * (KP + 4) + 4 * sc0;
        int4 sv[kQ];
#pragma unroll
        for (int q = 0; q < kQ; ++q) {
          const int qq = (q < sqn && 16 * UT * q + sc0 < 16 * KS2) ? q : 0;
          sv[q] = cluster::load_coherent16(xr, src + 256u * UT * qq);
        }
#pragma unroll
        for (int q = 0; q < kQ; ++q)
          if (q < sqn && 16 * UT * q + sc0 < 16 * KS2)
            *reinterpret_cast<int4 *>(dst + 64 * UT * q) = sv[q];
      }
      __syncthreads();
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      {
        // A: row l % 16, channels 16 kq KS2 + 32 kb + 8 (l / 16) + 0..7 (zero past the wave's
        // channels, which another wave contracts), split into three bf16 terms, smallest first
        const float *arow = xs + (l % 16) * (KP + 4) + 16 * (kq * KS2) + 8 * (l / 16);
#pragma unroll
        for (int kb = 0; kb < kBwMaxKB; ++kb)
          if (kb < nkb) {
            const bool in = 32 * kb + 8 * (l / 16) < 16 * KS2;
            const float *ap = arow + (in ? 32 * kb : 0);  // (a lane past the row reads its start)
            const v4f a0 = *reinterpret_cast<const v4f *>(ap);
            const v4f a1 = *reinterpret_cast<const v4f *>(ap + 4);
            const float v[8] = {in ? a0[0] : 0.f, in ? a0[1] : 0.f, in ? a0[2] : 0.f, in ? a0[3] : 0.f,
                                in ? a1[0] : 0.f, in ? a1[1] : 0.f, in ? a1[2] : 0.f, in ? a1[3] : 0.f};
            uint4 h, m, o;
            split3x8(v, h, m, o);
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl) {
              acc = mfma_bf16(__builtin_bit_cast(v8bf, o), rtb[pl][kb], acc);
              acc = mfma_bf16(__builtin_bit_cast(v8bf, m), rtb[pl][kb], acc);
              acc = mfma_bf16(__builtin_bit_cast(v8bf, h), rtb[pl][kb], acc);
            }
          }
      }
      myred[l] = acc;
      __syncthreads();
      float gsum = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        gsum += reinterpret_cast<const float *>(red + (static_cast<size_t>(utl) * 4 + k) * 64 + l)[kq];
      dhc = dhl + gsum;
    }
    if (valid && alive) {
      const uint32_t o = static_cast<uint32_t>(b) * H + j;
      a.dh0[o] = a.h0_m ? dhc * static_cast<float>(a.h0_m[o]) : dhc;
    }
  }
  // bias partials of this member's units: rows summed in a fixed order
#pragma unroll
  for (int gg = 0; gg < 3; ++gg) {
    sbw[gg] += __shfl_xor(sbw[gg], 16, 64);
    sbw[gg] += __shfl_xor(sbw[gg], 32, 64);
    sbr[gg] += __shfl_xor(sbr[gg], 16, 64);
    sbr[gg] += __shfl_xor(sbr[gg], 32, 64);
  }
  __syncthreads();
  if (l < 16) {
    double *d = bred + ((static_cast<size_t>(utl) * 4 + kq) * 16 + l) * 6;
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      d[gg] = sbw[gg];
      d[3 + gg] = sbr[gg];
    }
  }
  __syncthreads();
  if (kq == 0 && l < 16) {
    double x[6] = {0, 0, 0, 0, 0, 0};
    for (int k = 0; k < 4; ++k) {
      const double *d = bred + ((static_cast<size_t>(utl) * 4 + k) * 16 + l) * 6;
#pragma unroll
      for (int e = 0; e < 6; ++e) x[e] += d[e];
    }
    double *p = a.bias_partial + static_cast<size_t>(tile) * 2 * C;
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      p[gg * H + j] = x[gg];
      p[C + gg * H + j] = x[3 + gg];
    }
  }
}

template <int UT, int NPL>
__global__ __launch_bounds__(256 * UT) void bwd_recurrence_cl(BwdArgs a0, BwdArgs a1, BwdClArgs cl) {
  const cluster::Place pl = cluster::place(cl.G, cl.ncl);
  unsigned *counter = cl.counters + cluster::kCounterStride * pl.cluster;
  unsigned epoch = 0;
  bool alive = true;
  for (int pair = pl.cluster; pair < cl.ndir * cl.ntiles && alive; pair += cl.ncl) {
    const int d = pair / cl.ntiles, tile = pair % cl.ntiles;
    __syncthreads();
    // one copy of the step code for both directions (d is uniform across the workgroup)
    bwd_cl_pair<UT, NPL>(d == 0 ? a0 : a1, cl, tile, pl.member, counter, epoch, alive);
  }
}

// ---------------------------------------------------------------------------------
// stepped backward (H > 256): per step one pointwise launch and one dh GEMM launch
// ---------------------------------------------------------------------------------
// Step t: every (sequence, unit) takes dh_c = dhl + gsum of step t + 1 (zero at t = T - 1),
// stores dp, dq and dhl = z dh_t, and adds its bias terms to the partial sums of its 16-row
// chunk (bias_partial[chunk][2][3H], each slot owned by one thread, steps in order); the dh
// GEMM gsum = (dq_t scale_R) R_q^T then runs on the split-bf16 MFMA product (wgrad::nt).
__global__ __launch_bounds__(256) void bwd_step_point(BwdArgs a, int t, int S,
                                                      const float *__restrict__ gsum,
                                                      float *__restrict__ dhl) {
  // block: 64 units x 4 row groups; a 16-row chunk per block (row group y takes rows y + 4 i)
  __shared__ double red[3][6][64];
  const int H = a.H, C = 3 * H, B = a.B;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  const int j = blockIdx.x * 64 + tx, chunk = blockIdx.y;
  const bool on = j < H;
  const int jj = on ? j : 0;
  const BwdMasks mk = {mask_ref(a.h_m, a.v), mask_ref(a.gout_m, a.v), mask_ref(a.gin_m, a.v),
                       mask_ref(a.hh_m, a.v), mask_ref(a.ih_m, a.v)};
  double sb[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  const uint32_t BH = static_cast<uint32_t>(B) * H;
  const size_t split = static_cast<size_t>(B) * H;
#pragma unroll
  for (int i = 0; i < kBTile / 4; ++i) {
    const int b = chunk * kBTile + ty + 4 * i;
    if (!on || b >= B) continue;
    const uint32_t o = static_cast<uint32_t>(b) * H + jj;
    float dhc = 0.0f;
    if (t != a.T - 1) {
      float gs = gsum[o];
      for (int z = 1; z < S; ++z) gs += gsum[z * split + o];
      dhc = dhl[o] + gs;
    }
    float cur[kBwRaw];
    bwd_load_step(a, mk, t, b, jj, cur);
    float dpv[3], dqv[3];
    dhl[o] = bwd_point(cur, dhc, dpv, dqv);
    const uint32_t m = 3u * static_cast<uint32_t>(t) * BH + 3u * static_cast<uint32_t>(b) * H + jj;
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      a.dp[m + g * H] = dpv[g];
      a.dq[m + g * H] = dqv[g];
      sb[g] += static_cast<double>(dpv[g]);
      sb[3 + g] += static_cast<double>(dqv[g]);
    }
  }
  if (ty > 0)
#pragma unroll
    for (int e = 0; e < 6; ++e) red[ty - 1][e][tx] = sb[e];
  __syncthreads();
  if (ty == 0 && on) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int e = 0; e < 6; ++e) sb[e] += red[k][e][tx];
    double *p = a.bias_partial + static_cast<size_t>(chunk) * 2 * C;
    const bool first = t == a.T - 1;
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const double mw = a.bw_m ? static_cast<double>(a.bw_m[g * H + j]) : 1.0;
      const double mr = a.br_m ? static_cast<double>(a.br_m[g * H + j]) : 1.0;
      p[g * H + j] = (first ? 0.0 : p[g * H + j]) + sb[g] * mw;
      p[C + g * H + j] = (first ? 0.0 : p[C + g * H + j]) + sb[3 + g] * mr;
    }
  }
}

// dh0 = (dhl + gsum of step 0) * h0 mask (gsum: S K-split parts summed in order).
__global__ __launch_bounds__(256) void bwd_step_dh0(int64_t n, int S, const float *__restrict__ dhl,
                                                    const float *__restrict__ gsum,
                                                    const uint8_t *__restrict__ h0_m,
                                                    float *__restrict__ dh0) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float gs = gsum[i];
  for (int z = 1; z < S; ++z) gs += gsum[z * n + i];
  const float v = dhl[i] + gs;
  dh0[i] = h0_m ? v * static_cast<float>(h0_m[i]) : v;
}

__global__ __launch_bounds__(256) void zero_floats(int64_t n, float *p) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = 0.0f;
}


// swap_h > 0: written in the (r, z, n) gate order (the first two blocks of swap_h swapped).
__global__ __launch_bounds__(256) void fold_bias(int nwg, int C, const double *__restrict__ part,
                                                 float *__restrict__ dbw, float *__restrict__ dbr,
                                                 int swap_h) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int co = swap_h > 0 ? (c < swap_h ? c + swap_h : (c < 2 * swap_h ? c - swap_h : c)) : c;
  double x = 0.0, y = 0.0;
  for (int k = 0; k < nwg; ++k) {
    x += part[static_cast<size_t>(k) * 2 * C + c];
    y += part[static_cast<size_t>(k) * 2 * C + C + c];
  }
  dbw[co] = static_cast<float>(x);
  dbr[co] = static_cast<float>(y);
}

__global__ __launch_bounds__(256) void apply_masks(int64_t n0, int64_t n1, int64_t n2, float *d0,
                                                   const uint8_t *m0, float *d1, const uint8_t *m1,
                                                   float *d2, const uint8_t *m2) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n0 + n1 + n2;
       i += stride) {
    if (i < n0) {
      if (m0) d0[i] *= static_cast<float>(m0[i]);
    } else if (i < n0 + n1) {
      if (m1) d1[i - n0] *= static_cast<float>(m1[i - n0]);
    } else {
      if (m2) d2[i - n0 - n1] *= static_cast<float>(m2[i - n0 - n1]);
    }
  }
}

size_t bwd_lds_bytes(int KS2) {
  const int CP = KS2 * 64, ROW = CP + 16;
  return sizeof(float) * kBTile * CP + sizeof(unsigned) * kBTile + sizeof(int) * kBTile +
         static_cast<size_t>(kPlanes) * kBTile * ROW;
}

struct BwdWorkspace {
  size_t dp, dq, xt, ht, wb, qsc, rfrag, rowsum, effr, effw, bias, part, xch, rt, sync, rb, gsum,
      dhl, total;
  int Mp, S_w[2], kper_w[2], S_r[2], kper_r[2];  // K splits by number of B planes
  int Cp;                                         // 3H rounded up to a multiple of 32
  BwdWorkspace(int T, int B, int I, int H) {
    const size_t C = 3 * static_cast<size_t>(H);
    const size_t KS2 = (C + 63) / 64;
    const size_t nwg = (static_cast<size_t>(B) + kBTile - 1) / kBTile;
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t o = 0;
    dp = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * C);
    dq = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * C);
    // weight-gradient GEMM operands: x and h codes (transposed, rows padded to Mp) and W codes
    // as bf16 planes; the per-column scales of dW and dR
    const size_t M = static_cast<size_t>(T) * B;
    Mp = static_cast<int>((M + 31) / 32 * 32);
    xt = o; o += al(sizeof(__bf16) * 2 * I * static_cast<size_t>(Mp));
    ht = o; o += al(sizeof(__bf16) * 2 * H * static_cast<size_t>(Mp));
    wb = o; o += al(sizeof(__bf16) * 2 * I * ((C + 31) / 32 * 32));  // rows of Cp, zero past C
    // one host upload: eff_w [C] | eff_r [C] | GEMM column scales [I + H]
    effw = o;
    effr = effw + sizeof(float) * C;
    qsc = effr + sizeof(float) * C;
    o += al(sizeof(float) * (2 * C + I + H));
    rfrag = o; o += al(sizeof(v4i) * 64 * ((H + 15) / 16) * KS2);
    rowsum = o; o += al(sizeof(float) * H);
    bias = o; o += al(sizeof(double) * 2 * C * nwg);
    for (int np = 0; np < 2; ++np)
      wgrad::tn_plan(static_cast<int>(M), static_cast<int>(C), I, np + 1, &S_w[np], &kper_w[np]);
    for (int np = 0; np < 2; ++np)
      wgrad::tn_plan(static_cast<int>(M), static_cast<int>(C), H, np + 1, &S_r[np], &kper_r[np]);
    part = o;
    o += al(sizeof(float) * C *
            std::max(static_cast<size_t>(std::max(S_w[0], S_w[1])) * I,
                     static_cast<size_t>(std::max(S_r[0], S_r[1])) * H));
    // clustered recurrence: dq exchange, packed R_q values, counters
    const size_t Bpad = nwg * kBTile;
    xch = o; o += al(sizeof(float) * 2 * Bpad * KS2 * 64);
    rt = o; o += al(sizeof(uint4) * 2 * ((H + 15) / 16) * 4 * ((KS2 + 1) / 2) * 64);
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (2 * nwg + 2));  // clusters of both directions
    // stepped recurrence: R codes as bf16 planes [H][Cp], the dh GEMM output, dhl
    Cp = static_cast<int>((C + 31) / 32 * 32);
    rb = o; o += al(sizeof(__bf16) * 2 * H * static_cast<size_t>(Cp));
    gsum = o; o += al(sizeof(float) * kStepMaxSplit * static_cast<size_t>(B) * H);
    dhl = o; o += al(sizeof(float) * static_cast<size_t>(B) * H);
    total = o;
  }
};

// One direction's backward state between the phases.
struct BwdPlan {
  BwdArgs ba;
  const rxmet_gru_bwd_dir *d;
  char *wsb;
  int npx, nph, npw;  // bf16 planes of the x, h and W codes
  bool torch_layout;  // dW, dR, dbw, dbr in PyTorch's layout and (r, z, n) gate order
};

static int backward_prologue(int T, int B, int I, int H, const rxmet_gru_bwd_dir &d,
                             const rxmet_gru_saved_codes *codes, hipStream_t stream,
                             BwdPlan *plan, const rxmet_gru_grad_view *view = nullptr) {
  const rxmet_gru_qparams *params = d.params;
  RXMET_CHECK_ARG(params != nullptr, "params must be non-null");
  RXMET_CHECK_ARG(params->hidden == H, "params.hidden != hidden_size");
  RXMET_CHECK_ARG(d.W_q && d.R_q && d.x_q && (view || d.dh_new) && d.h && (codes || d.v) && d.dx && d.dW &&
                      d.dR && d.dbw && d.dbr && d.dh0 && d.workspace,
                  "required pointer is null");
  RXMET_CHECK_ARG(!codes || (codes->v_codes && codes->mask_bits),
                  "v_codes and mask_bits must be non-null");
  {
    const Bounds brq = bounds_of(params->chan_bits[RXMET_GRU_R], params->chan_unsigned[RXMET_GRU_R]);
    RXMET_CHECK_ARG(brq.lo >= -32768.0f && brq.hi <= 32767.0f,
                    "recurrent weights must fit signed 16 bits");
  }
  const int C = 3 * H;
  const int KS2 = (C + 63) / 64;
  const BwdWorkspace ws(T, B, I, H);
  char *wsb = static_cast<char *>(d.workspace);
  float *effr = reinterpret_cast<float *>(wsb + ws.effr);
  std::vector<float> host(8 * static_cast<size_t>(C));
  try {
    make_channel_factors(*params, H, host.data() + 4 * C, host.data() + 5 * C, host.data() + 6 * C,
                         host.data() + 7 * C, host.data(), host.data() + C, host.data() + 2 * C,
                         host.data() + 3 * C);
  } catch (const std::exception &e) {
    set_error(e.what());
    return -22;
  }

  // weight-gradient operands: x codes, h codes (recovered from the dequantised h) and W codes
  const float eff_x = effective_scale(params->g[RXMET_GRU_X].scale, params->use_pot2 != 0);
  const float zp_x = static_cast<float>(params->g[RXMET_GRU_X].zero_point);
  const float eff_h = effective_scale(params->g[RXMET_GRU_H].scale, params->use_pot2 != 0);
  const float zp_h = static_cast<float>(params->g[RXMET_GRU_H].zero_point);
  const Bounds bx = bounds_of(params->g[RXMET_GRU_X].bits, params->g[RXMET_GRU_X].is_unsigned);
  const Bounds bh = bounds_of(params->g[RXMET_GRU_H].bits, params->g[RXMET_GRU_H].is_unsigned);
  const Bounds bw = bounds_of(params->chan_bits[RXMET_GRU_W], params->chan_unsigned[RXMET_GRU_W]);
  plan->npx = wgrad::planes_for(bx.lo, bx.hi, zp_x);
  plan->nph = wgrad::planes_for(bh.lo, bh.hi, zp_h);
  plan->npw = wgrad::planes_for(bw.lo, bw.hi, 0.0);
  const int64_t M = static_cast<int64_t>(T) * B, Mp = ws.Mp;
  {
    rxmet::prof::Scope ps__("gru_bwd_codes", stream);
    if (int rc = wgrad::codes_t(d.x_q, M, nullptr, M, I, I, 1, zp_x, 1.0f, plan->npx,
                                reinterpret_cast<__bf16 *>(wsb + ws.xt), Mp,
                                static_cast<int64_t>(I) * Mp, stream))
      return rc;
    // h rows 0..T-1 are h_prev; each is (q - zp_h) eff_h
    if (int rc = wgrad::codes_t(d.h, M, nullptr, M, H, H, 1, 0.0f, eff_h, plan->nph,
                                reinterpret_cast<__bf16 *>(wsb + ws.ht), Mp,
                                static_cast<int64_t>(H) * Mp, stream))
      return rc;
    // W_q [I][C] kept as is: rows are the channels c (K), columns the inputs i
    if (int rc = wgrad::codes_t(d.W_q, C, nullptr, C, I, 1, C, 0.0f, 1.0f, plan->npw,
                                reinterpret_cast<__bf16 *>(wsb + ws.wb), ws.Cp,
                                static_cast<int64_t>(I) * ws.Cp, stream))
      return rc;
  }
  {
    // host holds eff_w, eff_r in its first 2C floats; the column scales follow
    host.resize(2 * static_cast<size_t>(C) + I + H);
    for (int k = 0; k < I; ++k) host[2 * static_cast<size_t>(C) + k] = eff_x;
    for (int k = 0; k < H; ++k) host[2 * static_cast<size_t>(C) + I + k] = eff_h;
    RXMET_CHECK_HIP(hipMemcpyAsync(wsb + ws.effw, host.data(), sizeof(float) * host.size(),
                                   hipMemcpyHostToDevice, stream));
  }
  BwdArgs &ba = plan->ba;
  ba.T = T; ba.B = B; ba.H = H; ba.KS2 = KS2;
  ba.dh_new = d.dh_new; ba.h = d.h; ba.v = d.v;
  ba.gv_on = view != nullptr;
  if (view) {
    RXMET_CHECK_ARG(view->col0 >= 0, "grad view: col0 must be non-negative");
    ba.gv = view->g; ba.gv_hn = view->g_hn;
    ba.gv_t = view->st; ba.gv_b = view->sb; ba.gv_k = view->sk;
    ba.gv_col0 = view->col0; ba.gv_rev = view->reverse != 0;
  }
  ba.ih_m = d.ih_mask; ba.hh_m = d.hh_mask; ba.gin_m = d.gate_in_mask; ba.gout_m = d.gate_out_mask;
  ba.h_m = d.h_mask; ba.bw_m = d.bw_mask; ba.br_m = d.br_mask; ba.h0_m = d.h0_mask;
  ba.vc = nullptr; ba.mb = nullptr;
  if (codes) {
    ba.v = nullptr;
    ba.ih_m = ba.hh_m = ba.gin_m = ba.gout_m = ba.h_m = nullptr;
    ba.vc = codes->v_codes;
    ba.mb = codes->mask_bits;
    const int fields[4] = {RXMET_GRU_Z_OUT, RXMET_GRU_R_OUT, RXMET_GRU_N_OUT, RXMET_GRU_RH};
    for (int q = 0; q < 4; ++q) {
      const rxmet_grid &g = params->g[fields[q]];
      const Bounds b = bounds_of(g.bits, g.is_unsigned);
      RXMET_CHECK_ARG(b.hi - b.lo <= 65535.0f,
                      "saved codes need gate output and weight_hh_linear grids of at most 16 bits");
      ba.vzl[q] = static_cast<float>(g.zero_point) - b.lo;
      ba.veff[q] = effective_scale(g.scale, params->use_pot2 != 0);
    }
  }
  ba.rfrag = reinterpret_cast<v4i *>(wsb + ws.rfrag);
  ba.rowsum = reinterpret_cast<float *>(wsb + ws.rowsum);
  ba.eff_r = effr;
  ba.dp = reinterpret_cast<float *>(wsb + ws.dp);
  ba.dq = reinterpret_cast<float *>(wsb + ws.dq);
  ba.bias_partial = reinterpret_cast<double *>(wsb + ws.bias);
  ba.dh0 = d.dh0;
  ba.xch = reinterpret_cast<float *>(wsb + ws.xch);
  ba.rt = reinterpret_cast<uint4 *>(wsb + ws.rt);
  plan->d = &d;
  plan->wsb = wsb;
  return 0;
}

// Clustered recurrence over every direction; 1 when launched, 0 when the caller must use the
// per-tile recurrence.
static int backward_recurrence_clustered(BwdPlan *plans, int ndir, int T, int B, int I, int H,
                                         hipStream_t stream, int **timeout_flag) {
  const int C = 3 * H, KS2 = (C + 63) / 64;
  if (KS2 > kBwMaxKS2 || std::getenv("RXMET_NO_CLUSTER") != nullptr) return 0;
  // the exchange buffer (2 Bpad KP floats) is addressed with 32-bit byte offsets
  if (8.0 * ((B + kBTile - 1) / kBTile * kBTile) * (64.0 * KS2) >= 2147483648.0) return 0;
  const size_t lds_cl = bwd_cl_lds(KS2 * 64);
  int device = 0, ncu = 0;
  RXMET_CHECK_HIP(hipGetDevice(&device));
  RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
  BwdClArgs cl;
  cl.ndir = ndir;
  cl.ntiles = (B + kBTile - 1) / kBTile;
  cl.Bpad = cl.ntiles * kBTile;
  cl.KP = KS2 * 64;
  const int pairs = ndir * cl.ntiles;
  // the smallest unit slice per workgroup whose grid fits one workgroup per CU, else the
  // largest slice
  int chosen = 0, ncl = 0;
  for (int UT = 1; UT <= 2 && !chosen; ++UT) {
    if ((H / 16) % UT) continue;
    const int G = H / (16 * UT);
    if (static_cast<int64_t>(pairs) * G <= ncu || UT == 2) {
      chosen = UT;
      cl.G = G;
    }
  }
  if (!chosen) return 0;
  // bf16 planes of the R codes (one when every direction's codes are within +-256)
  int npr = 1;
  for (int k = 0; k < ndir; ++k) {
    const rxmet_gru_qparams *q = plans[k].d->params;
    const Bounds br = bounds_of(q->chan_bits[RXMET_GRU_R], q->chan_unsigned[RXMET_GRU_R]);
    npr = std::max(npr, wgrad::planes_for(br.lo, br.hi, 0.0));
  }
  const void *fn = chosen == 1 ? (npr == 1 ? reinterpret_cast<const void *>(&bwd_recurrence_cl<1, 1>)
                                           : reinterpret_cast<const void *>(&bwd_recurrence_cl<1, 2>))
                               : (npr == 1 ? reinterpret_cast<const void *>(&bwd_recurrence_cl<2, 1>)
                                           : reinterpret_cast<const void *>(&bwd_recurrence_cl<2, 2>));
  RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds_cl)));
  int per_cu = 0;
  RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256 * chosen, lds_cl));
  ncl = per_cu * ncu / cl.G;
  if (ncl < 1) return 0;
  if (ncl > pairs) ncl = pairs;
  if (ncl >= 8) ncl -= ncl % 8;
  cl.UT = chosen;
  cl.ncl = ncl;
  const BwdWorkspace ws(T, B, I, H);
  cl.counters = reinterpret_cast<unsigned *>(plans[0].wsb + ws.sync);
  cl.timeout = reinterpret_cast<int *>(cl.counters + cluster::kCounterStride * ncl);
  cl.spin_limit = cluster::spin_limit();
  for (int k = 0; k < ndir; ++k) {
    hipLaunchKernelGGL(pack_rt_bf16, dim3((H / 16) * 4 * ((KS2 + 1) / 2)), dim3(64), 0, stream, H, KS2,
                       npr, plans[k].d->R_q, const_cast<uint4 *>(plans[k].ba.rt));
    RXMET_CHECK_LAUNCH();
    // padding channels of the exchange rows stay zero
    const int64_t nx = static_cast<int64_t>(2) * cl.Bpad * cl.KP;
    hipLaunchKernelGGL(zero_floats, dim3(256), dim3(256), 0, stream, nx, plans[k].ba.xch);
    RXMET_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, cl.counters,
                     cluster::kCounterStride * ncl + 1);
  RXMET_CHECK_LAUNCH();
  BwdArgs &a1 = plans[ndir > 1 ? 1 : 0].ba;
  void *args[] = {&plans[0].ba, &a1, &cl};
  {
    rxmet::prof::Scope ps__("gru_bwd_recurrence", stream);
    RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * cl.G), dim3(256 * cl.UT), args,
                                               static_cast<unsigned>(lds_cl), stream));
  }
  *timeout_flag = cl.timeout;
  return 1;
}

// The stepped recurrence of one direction (any H): 2 T launches.
static int backward_recurrence_stepped(BwdPlan &plan, int T, int B, int I, int H,
                                       hipStream_t stream) {
  const int C = 3 * H;
  const BwdWorkspace ws(T, B, I, H);
  const rxmet_gru_bwd_dir &d = *plan.d;
  const Bounds br = bounds_of(d.params->chan_bits[RXMET_GRU_R], d.params->chan_unsigned[RXMET_GRU_R]);
  const int npr = wgrad::planes_for(br.lo, br.hi, 0.0);
  __bf16 *rb = reinterpret_cast<__bf16 *>(plan.wsb + ws.rb);
  float *gsum = reinterpret_cast<float *>(plan.wsb + ws.gsum);
  float *dhl = reinterpret_cast<float *>(plan.wsb + ws.dhl);
  // R_q [H][3H] as is: rows are the units (N), the channels c are K
  if (int rc = wgrad::codes_t(d.R_q, C, nullptr, C, H, 1, C, 0.0f, 1.0f, npr, rb, ws.Cp,
                              static_cast<int64_t>(H) * ws.Cp, stream))
    return rc;
  rxmet::prof::Scope ps__("gru_bwd_recurrence", stream);
  const dim3 grid((H + 63) / 64, (B + kBTile - 1) / kBTile);
  wgrad::NtArgs na;
  na.lda = C;
  na.kscale = plan.ba.eff_r;
  na.Bt = rb; na.ldb = ws.Cp; na.bplane = static_cast<int64_t>(H) * ws.Cp;
  na.M = B; na.N = H; na.K = C; na.out = gsum; na.ldo = H;
  // K splits so that the dh GEMM fills the GPU (the parts are summed in order by the next
  // step's pointwise)
  wgrad::nt_plan(B, H, C, kStepMaxSplit, &na.ksplit, &na.kper);
  na.out_split = static_cast<int64_t>(B) * H;
  const int S = na.ksplit;
  for (int t = T - 1; t >= 0; --t) {
    hipLaunchKernelGGL(bwd_step_point, grid, dim3(256), 0, stream, plan.ba, t, S, gsum, dhl);
    RXMET_CHECK_LAUNCH();
    na.A = plan.ba.dq + static_cast<size_t>(t) * B * C;
    if (int rc = wgrad::nt(na, npr, stream)) return rc;
  }
  const int64_t n = static_cast<int64_t>(B) * H;
  hipLaunchKernelGGL(bwd_step_dh0, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                     n, S, dhl, gsum, plan.ba.h0_m, plan.ba.dh0);
  RXMET_CHECK_LAUNCH();
  return 0;
}

static int backward_recurrence_tiles(BwdPlan &plan, int B, int H, hipStream_t stream) {
  const int C = 3 * H, KS2 = (C + 63) / 64;
  hipLaunchKernelGGL(pack_rt_frags, dim3((H / 16) * KS2), dim3(64), 0, stream, H, KS2,
                     plan.d->R_q, const_cast<v4i *>(plan.ba.rfrag),
                     const_cast<float *>(plan.ba.rowsum));
  RXMET_CHECK_LAUNCH();
  const int nwg = (B + kBTile - 1) / kBTile;
  const size_t lds = bwd_lds_bytes(KS2);
  RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&bwd_recurrence),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
  rxmet::prof::Scope ps__("gru_bwd_recurrence", stream);
  hipLaunchKernelGGL(bwd_recurrence, dim3(nwg), dim3(64 * ((H + 31) / 32)), lds, stream, plan.ba);
  RXMET_CHECK_LAUNCH();
  return 0;
}

static int backward_epilogue(int T, int B, int I, int H, BwdPlan &plan, hipStream_t stream) {
  const rxmet_gru_bwd_dir &d = *plan.d;
  const int C = 3 * H;
  const BwdWorkspace ws(T, B, I, H);
  const int nwg = (B + kBTile - 1) / kBTile;
  const int swap_h = plan.torch_layout ? H : 0;
  hipLaunchKernelGGL(fold_bias, dim3((C + 255) / 256), dim3(256), 0, stream, nwg, C,
                     plan.ba.bias_partial, d.dbw, d.dbr, swap_h);
  RXMET_CHECK_LAUNCH();
  const int M = T * B;
  float *part = reinterpret_cast<float *>(plan.wsb + ws.part);
  const float *qsc = reinterpret_cast<const float *>(plan.wsb + ws.qsc);
  {
    rxmet::prof::Scope ps__("gru_bwd_weight_gemms", stream);
    // dx[m][i] = sum_c (dp[m][c] eff_w[c]) W_q[i][c]
    wgrad::NtArgs na;
    na.A = plan.ba.dp; na.lda = C;
    na.kscale = reinterpret_cast<const float *>(plan.wsb + ws.effw);
    na.Bt = reinterpret_cast<const __bf16 *>(plan.wsb + ws.wb); na.ldb = ws.Cp;
    na.bplane = static_cast<int64_t>(I) * ws.Cp;
    na.M = M; na.N = I; na.K = C; na.out = d.dx; na.ldo = I;
    if (int rc = wgrad::nt(na, plan.npw, stream)) return rc;
    // dW[i][c] = eff_x sum_m (x_q - zp_x)[m][i] dp[m][c]
    wgrad::TnArgs ta;
    ta.A = plan.ba.dp; ta.lda = C;
    ta.Bt = reinterpret_cast<const __bf16 *>(plan.wsb + ws.xt); ta.ldb = ws.Mp;
    ta.bplane = static_cast<int64_t>(I) * ws.Mp;
    ta.K = M; ta.P = C; ta.Q = I; ta.S = ws.S_w[plan.npx - 1]; ta.kper = ws.kper_w[plan.npx - 1];
    ta.part = part;
    ta.colsum = nullptr;
    if (int rc = wgrad::tn(ta, plan.npx, stream)) return rc;
    // haste layout dW [I][3H] (masked below), or PyTorch's [3H][I] with the W mask applied here
    if (int rc = plan.torch_layout
                     ? wgrad::tn_finish(part, ta.S, C, I, plan.npx, qsc, d.dW, I, false, nullptr,
                                        nullptr, stream, d.W_mask, H)
                     : wgrad::tn_finish(part, ta.S, C, I, plan.npx, qsc, d.dW, C, true, nullptr,
                                        nullptr, stream))
      return rc;
    // dR[j][c] = eff_h sum_m (h_prev codes)[m][j] dq[m][c]
    ta.A = plan.ba.dq;
    ta.Bt = reinterpret_cast<const __bf16 *>(plan.wsb + ws.ht);
    ta.bplane = static_cast<int64_t>(H) * ws.Mp;
    ta.Q = H; ta.S = ws.S_r[plan.nph - 1]; ta.kper = ws.kper_r[plan.nph - 1];
    if (int rc = wgrad::tn(ta, plan.nph, stream)) return rc;
    if (int rc = plan.torch_layout
                     ? wgrad::tn_finish(part, ta.S, C, H, plan.nph, qsc + I, d.dR, H, false, nullptr,
                                        nullptr, stream, d.R_mask, H)
                     : wgrad::tn_finish(part, ta.S, C, H, plan.nph, qsc + I, d.dR, C, true, nullptr,
                                        nullptr, stream))
      return rc;
  }
  const int64_t n0 = static_cast<int64_t>(T) * B * I,
                n1 = plan.torch_layout ? 0 : static_cast<int64_t>(I) * C,
                n2 = plan.torch_layout ? 0 : static_cast<int64_t>(H) * C;
  int64_t blocks = (n0 + n1 + n2 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  {
    rxmet::prof::Scope ps__("gru_bwd_apply_masks", stream);
    hipLaunchKernelGGL(apply_masks, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, n0, n1,
                       n2, d.dx, d.x_mask, d.dW, d.W_mask, d.dR, d.R_mask);
  }
  RXMET_CHECK_LAUNCH();
  return 0;
}

static int backward_dirs(int ndir, int T, int B, int I, int H, const rxmet_gru_bwd_dir *dirs,
                         bool torch_layout, hipStream_t stream,
                         const rxmet_gru_saved_codes *codes = nullptr,
                         const rxmet_gru_grad_view *views = nullptr) {
  RXMET_CHECK_ARG(ndir == 1 || ndir == 2, "ndir must be 1 or 2");
  RXMET_CHECK_ARG(dirs != nullptr, "dirs must be non-null");
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H % 16 == 0 && H <= kMaxHStepped,
                  "hidden_size must be a multiple of 16 and at most 1024");
  RXMET_CHECK_ARG(static_cast<double>(T + 1) * B * 4 * H < 4294967295.0,
                  "T*B*H too large for the recurrence's 32-bit element offsets");
  BwdPlan plans[2];
  for (int k = 0; k < ndir; ++k)
    if (int rc = backward_prologue(T, B, I, H, dirs[k], codes ? &codes[k] : nullptr, stream,
                                   &plans[k], views ? &views[k] : nullptr))
      return rc;
  for (int k = 0; k < ndir; ++k) plans[k].torch_layout = torch_layout;
  // H > 256 (more R values than the clustered and per-tile kernels keep in registers), or
  // RXMET_BWD_STEPPED set: one pointwise and one GEMM launch per step
  const bool stepped = H > 256 || std::getenv("RXMET_BWD_STEPPED") != nullptr;
  int *timeout_flag = nullptr;
  const int rc = stepped ? 0
                         : backward_recurrence_clustered(plans, ndir, T, B, I, H, stream,
                                                         &timeout_flag);
  if (rc < 0) return rc;
  // the per-tile recurrence holds R as int8 fragments: wider recurrent weights step instead
  bool wide_r = false;
  for (int k = 0; k < ndir; ++k)
    wide_r = wide_r || dirs[k].params->chan_bits[RXMET_GRU_R] > 8 ||
             dirs[k].params->chan_unsigned[RXMET_GRU_R] != 0;
  if (rc == 0)
    for (int k = 0; k < ndir; ++k)
      if (int r = (stepped || wide_r || codes) ? backward_recurrence_stepped(plans[k], T, B, I, H, stream)
                                      : backward_recurrence_tiles(plans[k], B, H, stream))
        return r;
  for (int k = 0; k < ndir; ++k)
    if (int r = backward_epilogue(T, B, I, H, plans[k], stream)) return r;
  if (timeout_flag != nullptr) {
    // a clustered wait that timed out: every gradient of every direction becomes NaN
    const int C = 3 * H;
    cluster::PoisonList pl{};
    for (int k = 0; k < ndir; ++k) {
      const rxmet_gru_bwd_dir &d = *plans[k].d;
      float *ps[6] = {d.dx, d.dW, d.dR, d.dbw, d.dbr, d.dh0};
      const int64_t ns[6] = {static_cast<int64_t>(T) * B * I, static_cast<int64_t>(I) * C,
                             static_cast<int64_t>(H) * C, C, C, static_cast<int64_t>(B) * H};
      for (int j = 0; j < 6; ++j) {
        pl.p[pl.count] = ps[j];
        pl.n[pl.count++] = ns[j];
      }
    }
    hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, timeout_flag, pl);
    RXMET_CHECK_LAUNCH();
  }
  return 0;
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int64_t rxmet_gru_backward_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  if (T < 0 || B < 0 || I < 0 || H < 0) return 0;
  return static_cast<int64_t>(BwdWorkspace(T, B, I, H).total);
}

int rxmet_gru_backward_quant(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_q,
                             const float *R_q, const float *bw_q, const float *br_q,
                             const float *x_q, const float *dh_new, const float *h,
                             const float *v, const rxmet_gru_qparams *params,
                             const uint8_t *x_mask, const uint8_t *h0_mask,
                             const uint8_t *W_mask, const uint8_t *R_mask,
                             const uint8_t *bw_mask, const uint8_t *br_mask,
                             const uint8_t *ih_mask, const uint8_t *hh_mask,
                             const uint8_t *gate_in_mask, const uint8_t *gate_out_mask,
                             const uint8_t *h_mask, float *dx, float *dW, float *dR, float *dbw,
                             float *dbr, float *dh0, void *workspace, void *stream_) {
  clear_error();
  const rxmet_gru_bwd_dir d = {W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, params, x_mask, h0_mask,
                               W_mask, R_mask, bw_mask, br_mask, ih_mask, hh_mask, gate_in_mask,
                               gate_out_mask, h_mask, dx, dW, dR, dbw, dbr, dh0, workspace};
  return backward_dirs(1, T, B, I, H, &d, false, static_cast<hipStream_t>(stream_));
}

int rxmet_gru_backward_quant_dirs(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                  const rxmet_gru_bwd_dir *dirs, void *stream_) {
  clear_error();
  return backward_dirs(ndir, T, B, I, H, dirs, false, static_cast<hipStream_t>(stream_));
}

int rxmet_gru_backward_quant_dirs_x(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                    const rxmet_gru_bwd_dir *dirs, int32_t flags, void *stream_) {
  clear_error();
  return backward_dirs(ndir, T, B, I, H, dirs, (flags & 1) != 0,
                       static_cast<hipStream_t>(stream_));
}

int rxmet_gru_backward_quant_dirs_codes(int32_t ndir, int32_t T, int32_t B, int32_t I, int32_t H,
                                        const rxmet_gru_bwd_dir *dirs, int32_t flags,
                                        const rxmet_gru_saved_codes *codes,
                                        const rxmet_gru_grad_view *views, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(codes != nullptr, "codes must be non-null");
  return backward_dirs(ndir, T, B, I, H, dirs, (flags & 1) != 0,
                       static_cast<hipStream_t>(stream_), codes, views);
}

}  // extern "C"
