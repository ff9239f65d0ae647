// gru_calib.hip — float GRU forward with MinMax statistics (PTQ calibration pass),
// behind rxmet_gru_forward_calibrate.
//
// The same kernel without statistics is the float forward behind rxmet_gru_forward_fp.
//
// Reference: forwardWithCalibrationCPU (operators/quant-gru/src/gru_forward_cpu.cc:58-151)
// and its GPU counterpart forwardWithCalibrationGPU (src/gru_interface.cc:930-1024).
// Main form (H a multiple of 16 up to 1024): the input projection of every step as one fp32
// MFMA GEMM (calib_gemm.h) and the recurrence as a clustered persistent kernel with R resident
// in VGPRs, the 13 activation ranges observed in registers and folded from per-workgroup
// partials.  Fallback (other H) and the float forward: one workgroup per sequence keeps h in
// LDS and walks the T steps with the reference's sequential fp32 summation order (sum over k,
// then + bias) and sigmoid in double, as the reference's CPU template does; its statistics
// are reduced with atomic min/max on order-preserving integer images of the floats.  Either
// way non-finite values are not observed, this call's ranges are merged into the caller's
// running ones, and the per-channel ranges of W, R, bw and br come from calib_params_part /
// calib_params_fold.
#include <cfloat>
#include <cstdlib>

#include "calib_gemm.h"
#include "cluster.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_gru.h"

namespace rxmet {
namespace gru {

constexpr int kCalThreads = 256;
constexpr int kNStat = RXMET_GRU_NGRIDS;

// Order-preserving float <-> uint for atomic min/max on floats.
__device__ __forceinline__ unsigned f2ord(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(unsigned u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

__device__ __forceinline__ void observe(float v, float &mn, float &mx) {
  if (isfinite(v)) {
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
}

template <bool STATS>
__global__ __launch_bounds__(kCalThreads) void calib_forward(
    int T, int B, int I, int H, const float *__restrict__ W, const float *__restrict__ R,
    const float *__restrict__ bw, const float *__restrict__ br, const float *__restrict__ x,
    const float *__restrict__ h0, float *__restrict__ hout, float *__restrict__ v,
    unsigned *__restrict__ gstat /* 2 x 13 ordered (min, max) */) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = 3 * H;
  float *hbuf = reinterpret_cast<float *>(smem);  // [2][H], h_t and h_{t+1}
  float *wx = hbuf + 2 * H;                       // [3H]
  float *rh = wx + C;                             // [3H]
  __shared__ unsigned smin[kNStat], smax[kNStat];
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid < kNStat) {
    smin[tid] = f2ord(FLT_MAX);
    smax[tid] = f2ord(-FLT_MAX);
  }
  const size_t BH = static_cast<size_t>(B) * H;
  for (int j = tid; j < H; j += kCalThreads) {
    const float v0 = h0 ? h0[static_cast<size_t>(b) * H + j] : 0.0f;
    hbuf[j] = v0;
    hout[static_cast<size_t>(b) * H + j] = v0;
  }
  float mn[kNStat], mx[kNStat];
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    mn[i] = FLT_MAX;
    mx[i] = -FLT_MAX;
  }
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const float *hs = hbuf + (t & 1) * H;
    float *hn_s = hbuf + ((t + 1) & 1) * H;
    const float *xt = x + (static_cast<size_t>(t) * B + b) * I;
    if (STATS)
      for (int k = tid; k < I; k += kCalThreads) observe(xt[k], mn[RXMET_GRU_X], mx[RXMET_GRU_X]);
    for (int c = tid; c < C; c += kCalThreads) {
      float si = 0.0f, sh = 0.0f;
      for (int k = 0; k < I; ++k) si += xt[k] * W[static_cast<size_t>(k) * C + c];
      for (int k = 0; k < H; ++k) sh += hs[k] * R[static_cast<size_t>(k) * C + c];
      const float a = si + bw[c], r = sh + br[c];
      wx[c] = a;
      rh[c] = r;
      if (STATS) {
        observe(a, mn[RXMET_GRU_WX], mx[RXMET_GRU_WX]);
        observe(r, mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
      }
    }
    __syncthreads();
    for (int j = tid; j < H; j += kCalThreads) {
      const float zp = wx[j] + rh[j];
      const float rp = wx[H + j] + rh[H + j];
      const float z = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(zp))));
      const float r = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(rp))));
      const float rec = rh[2 * H + j];
      const float rhm = r * rec;
      const float np = wx[2 * H + j] + rhm;
      const float n = tanhf(np);
      const float oldc = z * hs[j];
      const float newc = (1.0f - z) * n;
      const float hn = oldc + newc;
      if (STATS) {
        observe(zp, mn[RXMET_GRU_Z_IN], mx[RXMET_GRU_Z_IN]);
        observe(rp, mn[RXMET_GRU_R_IN], mx[RXMET_GRU_R_IN]);
        observe(np, mn[RXMET_GRU_N_IN], mx[RXMET_GRU_N_IN]);
        observe(z, mn[RXMET_GRU_Z_OUT], mx[RXMET_GRU_Z_OUT]);
        observe(r, mn[RXMET_GRU_R_OUT], mx[RXMET_GRU_R_OUT]);
        observe(n, mn[RXMET_GRU_N_OUT], mx[RXMET_GRU_N_OUT]);
        observe(rhm, mn[RXMET_GRU_MUL_RH], mx[RXMET_GRU_MUL_RH]);
        observe(newc, mn[RXMET_GRU_MUL_NEW], mx[RXMET_GRU_MUL_NEW]);
        observe(oldc, mn[RXMET_GRU_MUL_OLD], mx[RXMET_GRU_MUL_OLD]);
        observe(hn, mn[RXMET_GRU_H], mx[RXMET_GRU_H]);
      }
      hout[(t + 1) * BH + static_cast<size_t>(b) * H + j] = hn;
      if (v) {
        float *vb = v + (static_cast<size_t>(t) * B + b) * 4 * H + j;
        vb[0] = z;
        vb[H] = r;
        vb[2 * H] = n;
        vb[3 * H] = rec;
      }
      hn_s[j] = hn;
    }
    __syncthreads();
  }
  if (!STATS) return;
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    if (mn[i] <= mx[i]) {
      atomicMin(&smin[i], f2ord(mn[i]));
      atomicMax(&smax[i], f2ord(mx[i]));
    }
  }
  __syncthreads();
  if (tid < kNStat) {
    atomicMin(&gstat[tid], smin[tid]);
    atomicMax(&gstat[kNStat + tid], smax[tid]);
  }
}

// This call's ranges start empty (min=FLT_MAX, max=-FLT_MAX) in ordered-uint form.
__global__ void stats_init(unsigned *o) {
  const int i = threadIdx.x;
  if (i < kNStat) {
    o[i] = f2ord(FLT_MAX);
    o[kNStat + i] = f2ord(-FLT_MAX);
  }
}
// Merge this call's ranges into the running ones.  A tensor without any finite value
// contributes the range [0, 0], as the reference's min/max update does.
__global__ void stats_merge(const unsigned *o, float *s) {
  const int i = threadIdx.x;
  if (i < kNStat) {
    float lo = ord2f(o[i]), hi = ord2f(o[kNStat + i]);
    if (lo > hi) lo = hi = 0.0f;
    s[i] = lo < s[i] ? lo : s[i];
    s[kNStat + i] = hi > s[kNStat + i] ? hi : s[kNStat + i];
  }
}

// ---------------------------------------------------------------------------------
// MFMA form (H a multiple of 16, H <= 1024): the input projection of every step as one fp32
// MFMA GEMM, then the recurrence as a clustered persistent kernel with R resident in VGPRs.
// Products and sums are fp32 (v_mfma_f32_16x16x4f32) in another order than the sequential
// sums above; results agree to rounding (the calibration is held to 1e-5, not bit-exactness).
// Statistics: every workgroup writes its (min, max) partials to the workspace and one small
// kernel folds them, in a fixed order, into this call's ordered ranges (no contended atomics).
// ---------------------------------------------------------------------------------
constexpr int kCT = 16;      // batch rows of a tile
constexpr int kCMaxW = 16;   // waves of a recurrence workgroup

// Block-wide (min, max) of n statistics, written by thread 0 to part[0..n) / part[n..2n).
__device__ __forceinline__ void block_stats(const float *mn, const float *mx, int n, float *part) {
  __shared__ float smn[kCMaxW][kNStat], smx[kCMaxW][kNStat];
  const int w = threadIdx.x / kWave, nw = blockDim.x / kWave;
#pragma unroll
  for (int i = 0; i < n; ++i) {  // unrolled (n is a constant where inlined): mn, mx stay in registers
    const float lo = wave_min(mn[i]), hi = wave_max(mx[i]);
    if (threadIdx.x % kWave == 0) {
      smn[w][i] = lo;
      smx[w][i] = hi;
    }
  }
  __syncthreads();
  if (threadIdx.x < n) {
    float lo = smn[0][threadIdx.x], hi = smx[0][threadIdx.x];
    for (int ww = 1; ww < nw; ++ww) {
      lo = fminf(lo, smn[ww][threadIdx.x]);
      hi = fmaxf(hi, smx[ww][threadIdx.x]);
    }
    part[threadIdx.x] = lo;
    part[n + threadIdx.x] = hi;
  }
}

// Fold P partial blocks of 2 N floats (N statistics starting at i0) into the ordered ranges
// (statistics a block did not observe hold FLT_MAX / -FLT_MAX and change nothing).  Each
// thread takes whole partial blocks, all of a block's loads issued together, so the pass over
// P blocks is one latency per 256 blocks rather than one per statistic and block.
template <int N>
__global__ __launch_bounds__(256) void stats_fold(const float *__restrict__ part, int P, int i0,
                                                  unsigned *__restrict__ ostat) {
  __shared__ float smn[4][N], smx[4][N];
  const int w = threadIdx.x / kWave;
  float lo[N], hi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    lo[i] = FLT_MAX;
    hi[i] = -FLT_MAX;
  }
  for (int p = threadIdx.x; p < P; p += blockDim.x) {
    const float *q = part + static_cast<size_t>(p) * 2 * N;
    float v[2 * N];
#pragma unroll
    for (int i = 0; i < 2 * N; ++i) v[i] = q[i];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      lo[i] = fminf(lo[i], v[i]);
      hi[i] = fmaxf(hi[i], v[N + i]);
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float a = wave_min(lo[i]), b = wave_max(hi[i]);
    if (threadIdx.x % kWave == 0) {
      smn[w][i] = a;
      smx[w][i] = b;
    }
  }
  __syncthreads();
  if (threadIdx.x < N) {
    float a = smn[0][threadIdx.x], b = smx[0][threadIdx.x];
    for (int ww = 1; ww < 4; ++ww) {
      a = fminf(a, smn[ww][threadIdx.x]);
      b = fmaxf(b, smx[ww][threadIdx.x]);
    }
    if (a <= b) {  // merged: one thread per statistic, so no contention
      atomicMin(&ostat[i0 + threadIdx.x], f2ord(a));
      atomicMax(&ostat[kNStat + i0 + threadIdx.x], f2ord(b));
    }
  }
}

// The statistics the input GEMM observes, x and the input linear, lie among the first three.
constexpr int kGemmStat = 3;
static_assert(RXMET_GRU_X < kGemmStat && RXMET_GRU_WX < kGemmStat, "GEMM statistics layout");

// wx[m][c] = sum_k x[m][k] W[k][c] + bw[c] for m < M = T B, c < C = 3H (W [I][3H], K-major),
// with the X and WX statistics: the LDS-tiled fp32 MFMA block of calib_gemm.h, one partial
// block of statistics per workgroup.
template <bool STATS>
__global__ __launch_bounds__(256) void calib_input_gemm(int M, int K, int C,
                                                        const float *__restrict__ x,
                                                        const float *__restrict__ W,
                                                        const float *__restrict__ bw,
                                                        float *__restrict__ wx,
                                                        float *__restrict__ part) {
  float st_mn[kGemmStat], st_mx[kGemmStat];
#pragma unroll
  for (int i = 0; i < kGemmStat; ++i) {
    st_mn[i] = FLT_MAX;
    st_mx[i] = -FLT_MAX;
  }
  calgemm::gemm_block<true>(
      M, C, K, x, W, bw, wx, STATS && blockIdx.x == 0,
      [&](float v) {
        if (STATS) observe(v, st_mn[RXMET_GRU_X], st_mx[RXMET_GRU_X]);
      },
      [&](float v) {
        if (STATS) observe(v, st_mn[RXMET_GRU_WX], st_mx[RXMET_GRU_WX]);
      });
  if (STATS)
    block_stats(st_mn, st_mx, kGemmStat,
                part + (static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x) * 2 * kGemmStat);
}

struct CalClArgs {
  int T, B, H, NC, NWG, ntiles, Bpad, Hpad, G, ncl;
  const float *wx;   // [T, B, 3H] input projection with bw
  const float *R;    // [H, 3H]
  const float *br;   // [3H]
  const float *h0;   // [B, H] or null
  float *hout;       // [T+1, B, H]
  float *v;          // [T, B, 4H] or null
  float *hx;         // [2][Bpad][Hpad] exchanged h (padding columns zero)
  float *part;       // [ncl G][2 x 13] partial statistics
  unsigned *counters;
  int *timeout;
  unsigned spin_limit;
};

// The recurrent product of one member for one tile: wave w takes the consecutive items
// w IPW .. w IPW + IPW - 1 (item = 3 chunk + gate), so the three gates of a K chunk share one
// load of its h values; every chunk the wave needs is loaded before the first MFMA.  Partial
// tiles go to red[item][64].
template <int IPW>
__device__ __forceinline__ void calib_items(const float (&rfr)[IPW][16], int w, int l, int g,
                                            int nitems, __amdgpu_buffer_rsrc_t xr, unsigned rowoff,
                                            v4f *red) {
  // chunks a run of IPW items spans (IPW items from a multiple of 3 when IPW is one)
  constexpr int NCH = IPW % 3 == 0 ? IPW / 3 : (IPW + 1) / 3 + 1;
  const int first = (w * IPW) / 3;
  float hv[NCH][16];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = first + c;
    if (3 * ch < nitems) {
      const unsigned off = 4u * (rowoff + 64 * ch + 16 * g);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 v = cluster::load_coherent16(xr, off + 16u * q);
        hv[c][4 * q] = __int_as_float(v.x);
        hv[c][4 * q + 1] = __int_as_float(v.y);
        hv[c][4 * q + 2] = __int_as_float(v.z);
        hv[c][4 * q + 3] = __int_as_float(v.w);
      }
    }
  }
#pragma unroll
  for (int it = 0; it < IPW; ++it) {
    const int item = w * IPW + it;
    if (item >= nitems) break;
    // the item's chunk among the loaded ones: static when IPW is a multiple of 3, else selected
    // (a register array indexed at run time would live in scratch memory)
    const int c = IPW % 3 == 0 ? it / 3 : item / 3 - first;
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      float hs = hv[0][s];
#pragma unroll
      for (int cc = 1; cc < NCH; ++cc) hs = c == cc ? hv[cc][s] : hs;
      acc = mfma_f32(hs, rfr[it][s], acc);
    }
    red[item * kWave + l] = acc;
  }
}

// Member m of a cluster owns units 16 m .. 16 m + 15 of one 16-row batch tile.  The recurrent
// product splits into items (k chunk c of 64, gate): 3 NC items, dealt to the workgroup's NWG
// waves (wave w takes IPW consecutive items, calib_items).  An item is sixteen MFMAs, MFMA s
// taking k = 64 c + 16 g + s for lane group g, so a lane's A values are 16 consecutive h of its
// row (four 16-byte coherent loads) and its B values (R) stay in VGPRs for the whole launch.
// The items' partial tiles meet in LDS; each of the tile's 256 (row, unit) elements is then
// finished by one thread (the gates, the new h and the statistics), its previous h kept in a
// register.  NWG >= 4, so the 256 elements have threads of their own.
template <bool STATS, int IPW, int MAXW = kCMaxW>
__global__ __launch_bounds__(64 * MAXW) void calib_recurrence_cl(CalClArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  v4f *red = reinterpret_cast<v4f *>(smem);  // [3 NC][64]
  const cluster::Place pl = cluster::place(a.G, a.ncl);
  unsigned *counter = a.counters + cluster::kCounterStride * pl.cluster;
  const int H = a.H, C = 3 * H, B = a.B, NC = a.NC;
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave, r16 = l % 16, g = l / 16;
  const int u0 = 16 * pl.member;
  const int nitems = 3 * NC;
  float rfr[IPW][16];
#pragma unroll
  for (int it = 0; it < IPW; ++it) {
    const int item = w * IPW + it, ch = item / 3, gate = item % 3;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int k = 64 * ch + 16 * g + s;
      rfr[it][s] = item < nitems && k < H
                       ? a.R[static_cast<size_t>(k) * C + gate * H + u0 + r16] : 0.0f;
    }
  }
  // the finishing element of this thread (tid < 256): row 4 (tid % 64 / 16) + tid / 64 and
  // unit u0 + tid % 16 of the tile, which lane tid % 64 holds as accumulator tid / 64
  const bool fin = tid < 256;
  const int fl = tid % 64, fq = tid / 64;
  const int frow = 4 * (fl / 16) + fq, fu = u0 + fl % 16;
  const float bz = fin ? a.br[fu] : 0.0f, brr = fin ? a.br[H + fu] : 0.0f,
              bn = fin ? a.br[2 * H + fu] : 0.0f;
  float mn[kNStat], mx[kNStat];
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    mn[i] = FLT_MAX;
    mx[i] = -FLT_MAX;
  }
  const unsigned plane = static_cast<unsigned>(a.Bpad) * a.Hpad;  // floats per parity
  const auto xr = cluster::buffer_rsrc(a.hx, 2u * plane * 4u);
  unsigned *hxw = reinterpret_cast<unsigned *>(a.hx);
  const size_t BH = static_cast<size_t>(B) * H;
  unsigned epoch = 0;
  bool alive = true;
  for (int tile = pl.cluster; tile < a.ntiles && alive; tile += a.ncl) {
    __syncthreads();  // the previous tile's readers of the partial tiles are done
    const int b = tile * kCT + frow;
    const bool valid = fin && b < B;
    float hold = 0.0f;
    if (fin) {
      hold = valid && a.h0 ? a.h0[static_cast<size_t>(b) * H + fu] : 0.0f;
      cluster::store_coherent(hxw + b * a.Hpad + fu, __float_as_uint(hold));
      if (valid) a.hout[static_cast<size_t>(b) * H + fu] = hold;
    }
    // the step's weight_ih_linear values, loaded one step ahead (they do not depend on h)
    float wz = 0.0f, wr = 0.0f, wn = 0.0f;
    auto load_wx = [&](int t) {
      if (valid) {
        const float *wp = a.wx + (static_cast<size_t>(t) * B + b) * C + fu;
        wz = wp[0];
        wr = wp[H];
        wn = wp[2 * H];
      }
    };
    load_wx(0);
    alive = cluster::sync(counter, ++epoch * a.G, a.timeout, a.spin_limit);
    for (int t = 0; t < a.T && alive; ++t) {
      const int par = t & 1;
      const unsigned rowoff = par * plane + static_cast<unsigned>(tile * kCT + r16) * a.Hpad;
      // A: row tile*16 + r16, h[64 ch + 16 g .. + 15] of each item's chunk
      calib_items<IPW>(rfr, w, l, g, nitems, xr, rowoff, red);
      __syncthreads();
      if (fin) {
        float rh[3] = {bz, brr, bn};
        for (int ch = 0; ch < NC; ++ch)
#pragma unroll
          for (int gate = 0; gate < 3; ++gate) rh[gate] += red[(ch * 3 + gate) * kWave + fl][fq];
        const float zp = wz + rh[0];
        const float rp = wr + rh[1];
        const float z = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(zp))));
        const float r = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(rp))));
        const float rhm = r * rh[2];
        const float np = wn + rhm;
        const float n = tanhf(np);
        const float oldc = z * hold;
        const float newc = (1.0f - z) * n;
        const float hn = oldc + newc;
        hold = hn;
        cluster::store_coherent(hxw + (par ^ 1) * plane + b * a.Hpad + fu, __float_as_uint(hn));
        if (STATS && valid) {
          observe(rh[0], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(rh[1], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(rh[2], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(zp, mn[RXMET_GRU_Z_IN], mx[RXMET_GRU_Z_IN]);
          observe(rp, mn[RXMET_GRU_R_IN], mx[RXMET_GRU_R_IN]);
          observe(np, mn[RXMET_GRU_N_IN], mx[RXMET_GRU_N_IN]);
          observe(z, mn[RXMET_GRU_Z_OUT], mx[RXMET_GRU_Z_OUT]);
          observe(r, mn[RXMET_GRU_R_OUT], mx[RXMET_GRU_R_OUT]);
          observe(n, mn[RXMET_GRU_N_OUT], mx[RXMET_GRU_N_OUT]);
          observe(rhm, mn[RXMET_GRU_MUL_RH], mx[RXMET_GRU_MUL_RH]);
          observe(newc, mn[RXMET_GRU_MUL_NEW], mx[RXMET_GRU_MUL_NEW]);
          observe(oldc, mn[RXMET_GRU_MUL_OLD], mx[RXMET_GRU_MUL_OLD]);
          observe(hn, mn[RXMET_GRU_H], mx[RXMET_GRU_H]);
        }
        cluster::arrive(counter);
        ++epoch;
        if (valid) {
          a.hout[(static_cast<size_t>(t) + 1) * BH + static_cast<size_t>(b) * H + fu] = hn;
          if (a.v) {
            float *vb = a.v + (static_cast<size_t>(t) * B + b) * 4 * H + fu;
            vb[0] = z;
            vb[H] = r;
            vb[2 * H] = n;
            vb[3 * H] = rh[2];
          }
        }
        if (t + 1 < a.T) load_wx(t + 1);
      } else {
        cluster::arrive(counter);
        ++epoch;
      }
      alive = cluster::wait(counter, epoch * a.G, a.timeout, a.spin_limit);
    }
  }
  if (STATS) {
    __syncthreads();
    block_stats(mn, mx, kNStat,
                a.part + (static_cast<size_t>(blockIdx.x)) * 2 * kNStat);
  }
}

// The multi-tile form of calib_recurrence_cl, for clusters that own several batch tiles
// (ntiles > ncl; c5: 64 tiles over 4 clusters): each step runs all of the cluster's tiles, one
// after another, and meets the other members once, so a step pays one cluster barrier for up
// to kMtMax tiles instead of one per tile.  Each tile's previous h (one per finishing thread)
// waits in LDS between steps; the next tile's input linear is loaded while this one computes.
constexpr int kMtMax = 16;

template <bool STATS, int IPW, int MAXW = kCMaxW>
__global__ __launch_bounds__(64 * MAXW) void calib_recurrence_mt(CalClArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  v4f *red = reinterpret_cast<v4f *>(smem);                             // [3 NC][64]
  float *hl = reinterpret_cast<float *>(red + 3 * a.NC * kWave);        // [kMtMax][256]
  const cluster::Place pl = cluster::place(a.G, a.ncl);
  unsigned *counter = a.counters + cluster::kCounterStride * pl.cluster;
  const int H = a.H, C = 3 * H, B = a.B, NC = a.NC;
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave, r16 = l % 16, g = l / 16;
  const int u0 = 16 * pl.member;
  const int nitems = 3 * NC;
  const int nT = (a.ntiles - pl.cluster + a.ncl - 1) / a.ncl;  // <= kMtMax (launcher)
  float rfr[IPW][16];
#pragma unroll
  for (int it = 0; it < IPW; ++it) {
    const int item = w * IPW + it, ch = item / 3, gate = item % 3;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int k = 64 * ch + 16 * g + s;
      rfr[it][s] = item < nitems && k < H
                       ? a.R[static_cast<size_t>(k) * C + gate * H + u0 + r16] : 0.0f;
    }
  }
  const bool fin = tid < 256;
  const int fl = tid % 64, fq = tid / 64;
  const int frow = 4 * (fl / 16) + fq, fu = u0 + fl % 16;
  const float bz = fin ? a.br[fu] : 0.0f, brr = fin ? a.br[H + fu] : 0.0f,
              bn = fin ? a.br[2 * H + fu] : 0.0f;
  float mn[kNStat], mx[kNStat];
#pragma unroll
  for (int i = 0; i < kNStat; ++i) {
    mn[i] = FLT_MAX;
    mx[i] = -FLT_MAX;
  }
  const unsigned plane = static_cast<unsigned>(a.Bpad) * a.Hpad;  // floats per parity
  const auto xr = cluster::buffer_rsrc(a.hx, 2u * plane * 4u);
  unsigned *hxw = reinterpret_cast<unsigned *>(a.hx);
  const size_t BH = static_cast<size_t>(B) * H;
  // initial states of every tile
  for (int k = 0; k < nT; ++k) {
    const int b = (pl.cluster + k * a.ncl) * kCT + frow;
    if (fin) {
      const float h0 = b < B && a.h0 ? a.h0[static_cast<size_t>(b) * H + fu] : 0.0f;
      cluster::store_coherent(hxw + b * a.Hpad + fu, __float_as_uint(h0));
      if (b < B) a.hout[static_cast<size_t>(b) * H + fu] = h0;
      hl[k * 256 + tid] = h0;
    }
  }
  float wz = 0.0f, wr = 0.0f, wn = 0.0f;
  auto load_wx = [&](int t, int k) {
    const int b = (pl.cluster + k * a.ncl) * kCT + frow;
    if (fin && b < B) {
      const float *wp = a.wx + (static_cast<size_t>(t) * B + b) * C + fu;
      wz = wp[0];
      wr = wp[H];
      wn = wp[2 * H];
    }
  };
  load_wx(0, 0);
  unsigned epoch = 0;
  bool alive = cluster::sync(counter, ++epoch * a.G, a.timeout, a.spin_limit);
  for (int t = 0; t < a.T && alive; ++t) {
    const int par = t & 1;
    for (int k = 0; k < nT; ++k) {
      const int tile = pl.cluster + k * a.ncl;
      const int b = tile * kCT + frow;
      const bool valid = fin && b < B;
      const unsigned rowoff = par * plane + static_cast<unsigned>(tile * kCT + r16) * a.Hpad;
      calib_items<IPW>(rfr, w, l, g, nitems, xr, rowoff, red);
      __syncthreads();
      if (fin) {
        const float cz = wz, cr = wr, cn = wn;
        // the next tile's (or the next step's first tile's) input linear, in flight meanwhile
        if (k + 1 < nT)
          load_wx(t, k + 1);
        else if (t + 1 < a.T)
          load_wx(t + 1, 0);
        float rh[3] = {bz, brr, bn};
        for (int ch = 0; ch < NC; ++ch)
#pragma unroll
          for (int gate = 0; gate < 3; ++gate) rh[gate] += red[(ch * 3 + gate) * kWave + fl][fq];
        const float hold = hl[k * 256 + tid];
        const float zp = cz + rh[0];
        const float rp = cr + rh[1];
        const float z = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(zp))));
        const float r = static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(rp))));
        const float rhm = r * rh[2];
        const float np = cn + rhm;
        const float n = tanhf(np);
        const float oldc = z * hold;
        const float newc = (1.0f - z) * n;
        const float hn = oldc + newc;
        hl[k * 256 + tid] = hn;
        cluster::store_coherent(hxw + (par ^ 1) * plane + b * a.Hpad + fu, __float_as_uint(hn));
        if (STATS && valid) {
          observe(rh[0], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(rh[1], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(rh[2], mn[RXMET_GRU_RH], mx[RXMET_GRU_RH]);
          observe(zp, mn[RXMET_GRU_Z_IN], mx[RXMET_GRU_Z_IN]);
          observe(rp, mn[RXMET_GRU_R_IN], mx[RXMET_GRU_R_IN]);
          observe(np, mn[RXMET_GRU_N_IN], mx[RXMET_GRU_N_IN]);
          observe(z, mn[RXMET_GRU_Z_OUT], mx[RXMET_GRU_Z_OUT]);
          observe(r, mn[RXMET_GRU_R_OUT], mx[RXMET_GRU_R_OUT]);
          observe(n, mn[RXMET_GRU_N_OUT], mx[RXMET_GRU_N_OUT]);
          observe(rhm, mn[RXMET_GRU_MUL_RH], mx[RXMET_GRU_MUL_RH]);
          observe(newc, mn[RXMET_GRU_MUL_NEW], mx[RXMET_GRU_MUL_NEW]);
          observe(oldc, mn[RXMET_GRU_MUL_OLD], mx[RXMET_GRU_MUL_OLD]);
          observe(hn, mn[RXMET_GRU_H], mx[RXMET_GRU_H]);
        }
        if (valid) {
          a.hout[(static_cast<size_t>(t) + 1) * BH + static_cast<size_t>(b) * H + fu] = hn;
          if (a.v) {
            float *vb = a.v + (static_cast<size_t>(t) * B + b) * 4 * H + fu;
            vb[0] = z;
            vb[H] = r;
            vb[2 * H] = n;
            vb[3 * H] = rh[2];
          }
        }
      }
      __syncthreads();  // the partial tiles are read before the next tile rewrites them
    }
    cluster::arrive(counter);
    ++epoch;
    alive = cluster::wait(counter, epoch * a.G, a.timeout, a.spin_limit);
  }
  if (STATS) {
    __syncthreads();
    block_stats(mn, mx, kNStat, a.part + static_cast<size_t>(blockIdx.x) * 2 * kNStat);
  }
}

// Rows of W and R (concatenated) per workgroup of the parameter ranges.
constexpr int kPrmRows = 64;

struct CalWorkspace {
  size_t ord, wx, hx, part, sync, prm, total;
  int Bpad, Hpad, ntiles;
  int64_t nparts;
  int prm_slabs;
  CalWorkspace(int T, int B, int I, int H) {
    auto al = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    ntiles = (B + kCT - 1) / kCT;
    Bpad = ntiles * kCT;
    Hpad = (H + 63) / 64 * 64;
    const int64_t M = static_cast<int64_t>(T) * B;
    const int64_t gemm_blocks = (3 * static_cast<int64_t>(H) + 63) / 64 * ((M + 63) / 64);
    const int64_t rec_blocks = static_cast<int64_t>(ntiles) * (H / 16 > 0 ? H / 16 : 1);
    nparts = 2 * kNStat * (gemm_blocks > rec_blocks ? gemm_blocks : rec_blocks);
    size_t o = 0;
    ord = o; o += al(sizeof(unsigned) * 2 * kNStat);
    wx = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * 3 * H);
    hx = o; o += al(sizeof(float) * 2 * static_cast<size_t>(Bpad) * Hpad);
    part = o; o += al(sizeof(float) * static_cast<size_t>(nparts));
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (ntiles + 2));
    prm_slabs = (I + H + kPrmRows - 1) / kPrmRows;
    prm = o; o += al(sizeof(float) * 4 * static_cast<size_t>(prm_slabs) * 3 * H);
    total = o;
  }
};

// The MFMA form when it applies (H a multiple of 16 up to 1024, the clusters resident);
// returns 1 when launched, 0 when the caller must use the per-sequence kernel.
template <bool STATS>
static int calibrate_mfma(int T, int B, int I, int H, const float *W, const float *R,
                          const float *bw, const float *br, const float *x, const float *h0,
                          float *h, float *v, void *workspace, hipStream_t stream) {
  if (H % 16 != 0 || H > 1024 || std::getenv("RXMET_NO_CLUSTER") != nullptr) return 0;
  const CalWorkspace ws(T, B, I, H);
  if (2.0 * ws.Bpad * ws.Hpad * 4 >= 2147483648.0) return 0;  // 32-bit exchange offsets
  CalClArgs a{};
  a.T = T; a.B = B; a.H = H;
  a.NC = (H + 63) / 64;
  // up to 320 units: 4..16 waves of one item (1024 threads, 128 VGPRs); above, 8 waves of
  // 3..6 items (512 threads, 256 VGPRs: two or three items per wave at 1024 threads spilled)
  const bool wide = 3 * a.NC > kCMaxW;
  a.NWG = wide ? 8 : std::max(4, 3 * a.NC);
  const int ipw = (3 * a.NC + a.NWG - 1) / a.NWG;  // 1, or 3..6 when wide
  a.ntiles = ws.ntiles; a.Bpad = ws.Bpad; a.Hpad = ws.Hpad;
  a.G = H / 16;
  using K = const void *;
  const K cl_fns[7] = {nullptr,
                       reinterpret_cast<K>(&calib_recurrence_cl<STATS, 1>),
                       nullptr,
                       reinterpret_cast<K>(&calib_recurrence_cl<STATS, 3, 8>),
                       reinterpret_cast<K>(&calib_recurrence_cl<STATS, 4, 8>),
                       reinterpret_cast<K>(&calib_recurrence_cl<STATS, 5, 8>),
                       reinterpret_cast<K>(&calib_recurrence_cl<STATS, 6, 8>)};
  const K mt_fns[7] = {nullptr,
                       reinterpret_cast<K>(&calib_recurrence_mt<STATS, 1>),
                       nullptr,
                       reinterpret_cast<K>(&calib_recurrence_mt<STATS, 3, 8>),
                       reinterpret_cast<K>(&calib_recurrence_mt<STATS, 4, 8>),
                       reinterpret_cast<K>(&calib_recurrence_mt<STATS, 5, 8>),
                       reinterpret_cast<K>(&calib_recurrence_mt<STATS, 6, 8>)};
  const void *fn = cl_fns[ipw];
  size_t lds = sizeof(v4f) * kWave * 3 * static_cast<size_t>(a.NC);
  RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
  int device = 0, ncu = 0, per_cu = 0;
  RXMET_CHECK_HIP(hipGetDevice(&device));
  RXMET_CHECK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
  RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWave * a.NWG, lds));
  int ncl = per_cu * ncu / a.G;
  if (ncl < 1) return 0;
  if (ncl > a.ntiles) ncl = a.ntiles;
  if (ncl >= 8) ncl -= ncl % 8;
  a.ncl = ncl;
  // clusters owning several tiles run them all in each step (one barrier per step), when
  // the multi-tile kernel's occupancy allows the same cluster count
  if (a.ntiles > ncl && (a.ntiles + ncl - 1) / ncl <= kMtMax &&
      std::getenv("RXMET_CALIB_TILEWISE") == nullptr) {
    const void *mt = mt_fns[ipw];
    const size_t lds_mt = lds + sizeof(float) * kMtMax * 256;
    RXMET_CHECK_HIP(hipFuncSetAttribute(mt, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds_mt)));
    int per_cu_mt = 0;
    RXMET_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_mt, mt, kWave * a.NWG,
                                                                 lds_mt));
    if (per_cu_mt >= per_cu) {
      fn = mt;
      lds = lds_mt;
    }
  }
  char *wsb = static_cast<char *>(workspace);
  unsigned *ord = reinterpret_cast<unsigned *>(wsb + ws.ord);
  float *wx = reinterpret_cast<float *>(wsb + ws.wx);
  float *part = reinterpret_cast<float *>(wsb + ws.part);
  a.hx = reinterpret_cast<float *>(wsb + ws.hx);
  a.counters = reinterpret_cast<unsigned *>(wsb + ws.sync);
  a.timeout = reinterpret_cast<int *>(a.counters + cluster::kCounterStride * ncl);
  a.spin_limit = cluster::spin_limit();
  const int C = 3 * H;
  const int M = T * B;
  {
    rxmet::prof::Scope ps__("gru_calibrate_input_gemm", stream);
    const dim3 grid(static_cast<unsigned>((C + calgemm::kBN - 1) / calgemm::kBN),
                    static_cast<unsigned>((M + calgemm::kBM - 1) / calgemm::kBM));
    hipLaunchKernelGGL(calib_input_gemm<STATS>, grid, dim3(256), 0, stream, M, I, C, x, W, bw,
                       wx, part);
    RXMET_CHECK_LAUNCH();
    if (STATS) {
      hipLaunchKernelGGL(stats_fold<kGemmStat>, dim3(1), dim3(256), 0, stream, part,
                         static_cast<int>(grid.x * grid.y), 0, ord);
      RXMET_CHECK_LAUNCH();
    }
  }
  // the exchange buffer's padding columns must read as zero
  hipLaunchKernelGGL(cluster::zero_words, dim3(cluster::zero_blocks(2 * ws.Bpad * ws.Hpad)),
                     dim3(256), 0, stream, reinterpret_cast<unsigned *>(a.hx),
                     2 * ws.Bpad * ws.Hpad);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, a.counters,
                     cluster::kCounterStride * ncl + 1);
  RXMET_CHECK_LAUNCH();
  a.wx = wx; a.R = R; a.br = br; a.h0 = h0; a.hout = h; a.v = v; a.part = part;
  void *args[] = {&a};
  {
    rxmet::prof::Scope ps__("gru_calibrate_forward", stream);
    RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * a.G), dim3(kWave * a.NWG), args,
                                    static_cast<unsigned>(lds), stream));
    if (STATS) {
      hipLaunchKernelGGL(stats_fold<kNStat>, dim3(1), dim3(256), 0, stream, part, ncl * a.G, 0,
                         ord);
      RXMET_CHECK_LAUNCH();
    }
  }
  // a wait that timed out: the outputs become NaN (the statistics skip non-finite values)
  cluster::PoisonList pl{};
  pl.p[pl.count] = h;
  pl.n[pl.count++] = static_cast<int64_t>(T + 1) * B * H;
  if (v) {
    pl.p[pl.count] = v;
    pl.n[pl.count++] = static_cast<int64_t>(T) * B * 4 * H;
  }
  hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, a.timeout, pl);
  RXMET_CHECK_LAUNCH();
  return 1;
}

// Per-channel min / max over the finite values of W, R and the two biases, merged into the
// running ranges (a channel with no finite value contributes 0 to both).  calib_params_part:
// workgroup (x, s) takes 64 columns of rows [s kPrmRows, +kPrmRows) of W and R stacked, its four
// waves on interleaved rows, and writes the slab's min / max per column; calib_params_fold
// folds the slabs of a column and merges.
__global__ __launch_bounds__(256) void calib_params_part(int I, int H, const float *W,
                                                         const float *R,
                                                         float *part /* [S][2][2][C] */) {
  const int C = 3 * H;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int r0 = blockIdx.y * kPrmRows, r1 = min(I + H, r0 + kPrmRows);
  float lw = FLT_MAX, hw = -FLT_MAX, lr = FLT_MAX, hr = -FLT_MAX;
  if (c < C) {
    for (int r = r0 + w; r < r1; r += 4) {
      const bool in_w = r < I;
      const float v = in_w ? W[static_cast<size_t>(r) * C + c]
                           : R[static_cast<size_t>(r - I) * C + c];
      if (!isfinite(v)) continue;
      if (in_w) {
        lw = fminf(lw, v);
        hw = fmaxf(hw, v);
      } else {
        lr = fminf(lr, v);
        hr = fmaxf(hr, v);
      }
    }
  }
  __shared__ float red[4][4][64];
  red[w][0][lane] = lw;
  red[w][1][lane] = hw;
  red[w][2][lane] = lr;
  red[w][3][lane] = hr;
  __syncthreads();
  if (w != 0 || c >= C) return;
  for (int q = 1; q < 4; ++q) {
    lw = fminf(lw, red[q][0][lane]);
    hw = fmaxf(hw, red[q][1][lane]);
    lr = fminf(lr, red[q][2][lane]);
    hr = fmaxf(hr, red[q][3][lane]);
  }
  float *p = part + static_cast<size_t>(blockIdx.y) * 4 * C;
  p[c] = lw;
  p[C + c] = hw;
  p[2 * C + c] = lr;
  p[3 * C + c] = hr;
}

__global__ __launch_bounds__(256) void calib_params_fold(int H, int S, const float *part,
                                                         const float *bw, const float *br,
                                                         float *chan /* 4 x (min[C], max[C]) */) {
  const int C = 3 * H;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float lo[4], hi[4];
  lo[0] = lo[1] = FLT_MAX;
  hi[0] = hi[1] = -FLT_MAX;
  for (int s = 0; s < S; ++s) {
    const float *p = part + static_cast<size_t>(s) * 4 * C;
    lo[0] = fminf(lo[0], p[c]);
    hi[0] = fmaxf(hi[0], p[C + c]);
    lo[1] = fminf(lo[1], p[2 * C + c]);
    hi[1] = fmaxf(hi[1], p[3 * C + c]);
  }
  const float b0 = bw[c], b1 = br[c];
  lo[2] = hi[2] = isfinite(b0) ? b0 : 0.0f;
  lo[3] = hi[3] = isfinite(b1) ? b1 : 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float l = lo[k], h = hi[k];
    if (l > h) l = h = 0.0f;
    float *mn = chan + static_cast<size_t>(k) * 2 * C, *mx = mn + C;
    mn[c] = l < mn[c] ? l : mn[c];
    mx[c] = h > mx[c] ? h : mx[c];
  }
}

}  // namespace gru
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::gru;

extern "C" {

int64_t rxmet_gru_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  (void)I;
  if (T < 1 || B < 1 || H < 1) return static_cast<int64_t>(sizeof(unsigned) * 2 * kNStat);
  return static_cast<int64_t>(CalWorkspace(T, B, I, H).total);
}

int rxmet_gru_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W,
                                const float *R, const float *bw, const float *br,
                                const float *x, const float *h0, float *h, float *v,
                                float *stats, void *workspace, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 4096, "hidden_size above 4096 is not supported by the calibration pass");
  RXMET_CHECK_ARG(W && R && bw && br && x && h && stats && workspace, "required pointer is null");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  unsigned *ord = static_cast<unsigned *>(workspace);  // the workspace's first region
  hipLaunchKernelGGL(stats_init, dim3(1), dim3(64), 0, stream, ord);
  RXMET_CHECK_LAUNCH();
  const int mf = calibrate_mfma<true>(T, B, I, H, W, R, bw, br, x, h0, h, v, workspace, stream);
  if (mf < 0) return mf;
  if (mf == 0) {
    const size_t lds = sizeof(float) * 8 * static_cast<size_t>(H);
    if (lds > 64 * 1024)
      RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&calib_forward<true>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          static_cast<int>(lds)));
    rxmet::prof::Scope ps__("gru_calibrate_forward", stream);
    hipLaunchKernelGGL(calib_forward<true>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I, H, W, R, bw,
                       br, x, h0, h, v, ord);
  }
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(stats_merge, dim3(1), dim3(64), 0, stream, ord, stats);
  RXMET_CHECK_LAUNCH();
  const CalWorkspace cw(T, B, I, H);
  float *prm = reinterpret_cast<float *>(static_cast<char *>(workspace) + cw.prm);
  hipLaunchKernelGGL(calib_params_part, dim3((3 * H + 63) / 64, cw.prm_slabs), dim3(256), 0,
                     stream, I, H, W, R, prm);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(calib_params_fold, dim3((3 * H + 255) / 256), dim3(256), 0, stream, H,
                     cw.prm_slabs, prm, bw, br, stats + 2 * kNStat);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_gru_forward_fp(int32_t is_training, int32_t T, int32_t B, int32_t I, int32_t H,
                         const float *W, const float *R, const float *bw, const float *br,
                         const float *x, const float *h0, float *h, float *v, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 4096, "hidden_size above 4096 is not supported by the float forward");
  RXMET_CHECK_ARG(W && R && bw && br && x && h, "required pointer is null");
  RXMET_CHECK_ARG(!is_training || v, "v is required when is_training is set");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const size_t lds = sizeof(float) * 8 * static_cast<size_t>(H);
  if (lds > 64 * 1024)
    RXMET_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&calib_forward<false>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
  hipLaunchKernelGGL(calib_forward<false>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I, H, W,
                     R, bw, br, x, h0, h, is_training ? v : nullptr, nullptr);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // extern "C"
