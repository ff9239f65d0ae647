// lstm_calib.hip — float LSTM forward with MinMax statistics (PTQ calibration pass) and the
// plain float forward, behind rxmet_lstm_forward_calibrate / rxmet_lstm_forward_float.
//
// Reference: CalibrationSession.collect -> LstmCalibrationCollector::collect
// (src/lstm/calibration.cc:154-240) over lstmForwardFloatCpu (src/lstm/forward_float_cpu.cc:
// 57-153); the CUDA session runs the same observation set on device traces
// (src/lstm/calibration_cuda.cu:372-480).  Main form (H a multiple of 16 up to 512): the
// input projection on fp32 MFMA (calib_gemm.h) and a clustered recurrence with W_hh resident
// in VGPRs.  Fallback (other H): one workgroup per sequence keeps h and c in LDS and walks
// the T steps with the reference's summation order (bias first, then the products in index
// order).  In both, exp and tanh are evaluated in double and rounded once to float.
// Observed: x, h (h0 or zeros, then every h_t), c (c0 or zeros, then every c_t), both
// linears, the four gate inputs and outputs, tanh(c), and per-channel parameter ranges.
// Non-finite values are counted (the reference rejects them) instead of entering a range.
#include <algorithm>
#include <cfloat>
#include <cstdlib>

#include "calib_gemm.h"
#include "cluster.h"
#include "mfma_frag.h"
#include "rxmet_common.h"
#include "rxmet_lstm.h"

namespace rxmet {
namespace lstm {

constexpr int kCalThreads = 256;
constexpr int kN = RXMET_LSTM_NOPS;

__device__ __forceinline__ unsigned f2ord(float f) {
  const unsigned u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(unsigned u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

struct Obs {
  float mn[kN], mx[kN];
  unsigned bad;
};

__device__ __forceinline__ void observe(Obs &o, int op, float v) {
  if (isfinite(v)) {
    o.mn[op] = fminf(o.mn[op], v);
    o.mx[op] = fmaxf(o.mx[op], v);
  } else {
    ++o.bad;
  }
}

__device__ __forceinline__ float sigm(float x) {
  if (x >= 0.0f) {
    const float e = static_cast<float>(exp(-static_cast<double>(x)));
    return 1.0f / (1.0f + e);
  }
  const float e = static_cast<float>(exp(static_cast<double>(x)));
  return e / (1.0f + e);
}
__device__ __forceinline__ float tnh(float x) { return static_cast<float>(tanh(static_cast<double>(x))); }

template <bool STATS>
__global__ __launch_bounds__(kCalThreads) void lstm_float_forward(
    int T, int B, int I, int H, const float *__restrict__ Wi, const float *__restrict__ Wh,
    const float *__restrict__ bi, const float *__restrict__ bh, const float *__restrict__ x,
    const float *__restrict__ h0, const float *__restrict__ c0, float *__restrict__ out,
    float *__restrict__ hn, float *__restrict__ cn, unsigned *__restrict__ gstat /* 2*kN + 1 */) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int C = 4 * H;
  float *hs = reinterpret_cast<float *>(smem);  // [H]
  float *cs = hs + H;                           // [H]
  float *gates = cs + H;                        // [4H]
  __shared__ unsigned smin[kN], smax[kN], sbad;
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid < kN) {
    smin[tid] = f2ord(INFINITY);
    smax[tid] = f2ord(-INFINITY);
  }
  if (tid == 0) sbad = 0;
  Obs o;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    o.mn[i] = INFINITY;
    o.mx[i] = -INFINITY;
  }
  o.bad = 0;
  for (int j = tid; j < H; j += kCalThreads) {
    const size_t s = static_cast<size_t>(b) * H + j;
    hs[j] = h0 ? h0[s] : 0.0f;
    cs[j] = c0 ? c0[s] : 0.0f;
    if (STATS) {
      observe(o, RXMET_LSTM_OUTPUT, hs[j]);
      observe(o, RXMET_LSTM_CELL_STATE, cs[j]);
    }
  }
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const float *xt = x + (static_cast<size_t>(t) * B + b) * I;
    if (STATS)
      for (int k = tid; k < I; k += kCalThreads) observe(o, RXMET_LSTM_INPUT, xt[k]);
    for (int c = tid; c < C; c += kCalThreads) {
      float li = bi ? bi[c] : 0.0f, lh = bh ? bh[c] : 0.0f;
      const float *wi = Wi + static_cast<size_t>(c) * I, *wh = Wh + static_cast<size_t>(c) * H;
      for (int k = 0; k < I; ++k) li += wi[k] * xt[k];
      for (int k = 0; k < H; ++k) lh += wh[k] * hs[k];
      const float gsum = li + lh;
      gates[c] = gsum;
      if (STATS) {
        observe(o, RXMET_LSTM_IH_LINEAR, li);
        observe(o, RXMET_LSTM_HH_LINEAR, lh);
        observe(o, RXMET_LSTM_I_GATE_IN + c / H, gsum);
      }
    }
    __syncthreads();
    for (int j = tid; j < H; j += kCalThreads) {
      const float ig = sigm(gates[j]), fg = sigm(gates[H + j]);
      const float gg = tnh(gates[2 * H + j]), og = sigm(gates[3 * H + j]);
      const float cnew = fg * cs[j] + ig * gg;
      const float ct = tnh(cnew);
      const float hv = og * ct;
      cs[j] = cnew;
      hs[j] = hv;  // every gate of this step is already in `gates`
      out[(static_cast<size_t>(t) * B + b) * H + j] = hv;
      if (STATS) {
        observe(o, RXMET_LSTM_I_GATE_OUT, ig);
        observe(o, RXMET_LSTM_F_GATE_OUT, fg);
        observe(o, RXMET_LSTM_G_GATE_OUT, gg);
        observe(o, RXMET_LSTM_O_GATE_OUT, og);
        observe(o, RXMET_LSTM_CELL_STATE, cnew);
        observe(o, RXMET_LSTM_CELL_TANH, ct);
        observe(o, RXMET_LSTM_OUTPUT, hv);
      }
    }
    __syncthreads();
  }
  for (int j = tid; j < H; j += kCalThreads) {
    const size_t s = static_cast<size_t>(b) * H + j;
    hn[s] = hs[j];
    cn[s] = cs[j];
  }
  if (!STATS) return;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    if (o.mn[i] <= o.mx[i]) {
      atomicMin(&smin[i], f2ord(o.mn[i]));
      atomicMax(&smax[i], f2ord(o.mx[i]));
    }
  }
  if (o.bad) atomicAdd(&sbad, o.bad);
  __syncthreads();
  if (tid < kN) {
    atomicMin(&gstat[tid], smin[tid]);
    atomicMax(&gstat[kN + tid], smax[tid]);
  }
  if (tid == 0 && sbad) atomicAdd(&gstat[2 * kN], sbad);
}

__global__ void lstm_stats_init(unsigned *o) {
  const int i = threadIdx.x;
  if (i < kN) {
    o[i] = f2ord(INFINITY);
    o[kN + i] = f2ord(-INFINITY);
  }
  if (i == 0) o[2 * kN] = 0u;
}

__global__ void lstm_stats_merge(const unsigned *o, float *s, int64_t count_index) {
  const int i = threadIdx.x;
  if (i < kN) {
    const float lo = ord2f(o[i]), hi = ord2f(o[kN + i]);
    s[i] = fminf(s[i], lo);
    s[kN + i] = fmaxf(s[kN + i], hi);
  }
  if (i == 0) s[count_index] += static_cast<float>(o[2 * kN]);
}

// ---------------------------------------------------------------------------------
// MFMA form (H a multiple of 16, H <= 512): the input linear of every step as one fp32 MFMA
// GEMM, then the recurrence as a clustered persistent kernel with W_hh resident in VGPRs
// (the GRU calibration's structure, gru_calib.hip, with four gates and the cell state).  Sums
// are fp32 in another order than the per-sequence kernel's (bias first, products in index
// order); results agree to rounding.  Statistics: per-workgroup partials (min, max of the 18
// operators and the count of non-finite values) folded by one small kernel.
// ---------------------------------------------------------------------------------
constexpr int kCT = 16;
constexpr int kCMaxW = 8;  // waves of a recurrence workgroup (256 VGPRs: W_hh, h and the 18
                           // operators' statistics stay in registers)
constexpr int kPart = 2 * kN + 1;  // floats per partial block: min[18], max[18], non-finite

// The block's ranges of the first N statistics and its non-finite count as one partial block
// of 2 N + 1 floats: min[N], max[N], count.
template <int N = kN>
__device__ __forceinline__ void obs_block(const Obs &o, float *part) {
  __shared__ float smn[kCMaxW][N], smx[kCMaxW][N];
  __shared__ unsigned sbad;
  const int w = threadIdx.x / kWave, nw = blockDim.x / kWave;
  if (threadIdx.x == 0) sbad = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {  // unrolled: o stays in registers
    const float lo = wave_min(o.mn[i]), hi = wave_max(o.mx[i]);
    if (threadIdx.x % kWave == 0) {
      smn[w][i] = lo;
      smx[w][i] = hi;
    }
  }
  if (o.bad) atomicAdd(&sbad, o.bad);
  __syncthreads();
  if (threadIdx.x < N) {
    float lo = smn[0][threadIdx.x], hi = smx[0][threadIdx.x];
    for (int ww = 1; ww < nw; ++ww) {
      lo = fminf(lo, smn[ww][threadIdx.x]);
      hi = fmaxf(hi, smx[ww][threadIdx.x]);
    }
    part[threadIdx.x] = lo;
    part[N + threadIdx.x] = hi;
  }
  if (threadIdx.x == 0) part[2 * N] = static_cast<float>(sbad);  // exact: far below 2^24
}

__device__ __forceinline__ void obs_init(Obs &o) {
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    o.mn[i] = INFINITY;
    o.mx[i] = -INFINITY;
  }
  o.bad = 0;
}

// P partial blocks of the first N statistics (obs_block<N>) folded into this call's ordered
// ranges and count.  Each thread takes whole partial blocks, all of a block's loads issued
// together: one load latency per 256 blocks rather than one per statistic and block.
template <int N>
__global__ __launch_bounds__(256) void lstm_stats_fold(const float *__restrict__ part, int P,
                                                       unsigned *__restrict__ ostat) {
  __shared__ float smn[4][N], smx[4][N];
  __shared__ unsigned sbad;
  const int w = threadIdx.x / kWave;
  if (threadIdx.x == 0) sbad = 0;
  __syncthreads();
  float lo[N], hi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    lo[i] = INFINITY;
    hi[i] = -INFINITY;
  }
  unsigned bad = 0;
  for (int p = threadIdx.x; p < P; p += blockDim.x) {
    const float *q = part + static_cast<size_t>(p) * (2 * N + 1);
    float v[2 * N + 1];
#pragma unroll
    for (int i = 0; i < 2 * N + 1; ++i) v[i] = q[i];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      lo[i] = fminf(lo[i], v[i]);
      hi[i] = fmaxf(hi[i], v[N + i]);
    }
    bad += static_cast<unsigned>(v[2 * N]);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float a = wave_min(lo[i]), b = wave_max(hi[i]);
    if (threadIdx.x % kWave == 0) {
      smn[w][i] = a;
      smx[w][i] = b;
    }
  }
  if (bad) atomicAdd(&sbad, bad);
  __syncthreads();
  if (threadIdx.x < N) {
    float a = smn[0][threadIdx.x], b = smx[0][threadIdx.x];
    for (int ww = 1; ww < 4; ++ww) {
      a = fminf(a, smn[ww][threadIdx.x]);
      b = fmaxf(b, smx[ww][threadIdx.x]);
    }
    if (a <= b) {  // one thread per operator: no contention
      atomicMin(&ostat[threadIdx.x], f2ord(a));
      atomicMax(&ostat[kN + threadIdx.x], f2ord(b));
    }
  }
  if (threadIdx.x == 0 && sbad) atomicAdd(&ostat[2 * kN], sbad);
}

// The statistics the input GEMM observes, the input and the input linear, lie among the first
// kGemmStat operators.
constexpr int kGemmStat = RXMET_LSTM_IH_LINEAR + 1;
static_assert(RXMET_LSTM_INPUT < kGemmStat, "GEMM statistics layout");

// li[m][c] = sum_k x[m][k] W_ih[c][k] + b_ih[c] for m < M = T B, c < C = 4H (W_ih [4H][I],
// N-major), with the INPUT and IH_LINEAR statistics: the LDS-tiled fp32 MFMA block of
// calib_gemm.h, one partial block of statistics per workgroup.
template <bool STATS>
__global__ __launch_bounds__(256) void lstm_input_gemm(int M, int K, int C,
                                                       const float *__restrict__ x,
                                                       const float *__restrict__ Wi,
                                                       const float *__restrict__ bi,
                                                       float *__restrict__ li,
                                                       float *__restrict__ part) {
  Obs o;
  obs_init(o);
  calgemm::gemm_block<false>(
      M, C, K, x, Wi, bi, li, STATS && blockIdx.x == 0,
      [&](float v) {
        if (STATS) observe(o, RXMET_LSTM_INPUT, v);
      },
      [&](float v) {
        if (STATS) observe(o, RXMET_LSTM_IH_LINEAR, v);
      });
  if (STATS)
    obs_block<kGemmStat>(o, part + (static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x) *
                                       (2 * kGemmStat + 1));
}

struct LCalArgs {
  int T, B, H, NC, NWG, ntiles, Bpad, Hpad, G, ncl;
  const float *li;   // [T, B, 4H] input linear with b_ih
  const float *Wh;   // [4H, H]
  const float *bh;   // [4H] or null
  const float *h0, *c0;  // [B, H] or null
  float *out, *hn, *cn;  // [T, B, H], [B, H], [B, H]
  float *hx;         // [2][Bpad][Hpad] exchanged h (padding columns zero)
  float *part;       // [ncl G][kPart] partial statistics, or null
  unsigned *counters;
  int *timeout;
  unsigned spin_limit;
};

// The GRU calibration recurrence's scheme with four gates: items (k chunk, gate) of sixteen
// MFMAs dealt to the NWG waves, W_hh fragments resident, the tile's 256 (row, unit) elements
// finished one per thread with h and c kept in registers.
template <bool STATS, int IPW>
__global__ __launch_bounds__(64 * kCMaxW) void lstm_calib_recurrence_cl(LCalArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  v4f *red = reinterpret_cast<v4f *>(smem);  // [4 NC][64]
  const cluster::Place pl = cluster::place(a.G, a.ncl);
  unsigned *counter = a.counters + cluster::kCounterStride * pl.cluster;
  const int H = a.H, C = 4 * H, B = a.B, NC = a.NC, NWG = a.NWG;
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave, r16 = l % 16, g = l / 16;
  const int u0 = 16 * pl.member;
  const int nitems = 4 * NC;
  float rfr[IPW][16];
#pragma unroll
  for (int it = 0; it < IPW; ++it) {
    const int item = w + it * NWG, ch = item / 4, gate = item % 4;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int k = 64 * ch + 16 * g + s;
      rfr[it][s] = item < nitems && k < H
                       ? a.Wh[static_cast<size_t>(gate * H + u0 + r16) * H + k] : 0.0f;
    }
  }
  const bool fin = tid < 256;
  const int fl = tid % 64, fq = tid / 64;
  const int frow = 4 * (fl / 16) + fq, fu = u0 + fl % 16;
  float bh4[4];
#pragma unroll
  for (int gate = 0; gate < 4; ++gate) bh4[gate] = fin && a.bh ? a.bh[gate * H + fu] : 0.0f;
  Obs o;
  obs_init(o);
  const unsigned plane = static_cast<unsigned>(a.Bpad) * a.Hpad;
  const auto xr = cluster::buffer_rsrc(a.hx, 2u * plane * 4u);
  unsigned *hxw = reinterpret_cast<unsigned *>(a.hx);
  unsigned epoch = 0;
  bool alive = true;
  for (int tile = pl.cluster; tile < a.ntiles && alive; tile += a.ncl) {
    __syncthreads();
    const int b = tile * kCT + frow;
    const bool valid = fin && b < B;
    float hold = 0.0f, cold = 0.0f;
    if (fin) {
      const size_t e = static_cast<size_t>(b) * H + fu;
      hold = valid && a.h0 ? a.h0[e] : 0.0f;
      cold = valid && a.c0 ? a.c0[e] : 0.0f;
      cluster::store_coherent(hxw + b * a.Hpad + fu, __float_as_uint(hold));
      if (STATS && valid) {
        observe(o, RXMET_LSTM_OUTPUT, hold);
        observe(o, RXMET_LSTM_CELL_STATE, cold);
      }
    }
    float lin[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto load_li = [&](int t) {
      if (valid) {
        const float *lp = a.li + (static_cast<size_t>(t) * B + b) * C + fu;
#pragma unroll
        for (int gate = 0; gate < 4; ++gate) lin[gate] = lp[gate * H];
      }
    };
    load_li(0);
    alive = cluster::sync(counter, ++epoch * a.G, a.timeout, a.spin_limit);
    for (int t = 0; t < a.T && alive; ++t) {
      const int par = t & 1;
      const unsigned rowoff = par * plane + static_cast<unsigned>(tile * kCT + r16) * a.Hpad;
#pragma unroll
      for (int it = 0; it < IPW; ++it) {
        const int item = w + it * NWG;
        if (item >= nitems) break;
        const int ch = item / 4;
        float hv[16];
        const unsigned off = 4u * (rowoff + 64 * ch + 16 * g);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int4 v = cluster::load_coherent16(xr, off + 16u * q);
          hv[4 * q] = __int_as_float(v.x);
          hv[4 * q + 1] = __int_as_float(v.y);
          hv[4 * q + 2] = __int_as_float(v.z);
          hv[4 * q + 3] = __int_as_float(v.w);
        }
        v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; ++s) acc = mfma_f32(hv[s], rfr[it][s], acc);
        red[item * kWave + l] = acc;
      }
      __syncthreads();
      if (fin) {
        float lh[4] = {bh4[0], bh4[1], bh4[2], bh4[3]};
        for (int ch = 0; ch < NC; ++ch)
#pragma unroll
          for (int gate = 0; gate < 4; ++gate) lh[gate] += red[(ch * 4 + gate) * kWave + fl][fq];
        float gs[4];
#pragma unroll
        for (int gate = 0; gate < 4; ++gate) gs[gate] = lin[gate] + lh[gate];
        const float ig = sigm(gs[0]), fg = sigm(gs[1]), gg = tnh(gs[2]), og = sigm(gs[3]);
        const float cnew = fg * cold + ig * gg;
        const float ct = tnh(cnew);
        const float hv = og * ct;
        hold = hv;
        cold = cnew;
        cluster::store_coherent(hxw + (par ^ 1) * plane + b * a.Hpad + fu, __float_as_uint(hv));
        cluster::arrive(counter);
        ++epoch;
        if (valid) {
          if (STATS) {
#pragma unroll
            for (int gate = 0; gate < 4; ++gate) {
              observe(o, RXMET_LSTM_HH_LINEAR, lh[gate]);
              observe(o, RXMET_LSTM_I_GATE_IN + gate, gs[gate]);
            }
            observe(o, RXMET_LSTM_I_GATE_OUT, ig);
            observe(o, RXMET_LSTM_F_GATE_OUT, fg);
            observe(o, RXMET_LSTM_G_GATE_OUT, gg);
            observe(o, RXMET_LSTM_O_GATE_OUT, og);
            observe(o, RXMET_LSTM_CELL_STATE, cnew);
            observe(o, RXMET_LSTM_CELL_TANH, ct);
            observe(o, RXMET_LSTM_OUTPUT, hv);
          }
          a.out[(static_cast<size_t>(t) * B + b) * H + fu] = hv;
          if (t + 1 == a.T) {
            a.hn[static_cast<size_t>(b) * H + fu] = hv;
            a.cn[static_cast<size_t>(b) * H + fu] = cnew;
          }
        }
        if (t + 1 < a.T) load_li(t + 1);
      } else {
        cluster::arrive(counter);
        ++epoch;
      }
      alive = cluster::wait(counter, epoch * a.G, a.timeout, a.spin_limit);
    }
  }
  if (STATS) {
    __syncthreads();
    obs_block(o, a.part + static_cast<size_t>(blockIdx.x) * kPart);
  }
}

struct LCalWorkspace {
  size_t ord, li, hx, part, sync, total;
  int Bpad, Hpad, ntiles;
  LCalWorkspace(int T, int B, int H) {
    auto al = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    ntiles = (B + kCT - 1) / kCT;
    Bpad = ntiles * kCT;
    Hpad = (H + 63) / 64 * 64;
    const int64_t M = static_cast<int64_t>(T) * B;
    const int64_t gemm_blocks = (4 * static_cast<int64_t>(H) + 63) / 64 * ((M + 63) / 64);
    const int64_t rec_blocks = static_cast<int64_t>(ntiles) * (H / 16 > 0 ? H / 16 : 1);
    const int64_t nparts = kPart * std::max(gemm_blocks, rec_blocks);
    size_t o = 0;
    ord = o; o += al(sizeof(unsigned) * (2 * kN + 1));
    li = o; o += al(sizeof(float) * static_cast<size_t>(T) * B * 4 * H);
    hx = o; o += al(sizeof(float) * 2 * static_cast<size_t>(Bpad) * Hpad);
    part = o; o += al(sizeof(float) * static_cast<size_t>(nparts));
    sync = o; o += al(sizeof(unsigned) * cluster::kCounterStride * (ntiles + 2));
    total = o;
  }
};

// The MFMA form when it applies; 1 when launched, 0 when the caller must use the
// per-sequence kernel.
template <bool STATS>
static int lstm_float_mfma(int T, int B, int I, int H, const float *Wi, const float *Wh,
                           const float *bi, const float *bh, const float *x, const float *h0,
                           const float *c0, float *out, float *hn, float *cn, void *workspace,
                           hipStream_t stream) {
  if (workspace == nullptr || H % 16 != 0 || H > 512 || std::getenv("RXMET_NO_CLUSTER") != nullptr)
    return 0;
  const LCalWorkspace ws(T, B, H);
  if (2.0 * ws.Bpad * ws.Hpad * 4 >= 2147483648.0) return 0;
  LCalArgs a{};
  a.T = T; a.B = B; a.H = H;
  a.NC = (H + 63) / 64;
  a.NWG = std::min(kCMaxW, std::max(4, 4 * a.NC));
  const int ipw = (4 * a.NC + a.NWG - 1) / a.NWG;  // 1 (H <= 128) .. 4 (H <= 512)
  if (ipw > 4) return 0;  // H above 512: more W_hh fragments than the registers hold
  a.ntiles = ws.ntiles; a.Bpad = ws.Bpad; a.Hpad = ws.Hpad;
  a.G = H / 16;
  const void *fn = ipw == 1 ? reinterpret_cast<const void *>(&lstm_calib_recurrence_cl<STATS, 1>)
                 : ipw == 2 ? reinterpret_cast<const void *>(&lstm_calib_recurrence_cl<STATS, 2>)
                 : ipw == 3 ? reinterpret_cast<const void *>(&lstm_calib_recurrence_cl<STATS, 3>)
                            : reinterpret_cast<const void *>(&lstm_calib_recurrence_cl<STATS, 4>);
  const size_t lds = sizeof(v4f) * kWave * 4 * static_cast<size_t>(a.NC);
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
  char *wsb = static_cast<char *>(workspace);
  unsigned *ord = reinterpret_cast<unsigned *>(wsb + ws.ord);
  float *li = reinterpret_cast<float *>(wsb + ws.li);
  float *part = reinterpret_cast<float *>(wsb + ws.part);
  a.hx = reinterpret_cast<float *>(wsb + ws.hx);
  a.counters = reinterpret_cast<unsigned *>(wsb + ws.sync);
  a.timeout = reinterpret_cast<int *>(a.counters + cluster::kCounterStride * ncl);
  a.spin_limit = cluster::spin_limit();
  const int C = 4 * H, M = T * B;
  {
    rxmet::prof::Scope ps__("lstm_calibrate_input_gemm", stream);
    const dim3 grid(static_cast<unsigned>((C + calgemm::kBN - 1) / calgemm::kBN),
                    static_cast<unsigned>((M + calgemm::kBM - 1) / calgemm::kBM));
    hipLaunchKernelGGL(lstm_input_gemm<STATS>, grid, dim3(256), 0, stream, M, I, C, x, Wi, bi,
                       li, part);
    RXMET_CHECK_LAUNCH();
    if (STATS) {
      hipLaunchKernelGGL(lstm_stats_fold<kGemmStat>, dim3(1), dim3(256), 0, stream, part,
                         static_cast<int>(grid.x * grid.y), ord);
      RXMET_CHECK_LAUNCH();
    }
  }
  hipLaunchKernelGGL(cluster::zero_words, dim3(cluster::zero_blocks(2 * ws.Bpad * ws.Hpad)),
                     dim3(256), 0, stream, reinterpret_cast<unsigned *>(a.hx),
                     2 * ws.Bpad * ws.Hpad);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(cluster::zero_words, dim3(1), dim3(256), 0, stream, a.counters,
                     cluster::kCounterStride * ncl + 1);
  RXMET_CHECK_LAUNCH();
  a.li = li; a.Wh = Wh; a.bh = bh; a.h0 = h0; a.c0 = c0;
  a.out = out; a.hn = hn; a.cn = cn; a.part = part;
  void *args[] = {&a};
  {
    rxmet::prof::Scope ps__("lstm_calibrate_forward", stream);
    RXMET_CHECK_HIP(cluster::launch(fn, dim3(ncl * a.G), dim3(kWave * a.NWG), args,
                                    static_cast<unsigned>(lds), stream));
    if (STATS) {
      hipLaunchKernelGGL(lstm_stats_fold<kN>, dim3(1), dim3(256), 0, stream, part, ncl * a.G, ord);
      RXMET_CHECK_LAUNCH();
    }
  }
  cluster::PoisonList pl{};
  pl.p[pl.count] = out;
  pl.n[pl.count++] = static_cast<int64_t>(T) * B * H;
  pl.p[pl.count] = hn;
  pl.n[pl.count++] = static_cast<int64_t>(B) * H;
  pl.p[pl.count] = cn;
  pl.n[pl.count++] = static_cast<int64_t>(B) * H;
  hipLaunchKernelGGL(cluster::poison_list, dim3(256), dim3(256), 0, stream, a.timeout, pl);
  RXMET_CHECK_LAUNCH();
  return 1;
}

// Per-channel ranges of W_ih / W_hh rows and biases, merged into the running ranges; a
// non-finite parameter value is counted.
__global__ __launch_bounds__(64) void lstm_param_stats(int I, int H, const float *Wi,
                                                       const float *Wh, const float *bi,
                                                       const float *bh, float *chan,
                                                       unsigned *bad) {
  const int C = 4 * H;
  const int c = blockIdx.x, l = threadIdx.x;
  const float *src[4] = {Wi + static_cast<size_t>(c) * I, Wh + static_cast<size_t>(c) * H,
                         bi ? bi + c : nullptr, bh ? bh + c : nullptr};
  const int n[4] = {I, H, 1, 1};
  unsigned nb = 0;
  for (int k = 0; k < 4; ++k) {
    if (!src[k]) continue;
    float lo = INFINITY, hi = -INFINITY;
    for (int e = l; e < n[k]; e += 64) {
      const float v = src[k][e];
      if (isfinite(v)) {
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      } else {
        ++nb;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, off, 64));
      hi = fmaxf(hi, __shfl_xor(hi, off, 64));
    }
    if (l == 0) {
      float *mn = chan + static_cast<size_t>(k) * 2 * C, *mx = mn + C;
      mn[c] = fminf(mn[c], lo);
      mx[c] = fmaxf(mx[c], hi);
    }
  }
  if (nb) atomicAdd(bad, nb);
}

}  // namespace lstm
}  // namespace rxmet

using namespace rxmet;
using namespace rxmet::lstm;

extern "C" {

int64_t rxmet_lstm_calibrate_workspace_bytes(int32_t T, int32_t B, int32_t I, int32_t H) {
  (void)I;
  if (T < 1 || B < 1 || H < 1) return static_cast<int64_t>(sizeof(unsigned) * (2 * kN + 1));
  return static_cast<int64_t>(LCalWorkspace(T, B, H).total);
}

static int launch_float(bool stats, int T, int B, int I, int H, const float *Wi, const float *Wh,
                        const float *bi, const float *bh, const float *x, const float *h0,
                        const float *c0, float *out, float *hn, float *cn, unsigned *ord,
                        hipStream_t stream) {
  const size_t lds = sizeof(float) * 6 * static_cast<size_t>(H);
  const void *fn = stats ? reinterpret_cast<const void *>(&lstm_float_forward<true>)
                         : reinterpret_cast<const void *>(&lstm_float_forward<false>);
  if (lds > 64 * 1024)
    RXMET_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
  if (stats)
    hipLaunchKernelGGL(lstm_float_forward<true>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I,
                       H, Wi, Wh, bi, bh, x, h0, c0, out, hn, cn, ord);
  else
    hipLaunchKernelGGL(lstm_float_forward<false>, dim3(B), dim3(kCalThreads), lds, stream, T, B, I,
                       H, Wi, Wh, bi, bh, x, h0, c0, out, hn, cn, ord);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_lstm_forward_calibrate(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                                 const float *W_hh, const float *b_ih, const float *b_hh,
                                 const float *x, const float *h0, const float *c0,
                                 float *output, float *h_n, float *c_n, float *stats,
                                 void *workspace, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 8192, "hidden_size above 8192 is not supported by the calibration pass");
  RXMET_CHECK_ARG(W_ih && W_hh && x && output && h_n && c_n && stats && workspace,
                  "required pointer is null");
  RXMET_CHECK_ARG((h0 == nullptr) == (c0 == nullptr), "h0 and c0 must be given together");
  RXMET_CHECK_ARG((b_ih == nullptr) == (b_hh == nullptr), "b_ih and b_hh must be given together");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  unsigned *ord = static_cast<unsigned *>(workspace);
  hipLaunchKernelGGL(lstm_stats_init, dim3(1), dim3(64), 0, stream, ord);
  RXMET_CHECK_LAUNCH();
  const int mf = lstm_float_mfma<true>(T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, output,
                                       h_n, c_n, workspace, stream);
  if (mf < 0) return mf;
  if (mf == 0) {
    rxmet::prof::Scope ps__("lstm_calibrate_forward", stream);
    if (int rc = launch_float(true, T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, output, h_n, c_n,
                              ord, stream))
      return rc;
  }
  hipLaunchKernelGGL(lstm_param_stats, dim3(4 * H), dim3(64), 0, stream, I, H, W_ih, W_hh, b_ih,
                     b_hh, stats + 2 * kN, ord + 2 * kN);
  RXMET_CHECK_LAUNCH();
  hipLaunchKernelGGL(lstm_stats_merge, dim3(1), dim3(64), 0, stream, ord, stats,
                     rxmet_lstm_stats_size(H) - 1);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int rxmet_lstm_forward_float(int32_t T, int32_t B, int32_t I, int32_t H, const float *W_ih,
                             const float *W_hh, const float *b_ih, const float *b_hh,
                             const float *x, const float *h0, const float *c0, float *output,
                             float *h_n, float *c_n, void *stream_) {
  clear_error();
  RXMET_CHECK_ARG(T >= 1 && B >= 1 && I >= 1 && H >= 1, "dimensions must be positive");
  RXMET_CHECK_ARG(H <= 8192, "hidden_size above 8192 is not supported by the float forward");
  RXMET_CHECK_ARG(W_ih && W_hh && x && output && h_n && c_n, "required pointer is null");
  RXMET_CHECK_ARG((h0 == nullptr) == (c0 == nullptr), "h0 and c0 must be given together");
  RXMET_CHECK_ARG((b_ih == nullptr) == (b_hh == nullptr), "b_ih and b_hh must be given together");
  return launch_float(false, T, B, I, H, W_ih, W_hh, b_ih, b_hh, x, h0, c0, output, h_n, c_n,
                      nullptr, static_cast<hipStream_t>(stream_));
}

}  // extern "C"
