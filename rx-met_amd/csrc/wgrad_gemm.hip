// wgrad_gemm.hip — see wgrad_gemm.h.
#include "wgrad_gemm.h"

#include "mfma_frag.h"
#include "rxmet_common.h"

namespace rxmet {
namespace wgrad {

constexpr int kKC = 32;         // K per chunk: one v_mfma_f32_16x16x32_bf16
constexpr int kRow = kKC + 8;   // LDS row in bf16 (80 bytes: 16-byte reads without conflicts)

// a = hi + mid + lo exactly: each term is the RNE bf16 of what the previous ones leave (the
// differences are exact in fp32).  Non-finite inputs give non-finite terms.
__device__ __forceinline__ void split3(float a, __bf16 &hi, __bf16 &mid, __bf16 &lo) {
  hi = static_cast<__bf16>(a);
  const float r1 = a - static_cast<float>(hi);
  mid = static_cast<__bf16>(r1);
  const float r2 = r1 - static_cast<float>(mid);
  lo = static_cast<__bf16>(r2);
}

// ---------------------------------------------------------------------------------
// TN: part[s][p][q] = sum_k A[k][p] Bt[q][k].  256 threads as 2 x 2 waves, each wave a
// (16 WI) x (16 WJ) tile, so the block tile is BP = 32 WI by BQ = 32 WJ.  K runs in chunks of
// 32 staged in LDS (A split into three bf16 planes on the way); the next chunk's global loads
// are issued before the current chunk's MFMAs.
// ---------------------------------------------------------------------------------
template <int NPL, int WI, int WJ>
__global__ __launch_bounds__(256) void tn_kernel(TnArgs a, int ntp, int ntq, int ngroups) {
  constexpr int BP = 32 * WI, BQ = 32 * WJ;
  constexpr int ATH = 256 / BP;     // threads per A column (k groups of 8 dealt round robin)
  constexpr int AG = 4 / ATH;       // k groups of 8 per thread
  constexpr int BCH = BQ / 64;      // B rows per thread (4 chunks of 16 bytes per row)
  __shared__ __align__(16) __bf16 As[3][BP][kRow];
  __shared__ __align__(16) __bf16 Bs[NPL][BQ][kRow];
  // blocks 8 r + x run on XCD x; the ntq q-tiles of one (p-tile, split) group are consecutive
  // blocks of one XCD, so they share the group's A rows in that XCD's L2
  const int xcd = blockIdx.x % 8, r8 = blockIdx.x / 8;
  const int qt = r8 % ntq, grp = (r8 / ntq) * 8 + xcd;
  if (grp >= ngroups) return;
  const int pt = grp % ntp, s = grp / ntp;
  const int p0 = BP * pt, q0 = BQ * qt;
  const int kbeg = s * a.kper;
  const int kend = min(a.K, kbeg + a.kper);
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int wm = w / 2, wn = w % 2;

  // staging roles: A column sp with k groups sg + ATH g; B rows bq + 64 h, 16-byte chunk bc
  const int sp = tid % BP, sg = tid / BP;
  const bool pin = p0 + sp < a.P;
  const float *ap = a.A + (p0 + sp);
  const int bq = tid / 4, bc = tid % 4;
  bool qin[BCH];
  const __bf16 *bp[BCH];
#pragma unroll
  for (int h = 0; h < BCH; ++h) {
    qin[h] = q0 + bq + 64 * h < a.Q;
    // rows past Q read row 0 and are replaced by zeros (value select, not pointer select)
    bp[h] = a.Bt + static_cast<int64_t>(qin[h] ? q0 + bq + 64 * h : 0) * a.ldb + 8 * bc;
  }
  const bool want_sum = a.colsum != nullptr && qt == 0;

  float av[AG][8];
  int4 bv[NPL][BCH];
#define RXMET_TN_LOAD(K0)                                                                     \
  {                                                                                           \
    _Pragma("unroll") for (int gi = 0; gi < AG; ++gi)                                         \
    _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                           \
      const int k = (K0) + 8 * (sg + ATH * gi) + j;                                           \
      av[gi][j] = (pin && k < kend) ? ap[static_cast<int64_t>(k) * a.lda] : 0.0f;             \
    }                                                                                         \
    _Pragma("unroll") for (int pl = 0; pl < NPL; ++pl)                                        \
    _Pragma("unroll") for (int h = 0; h < BCH; ++h) {                                         \
      const int4 t = *reinterpret_cast<const int4 *>(bp[h] + pl * a.bplane + (K0));           \
      bv[pl][h] = qin[h] ? t : make_int4(0, 0, 0, 0);                                         \
    }                                                                                         \
  }

  v4f acc[WI][WJ];
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < WJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  float csum = 0.0f;

  if (kbeg < kend) RXMET_TN_LOAD(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += kKC) {
    __syncthreads();  // the previous chunk's fragments are read
#pragma unroll
    for (int gi = 0; gi < AG; ++gi) {
      v8bf h, m, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __bf16 x, y, z;
        split3(av[gi][j], x, y, z);
        h[j] = x; m[j] = y; lo[j] = z;
        if (want_sum) csum += av[gi][j];
      }
      const int kk = 8 * (sg + ATH * gi);
      *reinterpret_cast<v8bf *>(&As[0][sp][kk]) = h;
      *reinterpret_cast<v8bf *>(&As[1][sp][kk]) = m;
      *reinterpret_cast<v8bf *>(&As[2][sp][kk]) = lo;
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int h = 0; h < BCH; ++h)
        *reinterpret_cast<int4 *>(&Bs[pl][bq + 64 * h][8 * bc]) = bv[pl][h];
    __syncthreads();
    if (k0 + kKC < kend) RXMET_TN_LOAD(k0 + kKC);
    v8bf bf[NPL][WJ];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int j = 0; j < WJ; ++j)
        bf[pl][j] = *reinterpret_cast<const v8bf *>(&Bs[pl][16 * (WJ * wn + j) + l % 16][8 * (l / 16)]);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      v8bf af[3];
#pragma unroll
      for (int c = 0; c < 3; ++c)
        af[c] = *reinterpret_cast<const v8bf *>(&As[c][16 * (WI * wm + i) + l % 16][8 * (l / 16)]);
#pragma unroll
      for (int j = 0; j < WJ; ++j)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) {
          // small terms first
          acc[i][j] = mfma_bf16(af[2], bf[pl][j], acc[i][j]);
          acc[i][j] = mfma_bf16(af[1], bf[pl][j], acc[i][j]);
          acc[i][j] = mfma_bf16(af[0], bf[pl][j], acc[i][j]);
        }
    }
  }
#undef RXMET_TN_LOAD
  if (want_sum && pin) a.colsum[(static_cast<int64_t>(s) * ATH + sg) * a.P + p0 + sp] = csum;
  float *part = a.part + static_cast<int64_t>(s) * a.P * a.Q;
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
      const int q = q0 + 16 * (WJ * wn + j) + l % 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = p0 + 16 * (WI * wm + i) + 4 * (l / 16) + r;
        if (p < a.P && q < a.Q) part[static_cast<int64_t>(p) * a.Q + q] = acc[i][j][r];
      }
    }
}

// ---------------------------------------------------------------------------------
// NT: out[m][n] = sum_k (A[m][k] kscale[k]) Bt[n][k]; 128 x (32 WJ) tile, 256 threads (2 x 2
// waves of 64 x 16 WJ), K in chunks of 32.
// ---------------------------------------------------------------------------------
template <int NPL, int WJ>
__global__ __launch_bounds__(256) void nt_kernel(NtArgs a) {
  constexpr int BN = 32 * WJ, BCH = (4 * BN + 255) / 256;  // B 16-byte chunks per thread
  __shared__ __align__(16) __bf16 As[3][128][kRow];
  __shared__ __align__(16) __bf16 Bs[NPL][BN][kRow];
  const int m0 = 128 * blockIdx.x, n0 = BN * blockIdx.y;
  // K split blockIdx.z: k in [kz, kz + K), written to out + blockIdx.z * out_split
  const int kz = blockIdx.z * a.kper, K = min(a.kper, a.K - kz);
  const float *ks = a.kscale + kz;
  float *out = a.out + blockIdx.z * a.out_split;
  const int tid = threadIdx.x, w = tid / 64, l = tid % 64;
  const int wm = w / 2, wn = w % 2;
  // staging roles: A row sm, 16 k at 16 sh; B row bn, chunk bc
  const int sm = tid / 2, sh = tid % 2;
  const bool min_ = m0 + sm < a.M;
  const float *ap = a.A + static_cast<int64_t>(m0 + sm) * a.lda + kz + 16 * sh;
  // B chunk e = tid + 256 h: row e / 4, 16-byte chunk e % 4 (rows past N read row 0, zeroed)
  bool bok[BCH], nin[BCH];
  const __bf16 *bp[BCH];
#pragma unroll
  for (int h = 0; h < BCH; ++h) {
    const int e = tid + 256 * h, bn = e / 4, bc = e % 4;
    bok[h] = e < 4 * BN;
    nin[h] = bok[h] && n0 + bn < a.N;
    bp[h] = a.Bt + static_cast<int64_t>(nin[h] ? n0 + bn : 0) * a.ldb + kz + 8 * bc;
  }

  float4 av[4];
  float4 sv[4];
  int4 bv[NPL][BCH];
  auto load = [&](int k0) {
    const bool kin = k0 + 16 * sh < K;  // K is a multiple of 16
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      av[c] = (min_ && kin) ? *reinterpret_cast<const float4 *>(ap + k0 + 4 * c) : make_float4(0, 0, 0, 0);
      sv[c] = kin ? *reinterpret_cast<const float4 *>(ks + k0 + 16 * sh + 4 * c) : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int h = 0; h < BCH; ++h) {
        const int4 t = *reinterpret_cast<const int4 *>(bp[h] + pl * a.bplane + k0);
        bv[pl][h] = nin[h] ? t : make_int4(0, 0, 0, 0);
      }
  };

  v4f acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < WJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  load(0);
  for (int k0 = 0; k0 < K; k0 += kKC) {
    __syncthreads();
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      v8bf h, m, lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float4 x4 = av[2 * half + j / 4], s4 = sv[2 * half + j / 4];
        const float x = (j % 4 == 0 ? x4.x : j % 4 == 1 ? x4.y : j % 4 == 2 ? x4.z : x4.w);
        const float sc = (j % 4 == 0 ? s4.x : j % 4 == 1 ? s4.y : j % 4 == 2 ? s4.z : s4.w);
        __bf16 p, q, r;
        split3(x * sc, p, q, r);
        h[j] = p; m[j] = q; lo[j] = r;
      }
      const int kk = 16 * sh + 8 * half;
      *reinterpret_cast<v8bf *>(&As[0][sm][kk]) = h;
      *reinterpret_cast<v8bf *>(&As[1][sm][kk]) = m;
      *reinterpret_cast<v8bf *>(&As[2][sm][kk]) = lo;
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int h = 0; h < BCH; ++h) {
        const int e = tid + 256 * h;
        if (bok[h]) *reinterpret_cast<int4 *>(&Bs[pl][e / 4][8 * (e % 4)]) = bv[pl][h];
      }
    __syncthreads();
    if (k0 + kKC < K) load(k0 + kKC);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v8bf af[3];
#pragma unroll
      for (int c = 0; c < 3; ++c)
        af[c] = *reinterpret_cast<const v8bf *>(&As[c][64 * wm + 16 * i + l % 16][8 * (l / 16)]);
#pragma unroll
      for (int j = 0; j < WJ; ++j)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) {
          const v8bf bf = *reinterpret_cast<const v8bf *>(&Bs[pl][16 * (WJ * wn + j) + l % 16][8 * (l / 16)]);
          acc[i][j] = mfma_bf16(af[2], bf, acc[i][j]);
          acc[i][j] = mfma_bf16(af[1], bf, acc[i][j]);
          acc[i][j] = mfma_bf16(af[0], bf, acc[i][j]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
      const int n = n0 + 16 * (WJ * wn + j) + l % 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 64 * wm + 16 * i + 4 * (l / 16) + r;
        if (m < a.M && n < a.N) out[static_cast<int64_t>(m) * a.ldo + n] = acc[i][j][r];
      }
    }
}

__global__ __launch_bounds__(256) void tn_finish_kernel(const float *__restrict__ part, int S, int P,
                                                        int Q, const float *__restrict__ qscale,
                                                        float *__restrict__ out, int64_t ldo,
                                                        bool transpose, int ath,
                                                        const float *__restrict__ colsum,
                                                        float *__restrict__ bias,
                                                        const uint8_t *__restrict__ mask,
                                                        int swap_h) {
  const int64_t n = static_cast<int64_t>(P) * Q;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n + P; i += stride) {
    if (i < n) {
      float acc = part[i];
      for (int s = 1; s < S; ++s) acc += part[static_cast<int64_t>(s) * n + i];
      const int p = static_cast<int>(i / Q), q = static_cast<int>(i % Q);
      float v = qscale ? acc * qscale[q] : acc;
      if (mask) v *= static_cast<float>(mask[static_cast<int64_t>(q) * P + p]);
      int po = p;
      if (swap_h > 0) po = p < swap_h ? p + swap_h : (p < 2 * swap_h ? p - swap_h : p);
      if (transpose)
        out[q * ldo + po] = v;
      else
        out[po * ldo + q] = v;
    } else if (colsum && bias) {
      const int p = static_cast<int>(i - n);
      float acc = 0.0f;
      for (int s = 0; s < S * ath; ++s) acc += colsum[static_cast<int64_t>(s) * P + p];
      bias[p * ldo] = acc;
    }
  }
}

// Codes -> bf16 planes, transposed through a 64 x 64 LDS tile.
__global__ __launch_bounds__(256) void codes_t_kernel(const float *__restrict__ src0, int64_t rows0,
                                                      const float *__restrict__ src1, int64_t rows,
                                                      int cols, int64_t rs, int64_t cs, float zp,
                                                      float div, int nplanes,
                                                      __bf16 *__restrict__ dst, int64_t ldd,
                                                      int64_t plane) {
  __shared__ int tile[64][65];
  const int64_t r0 = 64 * static_cast<int64_t>(blockIdx.x);
  const int c0 = 64 * blockIdx.y;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int rr = e / 64, cc = e % 64;
    const int64_t r = r0 + rr;
    const int c = c0 + cc;
    int v = 0;
    if (r < rows && c < cols) {
      const float x = r < rows0 ? src0[r * rs + c * cs] : src1[(r - rows0) * rs + c * cs];
      v = static_cast<int>(rintf((x - zp) / div));
    }
    tile[cc][rr] = v;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int cc = e / 64, rr = e % 64;
    const int64_t r = r0 + rr;
    const int c = c0 + cc;
    if (c >= cols || r >= ldd) continue;
    const int v = tile[cc][rr];
    __bf16 *d = dst + static_cast<int64_t>(c) * ldd + r;
    if (nplanes == 1) {
      *d = static_cast<__bf16>(static_cast<float>(v));
    } else {
      const int hi = v >> 8;  // floor division: v = 256 hi + (v & 255)
      *d = static_cast<__bf16>(static_cast<float>(256 * hi));
      d[plane] = static_cast<__bf16>(static_cast<float>(v & 255));
    }
  }
}

int codes_t(const float *src0, int64_t rows0, const float *src1, int64_t rows, int cols, int64_t rs,
            int64_t cs, float zp, float div, int nplanes, __bf16 *dst, int64_t ldd, int64_t plane,
            hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(ldd >= rows && (rows0 >= rows || src1 != nullptr), "bad codes_t layout");
  const dim3 grid(static_cast<unsigned>((ldd + 63) / 64), static_cast<unsigned>((cols + 63) / 64));
  hipLaunchKernelGGL(codes_t_kernel, grid, dim3(256), 0, stream, src0, rows0, src1, rows, cols, rs,
                     cs, zp, div, nplanes, dst, ldd, plane);
  RXMET_CHECK_LAUNCH();
  return 0;
}

// Block tile of a TN product: wave tiles WI x WJ (of 16 x 16) chosen by the width Q.
struct TnTile {
  int wi, wj;
  int bp() const { return 32 * wi; }
  int bq() const { return 32 * wj; }
  int ath() const { return 256 / bp(); }
};
static TnTile tn_tile(int Q, int nplanes) {
  // two B planes: 128 x 128 at most, so that two waves fit each SIMD
  if (Q >= 256 && nplanes == 1) return {4, 8};
  if (Q <= 64) return {4, 2};
  return {4, 4};
}

void tn_plan(int K, int P, int Q, int nplanes, int *S, int *kper) {
  const TnTile t = tn_tile(Q, nplanes);
  const int tiles = ((P + t.bp() - 1) / t.bp()) * ((Q + t.bq() - 1) / t.bq());
  const int chunks = (K + kKC - 1) / kKC;
  // about 512 workgroups, each at least 32 chunks (fewer, larger partials)
  int s = (512 + tiles - 1) / tiles;
  if (s > chunks / 32) s = chunks / 32;
  if (s < 1) s = 1;
  const int per = (chunks + s - 1) / s;
  *kper = per * kKC;
  *S = (K + *kper - 1) / *kper;
}

template <int WI, int WJ>
static void tn_launch(const TnArgs &a, int nplanes, hipStream_t stream) {
  const int ntp = (a.P + 32 * WI - 1) / (32 * WI), ntq = (a.Q + 32 * WJ - 1) / (32 * WJ);
  const int ngroups = ntp * a.S, padded = (ngroups + 7) / 8 * 8;
  const dim3 grid(static_cast<unsigned>(padded * ntq));
  if (nplanes == 1)
    hipLaunchKernelGGL((tn_kernel<1, WI, WJ>), grid, dim3(256), 0, stream, a, ntp, ntq, ngroups);
  else
    hipLaunchKernelGGL((tn_kernel<2, WI, WJ>), grid, dim3(256), 0, stream, a, ntp, ntq, ngroups);
}

int tn(const TnArgs &a, int nplanes, hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(a.kper % kKC == 0 && a.ldb % 8 == 0, "bad TN layout");
  const TnTile t = tn_tile(a.Q, nplanes);
  if (t.wj == 8)
    tn_launch<4, 8>(a, nplanes, stream);
  else if (t.wj == 2)
    tn_launch<4, 2>(a, nplanes, stream);
  else
    tn_launch<4, 4>(a, nplanes, stream);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int nt(const NtArgs &a, int nplanes, hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(a.K % 16 == 0 && a.lda % 4 == 0 && a.ldb % 8 == 0, "bad NT layout");
  // B is read in whole 32-wide K chunks: its rows must hold zeros up to a multiple of 32
  RXMET_CHECK_ARG(a.ldb >= (a.K + 31) / 32 * 32, "NT B rows must be padded to a multiple of 32");
  RXMET_CHECK_ARG(a.ksplit >= 1 && (a.ksplit == 1 || (a.kper % 32 == 0 && a.kper * (a.ksplit - 1) < a.K)),
                  "bad NT K split");
  // one column tile when N <= 128 (64, 96 or 128 wide), else tiles of 128
  const int wj = a.N <= 64 ? 2 : a.N <= 96 ? 3 : 4;
  const dim3 grid((a.M + 127) / 128, (a.N + 32 * wj - 1) / (32 * wj), a.ksplit);
  NtArgs b = a;
  if (b.ksplit == 1) b.kper = b.K;
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, b); };
  if (nplanes == 1)
    wj == 2 ? go(nt_kernel<1, 2>) : wj == 3 ? go(nt_kernel<1, 3>) : go(nt_kernel<1, 4>);
  else
    wj == 2 ? go(nt_kernel<2, 2>) : wj == 3 ? go(nt_kernel<2, 3>) : go(nt_kernel<2, 4>);
  RXMET_CHECK_LAUNCH();
  return 0;
}

int tn_finish(const float *part, int S, int P, int Q, int nplanes, const float *qscale, float *out,
              int64_t ldo, bool transpose, const float *colsum, float *bias, hipStream_t stream,
              const uint8_t *mask, int swap_h) {
  const int64_t n = static_cast<int64_t>(P) * Q + P;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(tn_finish_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     part, S, P, Q, qscale, out, ldo, transpose, tn_tile(Q, nplanes).ath(), colsum,
                     bias, mask, swap_h);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // namespace wgrad
}  // namespace rxmet
