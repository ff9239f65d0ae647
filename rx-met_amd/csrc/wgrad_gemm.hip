// wgrad_gemm.hip — see wgrad_gemm.h.
#include "wgrad_gemm.h"

#include <algorithm>
#include <type_traits>

#include "mfma_frag.h"
#include "rxmet_common.h"

namespace rxmet {
namespace wgrad {

constexpr int kKC = 32;  // K per chunk: one v_mfma_f32_16x16x32_bf16

// ---------------------------------------------------------------------------------
// Wave-tile kernels (products whose B side is at most 80 wide).  Each wave computes a
// 64 x 16 WJ output tile with its operands loaded from global memory straight into MFMA
// operand layout: no LDS and no barriers, so the waves sharing a SIMD overlap one another's
// loads, splits and MFMAs.  The narrow B side is re-read by every wave from L1/L2.  Operand lane (r, kb) =
// (l % 16, l / 16) holds k = 8 kb + j (j = 0..7) of a 32-wide chunk, for A and B alike.  Two
// register sets: the next chunk's loads are in flight during the current chunk's MFMAs.
// ---------------------------------------------------------------------------------

// One gradient fragment (8 values of one row) as three bf16 planes, multiplied into every B
// fragment of the wave (smallest terms first).
template <int NPL, int WJ>
__device__ __forceinline__ void mma_split3(const float (&v)[8], const v8bf (&bf)[NPL][WJ],
                                           v4f (&acc)[WJ]) {
  uint4 h, m, o;
  split3x8(v, h, m, o);
  const v8bf hi = __builtin_bit_cast(v8bf, h), mid = __builtin_bit_cast(v8bf, m),
             lo = __builtin_bit_cast(v8bf, o);
#pragma unroll
  for (int jt = 0; jt < WJ; ++jt)
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl) {
      acc[jt] = mfma_bf16(lo, bf[pl][jt], acc[jt]);
      acc[jt] = mfma_bf16(mid, bf[pl][jt], acc[jt]);
      acc[jt] = mfma_bf16(hi, bf[pl][jt], acc[jt]);
    }
}

__device__ __forceinline__ float lane4(const float4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Block -> (p-tile, q-tile, split) of a TN product.  The tiles of one split are dealt in groups
// of up to gt (a whole number of p-tiles, at most one XCD's worth of resident workgroups) and
// the groups go round robin over the eight XCDs (block b runs on XCD b % 8): a group's
// workgroups start together on one XCD and walk the same K rows, so each chunk of A and B is
// fetched from HBM once and served to the group from that XCD's L2.
struct TnMap {
  int ntq, tiles, gt, gps, ngroups;  // q-tiles, tiles per split, group size, groups per split, groups
};

__device__ __forceinline__ bool tn_place(const TnMap &m, int *pt, int *qt, int *s) {
  const int xcd = blockIdx.x % 8, i = blockIdx.x / 8;
  const int g = (i / m.gt) * 8 + xcd;
  if (g >= m.ngroups) return false;
  const int t = (g % m.gps) * m.gt + i % m.gt;
  if (t >= m.tiles) return false;
  *s = g / m.gps;
  *pt = t / m.ntq;
  *qt = t % m.ntq;
  return true;
}

// TN: part[s][p][q] = sum_k A[k][p] Bt[q][k].  The A loads are 16 bytes along p, so a lane's
// four values belong to four sub-tiles: row r of sub-tile i is column p = pw + 4 r + i.
// Workgroups of WM x WN waves (a BP x BQ tile), placed by tn_place.
template <int NPL, int WM, int WN, int WJ>
__global__ __launch_bounds__(64 * WM * WN, 2) void tn_wave_kernel(TnArgs a, TnMap map) {
  constexpr int BP = 64 * WM, BQ = 16 * WJ * WN;
  int pt, qt, s;
  if (!tn_place(map, &pt, &qt, &s)) return;
  const int kbeg = s * a.kper, kend = min(a.K, kbeg + a.kper);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64, r = l % 16, kb = l / 16;
  const int pw = BP * pt + 64 * (w / WN), qw = BQ * qt + 16 * WJ * (w % WN);
  if (pw >= a.P || qw >= a.Q) return;  // whole wave; nothing below synchronises
  // columns and B rows are clamped into the matrices: a clamped lane only feeds outputs
  // past P or Q, which are not stored
  const float *ab = a.A + min(pw + 4 * r, a.P - 4) + static_cast<int64_t>(8 * kb) * a.lda;
  const __bf16 *bb[WJ];
#pragma unroll
  for (int jt = 0; jt < WJ; ++jt)
    bb[jt] = a.Bt + static_cast<int64_t>(min(qw + 16 * jt + r, a.Q - 1)) * a.ldb + 8 * kb;
  const bool want_sum = a.colsum != nullptr && qw == 0;

  struct Frag {
    float4 a[8];
    int4 b[NPL][WJ];
  };
  auto load = [&](Frag &f, int k0) {
    if (k0 + 32 <= kend) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        f.a[j] = *reinterpret_cast<const float4 *>(ab + static_cast<int64_t>(k0 + j) * a.lda);
    } else {
      // last chunk of the last split: rows from kend on read row kend - 1 and count as zeros
      // (B holds zeros there too, but a non-finite A value times zero is not zero)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = k0 + 8 * kb + j;
        const float4 t = *reinterpret_cast<const float4 *>(
            ab + static_cast<int64_t>(min(k, kend - 1) - 8 * kb) * a.lda);
        f.a[j] = k < kend ? t : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt)
        f.b[pl][jt] = *reinterpret_cast<const int4 *>(bb[jt] + pl * a.bplane + k0);
  };

  v4f acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) acc[i][jt] = v4f{0.f, 0.f, 0.f, 0.f};
  float csum[4] = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Frag &f) {
    v8bf bf[NPL][WJ];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt) bf[pl][jt] = __builtin_bit_cast(v8bf, f.b[pl][jt]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = lane4(f.a[j], i);
      if (want_sum) {
#pragma unroll
        for (int j = 0; j < 8; ++j) csum[i] += v[j];
      }
      mma_split3<NPL, WJ>(v, bf, acc[i]);
    }
  };

  Frag f0, f1;
  if (kbeg < kend) load(f0, kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += 64) {
    const bool more = k0 + 32 < kend;
    if (more) load(f1, k0 + 32);
    compute(f0);
    if (!more) break;
    if (k0 + 64 < kend) load(f0, k0 + 64);
    compute(f1);
  }

  if (want_sum) {
    // lanes r, r + 16, r + 32, r + 48 hold the four k groups of the same columns
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      csum[i] += __shfl_xor(csum[i], 16, 64);
      csum[i] += __shfl_xor(csum[i], 32, 64);
      const int p = pw + 4 * r + i;
      if (kb == 0 && p < a.P) a.colsum[static_cast<int64_t>(s) * a.P + p] = csum[i];
    }
  }
  float *part = a.part + static_cast<int64_t>(s) * a.P * a.Q;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) {
      const int q = qw + 16 * jt + r;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int p = pw + 16 * kb + 4 * rr + i;  // output row 4 kb + rr of sub-tile i
        if (p < a.P && q < a.Q) part[static_cast<int64_t>(p) * a.Q + q] = acc[i][jt][rr];
      }
    }
}

// TN through LDS with direct global->LDS loads (global_load_lds_dwordx4).  Every wave copies
// its share of the workgroup's tile of the next 32-wide chunk into the other of two LDS stages
// (no registers involved) while it multiplies the current chunk; one barrier per chunk.  Waves
// read their fragments from LDS: A as 16 bytes along p (the sub-tile layout of tn_wave_kernel),
// B rows with their four 16-byte units XOR-swizzled by (q / 4) % 4, so that sixteen
// consecutive lanes reading one unit of sixteen rows touch all 64 banks once.  Within a chunk
// the split of sub-tile i + 1 is interleaved with the MFMAs of sub-tile i.
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void *src, void *lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)(lds_dst), 16, 0, 0);
}

template <int V>
using IC = std::integral_constant<int, V>;

// s_waitcnt vmcnt(0) lgkmcnt(0): this wave's LDS accesses and LDS copies are complete.
__device__ __forceinline__ void wait_vm_lgkm() { __builtin_amdgcn_s_waitcnt(7 << 4); }

// Workgroup barrier without a memory fence: the caller has waited for what must be complete
// (a fence would also wait for the LDS copies of the next chunk, just issued).  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int NPL, int WM, int WN, int WJ>
__global__ __launch_bounds__(64 * WM * WN, 2) void tn_lds_kernel(TnArgs a, TnMap map) {
  constexpr int NW = WM * WN, BP = 64 * WM, BQ = 16 * WJ * WN;
  constexpr int UPR = BP / 4;            // 16-byte units per A row of the tile
  constexpr int RPI = 64 / UPR;          // A rows per DMA instruction (1 KB)
  constexpr int A_INST = 32 / RPI / NW;  // A instructions per wave per chunk
  constexpr int B_INST = BQ / 16 / NW;   // B instructions per wave per chunk and plane
  static_assert(UPR <= 64 && 64 % UPR == 0 && (32 / RPI) % NW == 0 && (BQ / 16) % NW == 0,
                "tile shape does not divide into whole DMA instructions per wave");
  // one variable per stage, so the compiler can tell the stages apart when it counts the
  // copies a read has to wait for
  __shared__ __align__(16) float As0[32 * BP], As1[32 * BP];
  __shared__ __align__(16) unsigned Bs0[NPL * BQ * 16], Bs1[NPL * BQ * 16];

  int pt, qt, s;
  if (!tn_place(map, &pt, &qt, &s)) return;  // whole workgroup
  const int kbeg = s * a.kper, kend = min(a.K, kbeg + a.kper);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64, r = l % 16, kb = l / 16;
  const int wm = w / WN, wn = w % WN;
  const int p0 = BP * pt, q0 = BQ * qt;
  // DMA roles.  A block b (1 KB): rows RPI b + l / UPR, unit l % UPR; columns clamped into
  // the matrix (they only feed output rows past P).  B block b of a plane: row 16 b + l / 4,
  // physical unit l % 4 holding logical unit (l % 4) ^ ((row / 4) % 4); rows clamped to Q - 1.
  const float *asrc = a.A + min(p0 + 4 * (l % UPR), a.P - 4);
  const int arow = l / UPR;
  const __bf16 *bsrc[B_INST];
#pragma unroll
  for (int t = 0; t < B_INST; ++t) {
    const int q = 16 * (w * B_INST + t) + l / 4;
    bsrc[t] = a.Bt + static_cast<int64_t>(min(q0 + q, a.Q - 1)) * a.ldb + 8 * ((l % 4) ^ ((q / 4) % 4));
  }
  auto stage_a = [&](auto st) -> float * {
    if constexpr (decltype(st)::value == 0) return As0;
    else return As1;
  };
  auto stage_b = [&](auto st) -> unsigned * {
    if constexpr (decltype(st)::value == 0) return Bs0;
    else return Bs1;
  };
  auto issue = [&](auto st, int k0) {
    float *as = stage_a(st);
    unsigned *bs = stage_b(st);
#pragma unroll
    for (int t = 0; t < A_INST; ++t) {
      const int b = w * A_INST + t;
      const int row = min(k0 + RPI * b + arow, kend - 1);  // rows from kend on are zeroed on use
      dma16(asrc + static_cast<int64_t>(row) * a.lda, as + 256 * b);
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int t = 0; t < B_INST; ++t)
        dma16(bsrc[t] + pl * a.bplane + k0, bs + pl * BQ * 16 + 256 * (w * B_INST + t));
  };

  v4f acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) acc[i][jt] = v4f{0.f, 0.f, 0.f, 0.f};
  const bool want_sum = a.colsum != nullptr && q0 + 16 * WJ * wn == 0;
  float csum[4] = {0.f, 0.f, 0.f, 0.f};
  const int nch = (kend - kbeg + 31) / 32;

  // chunk c lives in stage c % 2; step(st, c) is called with st == c % 2
  auto step = [&](auto st, int c) {
    const int k0 = kbeg + 32 * c;
    wait_vm_lgkm();  // this wave's copies of chunk c are complete
    raw_barrier();   // so are every wave's; the other stage is free
    if (c + 1 < nch) issue(IC<1 - decltype(st)::value>{}, k0 + 32);
    const float *as = stage_a(st);
    const unsigned *bs = stage_b(st);
    float4 fa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      fa[j] = *reinterpret_cast<const float4 *>(as + (8 * kb + j) * BP + 64 * wm + 4 * r);
    if (k0 + 32 > kend) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + 8 * kb + j >= kend) fa[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (want_sum) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) csum[i] += lane4(fa[j], i);
    }
    v8bf bf[NPL][WJ];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt) {
        const int q = 16 * WJ * wn + 16 * jt + r;
        bf[pl][jt] = *reinterpret_cast<const v8bf *>(bs + pl * BQ * 16 + 16 * q + 4 * (kb ^ ((q / 4) % 4)));
      }
    uint4 h[4], m[4], o[4];
    {
      const float v[8] = {fa[0].x, fa[1].x, fa[2].x, fa[3].x, fa[4].x, fa[5].x, fa[6].x, fa[7].x};
      split3x8(v, h[0], m[0], o[0]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i + 1 < 4) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = lane4(fa[j], i + 1);
        split3x8(v, h[i + 1], m[i + 1], o[i + 1]);
      }
      const v8bf hi = __builtin_bit_cast(v8bf, h[i]), mid = __builtin_bit_cast(v8bf, m[i]),
                 lo = __builtin_bit_cast(v8bf, o[i]);
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) {
          acc[i][jt] = mfma_bf16(lo, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(mid, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(hi, bf[pl][jt], acc[i][jt]);
        }
      if (i + 1 < 4) {
        // the next sub-tile's split (about 44 VALU) between this sub-tile's MFMAs
#pragma unroll
        for (int g = 0; g < 3 * WJ * NPL; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      }
    }
  };

  if (0 < nch) issue(IC<0>{}, kbeg);
  for (int c = 0; c < nch; c += 2) {
    step(IC<0>{}, c);
    if (c + 1 >= nch) break;
    step(IC<1>{}, c + 1);
  }

  const int pw = p0 + 64 * wm, qw = q0 + 16 * WJ * wn;
  if (want_sum) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      csum[i] += __shfl_xor(csum[i], 16, 64);
      csum[i] += __shfl_xor(csum[i], 32, 64);
      const int p = pw + 4 * r + i;
      if (kb == 0 && p < a.P) a.colsum[static_cast<int64_t>(s) * a.P + p] = csum[i];
    }
  }
  float *part = a.part + static_cast<int64_t>(s) * a.P * a.Q;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) {
      const int q = qw + 16 * jt + r;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int p = pw + 16 * kb + 4 * rr + i;
        if (p < a.P && q < a.Q) part[static_cast<int64_t>(p) * a.Q + q] = acc[i][jt][rr];
      }
    }
}

// NT: out[m][n] = sum_k (A[m][k] kscale[k]) Bt[n][k]; A rows are k-contiguous, so a lane loads
// its 8 values of a row as two 16-byte pieces.  Workgroups of WM x WN waves; blockIdx.z is the
// K split.  One register set: a chunk's gradient fragments are split into bf16 planes and its
// B fragments copied out first, then the next chunk's loads are issued into the same
// registers and run under this chunk's MFMAs.
template <int NPL, int WM, int WN, int WJ>
__global__ __launch_bounds__(64 * WM * WN, 2) void nt_wave_kernel(NtArgs a) {
  constexpr int BM = 64 * WM, BN = 16 * WJ * WN;
  const int w = threadIdx.x / 64, l = threadIdx.x % 64, r = l % 16, kb = l / 16;
  const int mw = BM * blockIdx.x + 64 * (w / WN), nw = BN * blockIdx.y + 16 * WJ * (w % WN);
  if (mw >= a.M || nw >= a.N) return;  // whole wave; nothing below synchronises
  const int kz = blockIdx.z * a.kper, K = min(a.kper, a.K - kz);
  // rows are clamped into the matrices: a clamped lane only feeds outputs past M or N
  const float *ap = a.A + static_cast<int64_t>(min(mw + r, a.M - 1)) * a.lda + kz + 8 * kb;
  int aoff[4];  // element offsets of the sub-tile rows from row mw + r
#pragma unroll
  for (int i = 0; i < 4; ++i)
    aoff[i] = (min(mw + 16 * i + r, a.M - 1) - min(mw + r, a.M - 1)) * static_cast<int>(a.lda);
  const float *ks = a.kscale + kz + 8 * kb;
  const __bf16 *bb[WJ];
#pragma unroll
  for (int jt = 0; jt < WJ; ++jt)
    bb[jt] = a.Bt + static_cast<int64_t>(min(nw + 16 * jt + r, a.N - 1)) * a.ldb + kz + 8 * kb;
  float *out = a.out + blockIdx.z * a.out_split;

  float4 fa[4][2], fs[2];
  int4 fb[NPL][WJ];
  auto load = [&](int k0) {
    if (k0 + 32 <= K) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fa[i][h] = *reinterpret_cast<const float4 *>(ap + aoff[i] + k0 + 4 * h);
        fs[h] = *reinterpret_cast<const float4 *>(ks + k0 + 4 * h);
      }
    } else {
      // K is a multiple of 16: in a 16-wide last chunk the lanes with kb >= 2 lie past K;
      // they read at k0 and count as zeros
      const bool kin = k0 + 8 * kb < K;
      const int ko = kin ? k0 : k0 - 8 * kb;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 t = *reinterpret_cast<const float4 *>(ap + aoff[i] + ko + 4 * h);
          fa[i][h] = kin ? t : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const float4 t = *reinterpret_cast<const float4 *>(ks + ko + 4 * h);
        fs[h] = kin ? t : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt)
        fb[pl][jt] = *reinterpret_cast<const int4 *>(bb[jt] + pl * a.bplane + k0);
  };

  v4f acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) acc[i][jt] = v4f{0.f, 0.f, 0.f, 0.f};

  if (K > 0) load(0);
  for (int k0 = 0; k0 < K; k0 += kKC) {
    v8bf bf[NPL][WJ];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt) bf[pl][jt] = __builtin_bit_cast(v8bf, fb[pl][jt]);
    uint4 hi[4], mid[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 x0 = fa[i][0], x1 = fa[i][1], s0 = fs[0], s1 = fs[1];
      const float v[8] = {x0.x * s0.x, x0.y * s0.y, x0.z * s0.z, x0.w * s0.w,
                          x1.x * s1.x, x1.y * s1.y, x1.z * s1.z, x1.w * s1.w};
      split3x8(v, hi[i], mid[i], lo[i]);
    }
    if (k0 + kKC < K) load(k0 + kKC);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v8bf h = __builtin_bit_cast(v8bf, hi[i]), m = __builtin_bit_cast(v8bf, mid[i]),
                 o = __builtin_bit_cast(v8bf, lo[i]);
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) {
          acc[i][jt] = mfma_bf16(o, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(m, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(h, bf[pl][jt], acc[i][jt]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) {
      const int n = nw + 16 * jt + r;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int m = mw + 16 * i + 4 * kb + rr;
        if (m < a.M && n < a.N) out[static_cast<int64_t>(m) * a.ldo + n] = acc[i][jt][rr];
      }
    }
}

// NT through LDS with direct copies, as tn_lds_kernel: 2 x 2 waves of 64 x 16 WJ.  A rows
// (the 128 bytes of one 32-wide chunk) hold their eight 16-byte units XOR-swizzled by
// (m / 2) % 8, so that sixteen lanes reading one unit of sixteen consecutive rows touch all
// 64 banks once; B as in tn_lds_kernel; wave 0 copies the chunk's 32 k-scales.
template <int NPL, int WJ>
__global__ __launch_bounds__(256, 2) void nt_lds_kernel(NtArgs a) {
  constexpr int BM = 128, BN = 32 * WJ;
  constexpr int A_INST = BM / 8 / 4;   // 1 KB = 8 rows per instruction, per wave
  constexpr int B_INST = BN / 16 / 4;  // per wave and plane
  static_assert((BN / 16) % 4 == 0, "B rows must divide into whole instructions per wave");
  __shared__ __align__(16) float As0[BM * 32], As1[BM * 32];
  __shared__ __align__(16) unsigned Bs0[NPL * BN * 16], Bs1[NPL * BN * 16];
  __shared__ __align__(16) float Ks0[32], Ks1[32];
  const int w = threadIdx.x / 64, l = threadIdx.x % 64, r = l % 16, kb = l / 16;
  const int wm = w / 2, wn = w % 2;
  const int m0 = BM * blockIdx.x, n0 = BN * blockIdx.y;
  const int kz = blockIdx.z * a.kper, K = min(a.kper, a.K - kz);
  // A block b: rows 8 b + l / 8, physical unit l % 8 holding logical unit (l % 8) ^ ((row / 2)
  // % 8); rows clamped into the matrix (they only feed outputs past M)
  const float *asrc[A_INST];
  int au[A_INST];
#pragma unroll
  for (int t = 0; t < A_INST; ++t) {
    const int row = 8 * (w * A_INST + t) + l / 8;
    au[t] = 4 * ((l % 8) ^ ((row / 2) % 8));
    asrc[t] = a.A + static_cast<int64_t>(min(m0 + row, a.M - 1)) * a.lda + kz + au[t];
  }
  const __bf16 *bsrc[B_INST];
#pragma unroll
  for (int t = 0; t < B_INST; ++t) {
    const int q = 16 * (w * B_INST + t) + l / 4;
    bsrc[t] = a.Bt + static_cast<int64_t>(min(n0 + q, a.N - 1)) * a.ldb + kz + 8 * ((l % 4) ^ ((q / 4) % 4));
  }
  const float *ksrc = a.kscale + kz + 4 * (l % 8);
  auto stage_a = [&](auto st) -> float * {
    if constexpr (decltype(st)::value == 0) return As0;
    else return As1;
  };
  auto stage_b = [&](auto st) -> unsigned * {
    if constexpr (decltype(st)::value == 0) return Bs0;
    else return Bs1;
  };
  auto stage_k = [&](auto st) -> float * {
    if constexpr (decltype(st)::value == 0) return Ks0;
    else return Ks1;
  };
  // K is a multiple of 16: in a 16-wide last chunk the units past K read 16 columns earlier
  // (inside the row) and are zeroed on use
  auto issue = [&](auto st, int k0) {
    float *as = stage_a(st);
    unsigned *bs = stage_b(st);
#pragma unroll
    for (int t = 0; t < A_INST; ++t)
      dma16(asrc[t] + (k0 + au[t] < K ? k0 : k0 - 16), as + 256 * (w * A_INST + t));
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int t = 0; t < B_INST; ++t)
        dma16(bsrc[t] + pl * a.bplane + k0, bs + pl * BN * 16 + 256 * (w * B_INST + t));
    if (w == 0 && l < 8) dma16(ksrc + (k0 + 4 * l < K ? k0 : k0 - 16), stage_k(st));
  };

  v4f acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) acc[i][jt] = v4f{0.f, 0.f, 0.f, 0.f};
  const int nch = (K + 31) / 32;

  auto step = [&](auto st, int c) {
    const int k0 = 32 * c;
    wait_vm_lgkm();  // this wave's copies of chunk c are complete
    raw_barrier();   // so are every wave's; the other stage is free
    if (c + 1 < nch) issue(IC<1 - decltype(st)::value>{}, k0 + 32);
    const float *as = stage_a(st);
    const unsigned *bs = stage_b(st);
    const float *ks = stage_k(st);
    float4 fa[4][2], fs[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 64 * wm + 16 * i + r;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        fa[i][h] = *reinterpret_cast<const float4 *>(as + 32 * row + 4 * ((2 * kb + h) ^ ((row / 2) % 8)));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) fs[h] = *reinterpret_cast<const float4 *>(ks + 8 * kb + 4 * h);
    if (k0 + 32 > K && k0 + 8 * kb >= K) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        fs[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 4; ++i) fa[i][h] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    v8bf bf[NPL][WJ];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt) {
        const int q = 16 * WJ * wn + 16 * jt + r;
        bf[pl][jt] = *reinterpret_cast<const v8bf *>(bs + pl * BN * 16 + 16 * q + 4 * (kb ^ ((q / 4) % 4)));
      }
    auto prod = [&](int i, float (&v)[8]) {
      const float4 x0 = fa[i][0], x1 = fa[i][1], s0 = fs[0], s1 = fs[1];
      v[0] = x0.x * s0.x; v[1] = x0.y * s0.y; v[2] = x0.z * s0.z; v[3] = x0.w * s0.w;
      v[4] = x1.x * s1.x; v[5] = x1.y * s1.y; v[6] = x1.z * s1.z; v[7] = x1.w * s1.w;
    };
    uint4 h[4], m[4], o[4];
    {
      float v[8];
      prod(0, v);
      split3x8(v, h[0], m[0], o[0]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i + 1 < 4) {
        float v[8];
        prod(i + 1, v);
        split3x8(v, h[i + 1], m[i + 1], o[i + 1]);
      }
      const v8bf hi = __builtin_bit_cast(v8bf, h[i]), mid = __builtin_bit_cast(v8bf, m[i]),
                 lo = __builtin_bit_cast(v8bf, o[i]);
#pragma unroll
      for (int jt = 0; jt < WJ; ++jt)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) {
          acc[i][jt] = mfma_bf16(lo, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(mid, bf[pl][jt], acc[i][jt]);
          acc[i][jt] = mfma_bf16(hi, bf[pl][jt], acc[i][jt]);
        }
      if (i + 1 < 4) {
#pragma unroll
        for (int g = 0; g < 3 * WJ * NPL; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      }
    }
  };

  if (0 < nch) issue(IC<0>{}, 0);
  for (int c = 0; c < nch; c += 2) {
    step(IC<0>{}, c);
    if (c + 1 >= nch) break;
    step(IC<1>{}, c + 1);
  }

  float *out = a.out + blockIdx.z * a.out_split;
  const int mw = m0 + 64 * wm, nw = n0 + 16 * WJ * wn;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jt = 0; jt < WJ; ++jt) {
      const int n = nw + 16 * jt + r;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int mm = mw + 16 * i + 4 * kb + rr;
        if (mm < a.M && n < a.N) out[static_cast<int64_t>(mm) * a.ldo + n] = acc[i][jt][rr];
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
  // the partials are added in split order, eight loads in flight at a time
  auto sum_parts = [](const float *__restrict__ src, int64_t step, int count) {
    float acc = src[0];
    int s = 1;
    for (; s + 8 <= count; s += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[static_cast<int64_t>(s + u) * step];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; s < count; ++s) acc += src[static_cast<int64_t>(s) * step];
    return acc;
  };
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n + P; i += stride) {
    if (i < n) {
      const float acc = sum_parts(part + i, n, S);
      const int p = static_cast<int>(i / Q), q = static_cast<int>(i - static_cast<int64_t>(p) * Q);
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
      bias[p * ldo] = sum_parts(colsum + p, P, S * ath);
    }
  }
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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

// The same for a row-major source (cs = 1, rows 16-byte aligned): 16-byte loads of four
// columns, and 16-byte stores of eight consecutive rows per plane, through the same tile.
__global__ __launch_bounds__(256) void codes_t_rows_kernel(const float *__restrict__ src0,
                                                           int64_t rows0,
                                                           const float *__restrict__ src1,
                                                           int64_t rows, int cols, int64_t rs,
                                                           float zp, float div, int nplanes,
                                                           __bf16 *__restrict__ dst, int64_t ldd,
                                                           int64_t plane) {
  __shared__ int tile[64][65];
  const int64_t r0 = 64 * static_cast<int64_t>(blockIdx.x);
  const int c0 = 64 * blockIdx.y;
  const int cg = threadIdx.x % 16;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int rr = threadIdx.x / 16 + 16 * u;
    const int64_t r = r0 + rr;
    const int c = c0 + 4 * cg;
    int v[4] = {0, 0, 0, 0};
    if (r < rows) {
      const float *row = r < rows0 ? src0 + r * rs : src1 + (r - rows0) * rs;
      if (c + 4 <= cols) {
        const float4 x = *reinterpret_cast<const float4 *>(row + c);
        v[0] = static_cast<int>(rintf((x.x - zp) / div));
        v[1] = static_cast<int>(rintf((x.y - zp) / div));
        v[2] = static_cast<int>(rintf((x.z - zp) / div));
        v[3] = static_cast<int>(rintf((x.w - zp) / div));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < cols) v[e] = static_cast<int>(rintf((row[c + e] - zp) / div));
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[4 * cg + e][rr] = v[e];
  }
  __syncthreads();
  const int g = threadIdx.x % 8;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int cc = threadIdx.x / 8 + 32 * u;
    const int c = c0 + cc;
    const int64_t r = r0 + 8 * g;
    if (c >= cols || r >= ldd) continue;
    __bf16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = tile[cc][8 * g + e];
      if (nplanes == 1) {
        hi[e] = static_cast<__bf16>(static_cast<float>(v));
      } else {
        hi[e] = static_cast<__bf16>(static_cast<float>(256 * (v >> 8)));  // v = 256 hi + (v & 255)
        lo[e] = static_cast<__bf16>(static_cast<float>(v & 255));
      }
    }
    // ldd is a multiple of 8, so the eight rows lie inside the destination row
    __bf16 *d = dst + static_cast<int64_t>(c) * ldd + r;
    uint4 w;
    __builtin_memcpy(&w, hi, sizeof w);
    *reinterpret_cast<uint4 *>(d) = w;
    if (nplanes == 2) {
      __builtin_memcpy(&w, lo, sizeof w);
      *reinterpret_cast<uint4 *>(d + plane) = w;
    }
  }
}

int codes_t(const float *src0, int64_t rows0, const float *src1, int64_t rows, int cols, int64_t rs,
            int64_t cs, float zp, float div, int nplanes, __bf16 *dst, int64_t ldd, int64_t plane,
            hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(ldd >= rows && (rows0 >= rows || src1 != nullptr), "bad codes_t layout");
  const dim3 grid(static_cast<unsigned>((ldd + 63) / 64), static_cast<unsigned>((cols + 63) / 64));
  const bool rows_ok = cs == 1 && rs % 4 == 0 && aligned16(src0) && (src1 == nullptr || aligned16(src1)) &&
                       ldd % 8 == 0 && plane % 8 == 0 && aligned16(dst);
  if (rows_ok)
    hipLaunchKernelGGL(codes_t_rows_kernel, grid, dim3(256), 0, stream, src0, rows0, src1, rows, cols,
                       rs, zp, div, nplanes, dst, ldd, plane);
  else
    hipLaunchKernelGGL(codes_t_kernel, grid, dim3(256), 0, stream, src0, rows0, src1, rows, cols, rs,
                       cs, zp, div, nplanes, dst, ldd, plane);
  RXMET_CHECK_LAUNCH();
  return 0;
}

// Wave grid (WM x WN waves, each 64 x 16 WJ) of a TN or NT product, by the width of the B side.
struct WaveTile {
  int wm, wn, wj;
  bool lds = false;
  int rows() const { return 64 * wm; }
  int cols() const { return 16 * wj * wn; }
};
static WaveTile wave_tile(int width) {
  if (width <= 32) return {4, 1, 2};
  if (width <= 48) return {4, 1, 3};
  if (width <= 64) return {4, 1, 4};
  if (width <= 80) return {4, 1, 5};
  return {2, 2, 4};
}
// TN: widths up to 80 on tn_wave_kernel; wider ones through LDS (tn_lds_kernel), one code plane
// with 64 x 128 wave tiles from a width of 256 (the split of a gradient fragment then feeds
// twice as many MFMAs).
static WaveTile tn_tile(int width, int nplanes) {
  if (width <= 80) return wave_tile(width);
  if (nplanes == 1 && width >= 256) return {2, 2, 8, true};
  return {2, 2, 4, true};
}

// Placement of a TN product on bp x bq block tiles in S splits (see tn_place); `blocks` is the
// grid size.
constexpr int kXcdSlots = 64;  // resident workgroups per XCD: 32 CUs x 2
static TnMap tn_map(int P, int Q, int S, int bp, int bq, unsigned *blocks) {
  TnMap m;
  const int ntp = (P + bp - 1) / bp;
  m.ntq = (Q + bq - 1) / bq;
  m.tiles = ntp * m.ntq;
  // keep whole p-tiles in a group (their q-tiles share the A rows)
  m.gt = m.ntq >= kXcdSlots ? m.ntq : std::min(m.tiles, kXcdSlots / m.ntq * m.ntq);
  m.gps = (m.tiles + m.gt - 1) / m.gt;
  m.ngroups = m.gps * S;
  *blocks = static_cast<unsigned>(8 * ((m.ngroups + 7) / 8) * m.gt);
  return m;
}

void tn_plan(int K, int P, int Q, int nplanes, int *S, int *kper) {
  const WaveTile t = tn_tile(Q, nplanes);
  const int chunks = (K + kKC - 1) / kKC;
  // Makespan model in chunk times.  The groups of tn_place go round robin over the eight XCDs,
  // whose 64 workgroup slots (two per CU) take them in rounds; the busiest XCD sets the time.
  // Each split also adds one [P][Q] partial to write and re-read (about 6.5 MB per chunk time).
  const double part_cost = 8.0 * P * Q / 6.5e6;
  int best = 1;
  double best_cost = 0.0;
  const int smax = chunks / 16 > 1 ? chunks / 16 : 1;
  for (int s = 1; s <= smax; ++s) {
    const int per = (chunks + s - 1) / s;
    if ((s - 1) * per >= chunks) continue;  // an empty split
    unsigned blocks = 0;
    const TnMap m = tn_map(P, Q, s, t.rows(), t.cols(), &blocks);
    const int load = (m.ngroups + 7) / 8 * m.gt;  // workgroups of the busiest XCD
    const int rounds = (load + kXcdSlots - 1) / kXcdSlots;
    const double cost = static_cast<double>(rounds) * per + part_cost * s;
    if (s == 1 || cost < best_cost) {
      best = s;
      best_cost = cost;
    }
  }
  const int per = (chunks + best - 1) / best;
  *kper = per * kKC;
  *S = (K + *kper - 1) / *kper;
}

void nt_plan(int M, int N, int K, int max_split, int *S, int *kper) {
  const WaveTile t = wave_tile(N);
  const int waves = ((M + 63) / 64) * ((N + 16 * t.wj - 1) / (16 * t.wj));
  // about one wave per SIMD (1024 on the GPU), each over at least 8 chunks of K: two waves
  // per SIMD measured the same at c5 (a faster GEMM, but twice the partial sums to add)
  int s = (1024 + waves - 1) / waves;
  const int chunks = (K + kKC - 1) / kKC;
  if (s > chunks / 8) s = chunks / 8;
  if (s > max_split) s = max_split;
  if (s < 1) s = 1;
  int per = ((K + s - 1) / s + kKC - 1) / kKC * kKC;
  while (s > 1 && per * (s - 1) >= K) --s;
  *S = s;
  *kper = s > 1 ? per : K;
}

template <int NPL, int WM, int WN, int WJ>
static void tn_launch(const TnArgs &a, hipStream_t stream) {
  unsigned blocks = 0;
  const TnMap m = tn_map(a.P, a.Q, a.S, 64 * WM, 16 * WJ * WN, &blocks);
  hipLaunchKernelGGL((tn_wave_kernel<NPL, WM, WN, WJ>), dim3(blocks), dim3(64 * WM * WN), 0, stream,
                     a, m);
}

template <int NPL, int WJ>
static void tn_lds_launch(const TnArgs &a, hipStream_t stream) {
  unsigned blocks = 0;
  const TnMap m = tn_map(a.P, a.Q, a.S, 128, 32 * WJ, &blocks);
  hipLaunchKernelGGL((tn_lds_kernel<NPL, 2, 2, WJ>), dim3(blocks), dim3(256), 0, stream, a, m);
}

template <int NPL>
static void tn_dispatch(const TnArgs &a, hipStream_t stream) {
  const WaveTile t = tn_tile(a.Q, NPL);
  if (t.lds) {
    if constexpr (NPL == 1)
      if (t.wj == 8) return tn_lds_launch<1, 8>(a, stream);
    return tn_lds_launch<NPL, 4>(a, stream);
  }
  switch (t.wj) {
    case 2: return tn_launch<NPL, 4, 1, 2>(a, stream);
    case 3: return tn_launch<NPL, 4, 1, 3>(a, stream);
    case 4: return tn_launch<NPL, 4, 1, 4>(a, stream);
    default: return tn_launch<NPL, 4, 1, 5>(a, stream);
  }
}

int tn(const TnArgs &a, int nplanes, hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(a.kper % kKC == 0 && a.ldb % 8 == 0 && aligned16(a.Bt), "bad TN layout");
  // 16-byte A loads along p
  RXMET_CHECK_ARG(aligned16(a.A) && a.lda % 4 == 0 && a.P % 4 == 0 && a.P >= 4,
                  "TN gradient rows must be 16-byte aligned with P a multiple of 4");
  if (nplanes == 1)
    tn_dispatch<1>(a, stream);
  else
    tn_dispatch<2>(a, stream);
  RXMET_CHECK_LAUNCH();
  return 0;
}

template <int NPL, int WM, int WN, int WJ>
static void nt_launch(const NtArgs &a, hipStream_t stream) {
  constexpr int BM = 64 * WM, BN = 16 * WJ * WN;
  const dim3 grid((a.M + BM - 1) / BM, (a.N + BN - 1) / BN, a.ksplit);
  hipLaunchKernelGGL((nt_wave_kernel<NPL, WM, WN, WJ>), grid, dim3(64 * WM * WN), 0, stream, a);
}

template <int NPL>
static void nt_dispatch(const NtArgs &a, hipStream_t stream) {
  const WaveTile t = wave_tile(a.N);
  if (t.wn == 2) {  // widths above 80 through LDS
    const dim3 grid((a.M + 127) / 128, (a.N + 127) / 128, a.ksplit);
    hipLaunchKernelGGL((nt_lds_kernel<NPL, 4>), grid, dim3(256), 0, stream, a);
    return;
  }
  switch (t.wj) {
    case 2: return nt_launch<NPL, 4, 1, 2>(a, stream);
    case 3: return nt_launch<NPL, 4, 1, 3>(a, stream);
    case 4: return nt_launch<NPL, 4, 1, 4>(a, stream);
    default: return nt_launch<NPL, 4, 1, 5>(a, stream);
  }
}

int nt(const NtArgs &a, int nplanes, hipStream_t stream) {
  RXMET_CHECK_ARG(nplanes == 1 || nplanes == 2, "nplanes must be 1 or 2");
  RXMET_CHECK_ARG(a.K % 16 == 0 && a.lda % 4 == 0 && a.ldb % 8 == 0, "bad NT layout");
  RXMET_CHECK_ARG(aligned16(a.A) && aligned16(a.kscale) && aligned16(a.Bt),
                  "NT operands must be 16-byte aligned");
  // B is read in whole 32-wide K chunks: its rows must hold zeros up to a multiple of 32
  RXMET_CHECK_ARG(a.ldb >= (a.K + 31) / 32 * 32, "NT B rows must be padded to a multiple of 32");
  RXMET_CHECK_ARG(a.ksplit >= 1 && (a.ksplit == 1 || (a.kper % 32 == 0 && a.kper * (a.ksplit - 1) < a.K)),
                  "bad NT K split");
  NtArgs b = a;
  if (b.ksplit == 1) b.kper = b.K;
  if (nplanes == 1)
    nt_dispatch<1>(b, stream);
  else
    nt_dispatch<2>(b, stream);
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
                     part, S, P, Q, qscale, out, ldo, transpose, 1, colsum,
                     bias, mask, swap_h);
  RXMET_CHECK_LAUNCH();
  return 0;
}

}  // namespace wgrad
}  // namespace rxmet
