// mfma_frag.h — gfx950 MFMA wrappers and the fragment layouts the kernels use.
//
// v_mfma_i32_16x16x64_i8:  lane l supplies A[l % 16][16 * (l / 16) + j] and
//                          B[16 * (l / 16) + j][l % 16] for j = 0..15 (16 int8 = 4 VGPRs).
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l % 16][8 * (l / 16) + j] and
//                          B[8 * (l / 16) + j][l % 16] for j = 0..7 (8 bf16 = 4 VGPRs).
// v_mfma_f32_16x16x4_f32:   lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]
//                          (one fp32 each).
// All three: lane l receives D[4 * (l / 16) + r][l % 16] for r = 0..3.
// The contraction index only has to be assigned identically for A and B; the test
// rxmet_selftest_mfma checks these layouts on the device.
#pragma once

#include <hip/hip_runtime.h>

namespace rxmet {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f mfma_bf16(v8bf a, v8bf b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// The two bf16 halves of a packed word as floats (exact).
__device__ __forceinline__ v2f unpack_bf16x2(unsigned u) {
  return v2f{__builtin_bit_cast(float, u << 16), __builtin_bit_cast(float, u & 0xffff0000u)};
}

__device__ __forceinline__ unsigned pack_bf16x2(v2f a) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(a, v2bf));
}

// a = hi + mid + lo exactly, for two values at once (packed bf16 pairs, first value in the
// low half): each term is the RNE bf16 of what the previous ones leave (the differences are
// exact in fp32).  Non-finite inputs give non-finite terms.
__device__ __forceinline__ void split3x2(v2f a, unsigned &hi, unsigned &mid, unsigned &lo) {
  hi = pack_bf16x2(a);
  const v2f r1 = a - unpack_bf16x2(hi);
  mid = pack_bf16x2(r1);
  const v2f r2 = r1 - unpack_bf16x2(mid);
  lo = pack_bf16x2(r2);
}

// Eight k-consecutive values -> three 16-byte bf16 planes (MFMA operand fragments).
__device__ __forceinline__ void split3x8(const float (&v)[8], uint4 &hi, uint4 &mid, uint4 &lo) {
  unsigned h[4], m[4], o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) split3x2(v2f{v[2 * e], v[2 * e + 1]}, h[e], m[e], o[e]);
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  mid = make_uint4(m[0], m[1], m[2], m[3]);
  lo = make_uint4(o[0], o[1], o[2], o[3]);
}

// Pack four int8 values into one 32-bit word (byte 0 = a).
__device__ __forceinline__ int pack4_i8(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((d & 0xff) << 24);
}

}  // namespace rxmet
