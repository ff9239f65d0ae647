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

// Pack four int8 values into one 32-bit word (byte 0 = a).
__device__ __forceinline__ int pack4_i8(int a, int b, int c, int d) {
  return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((d & 0xff) << 24);
}

}  // namespace rxmet
