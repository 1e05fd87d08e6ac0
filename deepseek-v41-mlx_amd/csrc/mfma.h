// gfx950 MFMA operand types and helpers shared by the indexer and sparse-MLA kernels.
//
// v_mfma_f32_16x16x32_bf16: D[16x16] += A[16x32] * B[32x16]. Lane j supplies A row (j % 16)
// and B column (j % 16), each as 8 bf16 of the k range owned by lane group g = j / 16; A and
// B use the same lane -> k assignment, so any permutation of k that both operands share gives
// the same contraction. Lane j receives D[4*g + i][j % 16], i = 0..3.
#pragma once

#include "common.h"

namespace dsv41 {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ bf16x8 ld_bf16x8(const void* p) {
  return as_bf16x8(*reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ bf16x8 zero_bf16x8() { return as_bf16x8(make_uint4(0, 0, 0, 0)); }

// Pack 8 floats (rounded to nearest even) into an MFMA operand.
__device__ __forceinline__ bf16x8 pack_bf16x8(const float* v) {
  uint4 u;
  u.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  u.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  u.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
  u.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
  return as_bf16x8(u);
}

}  // namespace dsv41
