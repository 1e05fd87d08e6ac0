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
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x16_bf16: 4 bf16 per lane, lane group g owns k = 4g..4g+3.
__device__ __forceinline__ f32x4 mfma16x16x16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;

// ds_read_b64_tr_b16: within each 16-lane group, lane i returns element (i % 4) of the 8-byte
// reads of lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12. If lane r of a group reads 4 consecutive
// 16-bit values of row (r / 4) at column 4 * (r % 4), lane i receives column i of those 4 rows:
// a 4 x 16 block comes back transposed, one column per lane.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p));
}

// One 16-byte-per-lane global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes land at
// lds_base + 16 * l; lds_base must be wave-uniform. Completion is tracked by vmcnt only.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((gbl_void*)src, (lds_void*)lds_base, 16, 0, 0);
}

// Same copy, issued as inline asm (saddr form: `base` wave-uniform, `voff` per lane, LDS byte
// offset `lds` in M0). The compiler's wait-count pass cannot see an LDS write behind it, so it
// never adds a full vmcnt(0) drain in front of LDS reads that it cannot prove disjoint from the
// copies in flight; completion is tracked only by the caller's explicit vmcnt waits. M0 carries
// no other value in the kernels that use it.
__device__ __forceinline__ void dma16_sgpr(uint64_t base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}

// Same copy with a per-lane 64-bit address (vaddr form): lanes may read from different
// buffers, e.g. a row's data and its block scales in one instruction.
__device__ __forceinline__ void dma16_vaddr(uint64_t addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(addr), "s"(lds)
               : "memory", "m0");
}

// The vaddr-form copy with the non-temporal hint: for data read once (streamed key caches), so
// that it does not displace what later kernels read from L2 and the Infinity Cache.
__device__ __forceinline__ void dma16_vaddr_nt(uint64_t addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(addr), "s"(lds)
               : "memory", "m0");
}

// s_waitcnt immediate (gfx9 encoding): vmcnt 0, expcnt 7 and lgkmcnt 15 (no wait on those).
// As __builtin_amdgcn_s_waitcnt it is visible to the compiler's wait-count pass.
constexpr int kWaitVmcnt0 = 0x0F70;

// Wait until at most N vector-memory operations of this wave are outstanding (asm: invisible
// to the wait-count pass; used for the LDS copies it does not track).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Sum of v over the four 16-lane rows of the wave (lanes l, l^16, l^32, l^48), in every lane:
// (v[l] + v[l^16]) + (v[l^32] + v[l^48]), the additions of v + shfl_xor(v, 16) followed by
// + shfl_xor(., 32), but with gfx950's row-swap permutes (VALU) instead of LDS-routed shuffles.
// permlane16_swap(x, x) returns (x[l], x[l^16]) in row-pair order and permlane32_swap(x, x)
// (x[l], x[l^32]) (checked lane by lane on the hardware).
__device__ __forceinline__ float sum_rows4(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto s16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  const float y = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
  const uint32_t c = __float_as_uint(y);
  const auto s32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
}

// max(x, 0) as one integer max of the bits: a negative float has the sign bit set, so it becomes
// +0.0, and a non-negative one passes unchanged. fmaxf(x, 0.0f) costs two v_max_f32 in IEEE mode
// (the first quiets a signalling NaN); this differs from it only for NaN inputs and in giving +0.0
// for -0.0. Used on MFMA accumulators in the indexer epilogues.
__device__ __forceinline__ float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// LDS byte offset of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ i16x4 pack_bf16x4(const float* v) {
  i16x4 r;
  r[0] = (short)f2bf(v[0]);
  r[1] = (short)f2bf(v[1]);
  r[2] = (short)f2bf(v[2]);
  r[3] = (short)f2bf(v[3]);
  return r;
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

// 8 floats -> MFMA operand with the hardware round-to-nearest-even convert (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 cvt_bf16x8(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)v[i];
  return r;
}

// Two floats -> packed bf16 pair (a in the low half) with the hardware round-to-nearest-even
// convert (v_cvt_pk_bf16_f32): the bits of f2bf for every non-NaN value, in one instruction.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  bf16x2 v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// The two bf16 values of a packed pair (low half first), widened exactly and summed in fp32.
__device__ __forceinline__ float sum_bf16x2(uint32_t u) {
  return __uint_as_float(u << 16) + __uint_as_float(u & 0xFFFF0000u);
}

// 2^x with the bare v_exp_f32 (no denormal-range fix-up). Used for softmax weights 2^(s - m) with
// s - m <= the lazy-rescale threshold: results below 2^-126 are zero for the sum anyway.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 e4m3fn codes (two dwords, channel i in byte i) times a power-of-two scale -> MFMA operand.
// v_cvt_scalef32_pk_bf16_fp8 decodes two OCP e4m3fn codes (subnormals included), applies the
// scale's exponent -- all of a normal power of two (2^-126 .. 2^127), which the ue8m0 scales of
// the fp8 caches (bytes 1..254) are -- and packs the two bf16 results: one instruction per two
// channels (decoding to fp32 and packing separately took two). Exact: e4m3 values scaled by 2^k
// are bf16-representable within bf16's exponent range.
__device__ __forceinline__ bf16x8 dequant_e4m3x8(uint32_t lo, uint32_t hi, float scale) {
  typedef __attribute__((ext_vector_type(2))) __bf16 b2;
  const b2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, scale, false);
  const b2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, scale, true);
  const b2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, scale, false);
  const b2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, scale, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// 8 e2m1 codes (one dword; channel 2p in the low nibble of byte p) times an e4m3 block scale ->
// MFMA operand. v_cvt_scalef32_pk_f32_fp4 decodes the two codes of one byte (scale 1); the e4m3
// scale, which is not a power of two in general, is a separate multiply. Exact: an e2m1 value
// times an e4m3 value has at most 6 significant bits and lies inside bf16's exponent range.
__device__ __forceinline__ bf16x8 dequant_e2m1x8(uint32_t codes, float scale) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  const f2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, 1.0f, 0);
  const f2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, 1.0f, 1);
  const f2 c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, 1.0f, 2);
  const f2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(codes, 1.0f, 3);
  const float v[8] = {a[0] * scale, a[1] * scale, b[0] * scale, b[1] * scale,
                      c[0] * scale, c[1] * scale, d[0] * scale, d[1] * scale};
  return cvt_bf16x8(v);
}

}  // namespace dsv41
