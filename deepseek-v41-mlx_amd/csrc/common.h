// Shared device helpers and host-side error plumbing for the dsv41 HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/dsv41.h"

namespace dsv41 {

// ------------------------------------------------------------------ host errors

// Records a message for dsv41_last_error_string() and returns `code`.
int set_error(int code, const char* fmt, ...);
// Checks the launch that was just enqueued; returns 0 or the hipError_t.
int check_launch(const char* what);

#define DSV41_REQUIRE(cond, code, ...)                  \
  do {                                                  \
    if (!(cond)) return ::dsv41::set_error((code), __VA_ARGS__); \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// ------------------------------------------------------------------ numerics

typedef uint16_t bf16_t;  // raw bfloat16 bits

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float -> bfloat16, round to nearest even (torch / MLX semantics).
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (bf16_t)0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf2f(f2bf(f)); }

// Typed load/store: T = float or bf16_t; `rnd` rounds an fp32 value to T's precision.
template <typename T> struct io;
template <> struct io<float> {
  __device__ __forceinline__ static float ld(const float* p) { return *p; }
  __device__ __forceinline__ static void st(float* p, float v) { *p = v; }
  __device__ __forceinline__ static float rnd(float v) { return v; }
  static constexpr int kDtype = DSV41_F32;
};
template <> struct io<bf16_t> {
  __device__ __forceinline__ static float ld(const bf16_t* p) { return bf2f(*p); }
  __device__ __forceinline__ static void st(bf16_t* p, float v) { *p = f2bf(v); }
  __device__ __forceinline__ static float rnd(float v) { return round_bf16(v); }
  static constexpr int kDtype = DSV41_BF16;
};

// 2**ceil(log2(r)) from IEEE bits (the TileLang fast_round_scale, kernel.py:22-37).
// ue8m0 scale byte -> float 2^(e-127) (e = 0 is 2^-127, a subnormal; 255 is NaN).
// e << 23 is the float 2^(e-127) for 1 <= e <= 254; e = 0 and e = 255 differ from it in bit 22 only
// (0x00400000, 0x7fc00000), so the special cases are one select and the whole conversion has no
// branch.
__device__ __forceinline__ float e8m0_to_float(uint32_t e) {
  return __uint_as_float((e << 23) | ((e == 0u || e == 255u) ? 0x00400000u : 0u));
}

__device__ __forceinline__ float pow2_ceil_log2(float r) {
  uint32_t b = __float_as_uint(r);
  int e = (int)((b >> 23) & 0xFFu) - 127 + ((b & 0x7FFFFFu) != 0u);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// Nearest OCP e4m3fn value, ties to even; |x| <= 448 expected (callers clip first).
__device__ __forceinline__ float e4m3_round(float x) {
  float a = fabsf(x);
  float r;
  if (a < 0.015625f) {  // below 2^-6: subnormal grid, quantum 2^-9
    r = rintf(a * 512.0f) * (1.0f / 512.0f);
  } else {              // 3 mantissa bits, round to nearest even at bit 20
    uint32_t u = __float_as_uint(a);
    u = (u + 0x7FFFFu + ((u >> 20) & 1u)) & ~0xFFFFFu;
    r = __uint_as_float(u);
  }
  return copysignf(r, x);
}

// e4m3fn byte encoding of a value already on the e4m3 grid (|x| <= 448).
__device__ __forceinline__ uint8_t e4m3_encode(float q) {
  uint32_t s = (__float_as_uint(q) >> 31) << 7;
  float a = fabsf(q);
  if (a < 0.015625f) return (uint8_t)(s | (uint32_t)(a * 512.0f));
  uint32_t u = __float_as_uint(a);
  uint32_t e = ((u >> 23) & 0xFFu) - 127u + 7u;
  return (uint8_t)(s | (e << 3) | ((u >> 20) & 7u));
}

__device__ __forceinline__ float e4m3_decode(uint8_t c) {
  uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  float a = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * (1.0f / 512.0f);
  return (c & 0x80u) ? -a : a;
}

// Nearest e2m1 magnitude with the reference's tie table (fakequant.py:65-73), sign kept.
__device__ __forceinline__ float e2m1_round(float v) {
  float m = fabsf(v);
  float r = m > 5.0f    ? 6.0f
            : m >= 3.5f  ? 4.0f
            : m > 2.5f   ? 3.0f
            : m >= 1.75f ? 2.0f
            : m > 1.25f  ? 1.5f
            : m >= 0.75f ? 1.0f
            : m > 0.25f  ? 0.5f
                         : 0.0f;
  return copysignf(r, v);
}

// e2m1 code (sign in bit 3) of the value e2m1_round(v) gives: same thresholds, so the code's
// value is exactly that rounding (-0 keeps its sign, as copysignf does there).
__device__ __forceinline__ uint32_t e2m1_code(float v) {
  const float m = fabsf(v);
  const uint32_t c = m > 5.0f    ? 7u
                     : m >= 3.5f  ? 6u
                     : m > 2.5f   ? 5u
                     : m >= 1.75f ? 4u
                     : m > 1.25f  ? 3u
                     : m >= 0.75f ? 2u
                     : m > 0.25f  ? 1u
                                  : 0u;
  return c | ((__float_as_uint(v) >> 28) & 8u);
}

// MXFP4 encoding of N (a multiple of 8) values of one 32-value block whose absolute maximum is
// amax (the whole block's: callers holding part of a block combine the maxima of its lanes
// first), with fake_quant_fp4_ue8m0's scale and rounding (fakequant.py:96-106): codes[w] holds
// values 8w..8w+7, value 8w+i in nibble i (so byte p holds values 2p and 2p+1, the even one in
// the low nibble); returns the ue8m0 scale byte (scale 2^(byte-127)). Decoding
// e2m1(code) * scale gives exactly the fake-quantized value.
template <int N>
__device__ __forceinline__ uint32_t mxfp4_encode(const float* v, float amax, uint32_t* codes) {
  amax = fmaxf(amax, (float)(6.0 * 1.1754943508222875e-38));  // 6 * 2^-126
  const float s = pow2_ceil_log2(amax * (float)(1.0 / 6.0));
  const float inv = __fdiv_rn(1.0f, s);                       // exact: s is a power of two
#pragma unroll
  for (int w = 0; w < N / 8; ++w) {
    uint32_t c = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) c |= e2m1_code(fminf(fmaxf(v[8 * w + i] * inv, -6.0f), 6.0f)) << (4 * i);
    codes[w] = c;
  }
  return (__float_as_uint(s) >> 23) & 0xFFu;
}

// Rotation of the adjacent pair (x0, x1) by (c, s): x0 c - x1 s, x0 s + x1 c, each product and
// each sum rounded to fp32 on its own as the reference's separate float32 array operations round
// them. Contraction is off here: hipcc fuses a product into the following add by default, and a
// fused multiply-add rounds once where this arithmetic rounds twice.
__device__ __forceinline__ void rotate_pair(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
  const float xr = x0, xi = x1;
  x0 = xr * c - xi * s;
  x1 = xr * s + xi * c;
}

// ------------------------------------------------------------------ wave helpers

__device__ __forceinline__ float wave_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

__device__ __forceinline__ float group_max(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, wave_xor_f(v, o));
  return v;
}
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += wave_xor_f(v, o);
  return v;
}

}  // namespace dsv41
