// Row pipelines of the attention path: RMSNorm -> rope tail -> QAT fake-quant, each stage
// rounded to the activation dtype exactly where the reference rounds, fused into one pass
// over HBM. A thread owns EPT consecutive elements of a 32-element chunk of a row (fake-quant
// blocks of 16/32 and rope pairs never straddle chunks): with EPT = 8 the 4 lanes of a chunk
// form a block's maximum by two cross-lane steps and the row's lanes its RMSNorm sum, which
// keeps each thread's chain short (a decode step has only a few hundred rows); EPT = 32 serves
// norms over rows wider than 64 x 8 elements.
//
// Reference semantics: deepseek_v41_mlx/fakequant.py:47-119, layers.py:20-84,
// attention.py:119-122, 157-163, indexer.py:89-104, 179-181, cache.py:61-67.
#include "common.h"

namespace dsv41 {

// FQ_FP4_MX: the FQ_FP4_UE8M0 values stored packed (MXFP4 codes + ue8m0 scale bytes);
// FQ_FP8_PACK: the FQ_FP8_UE8M0 values stored packed (e4m3fn codes + ue8m0 scale bytes);
// FQ_FP4_E4M3_PACK: the FQ_FP4_E4M3 values stored packed, one row of dim/2 e2m1 code bytes then
// dim/16 e4m3 scale bytes
enum FqKind { FQ_NONE = 0, FQ_FP8_UE8M0 = 1, FQ_FP4_UE8M0 = 2, FQ_FP4_E4M3 = 3, FQ_FP4_MX = 4, FQ_FP8_PACK = 5,
              FQ_FP4_E4M3_PACK = 6 };

struct RowArgs {
  const void* src;          // [rows, dim] contiguous
  void* dst;                // row (b, s, h) at dst + b*dst_bstride + (tok_base+s)*dst_tstride + h*dim
  int64_t rows;
  int dim, cpr;             // cpr = dim / 32 chunks per row
  int S, H;                 // tokens per batch row, rows per token
  int64_t dst_bstride, dst_tstride;
  int tok_base;
  const float* norm_w;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  int rd, pos_base, pos_step, inverse;
  // packed stores (FQ_FP4_MX, FQ_FP8_PACK): dst takes dim/2 (fp4) or dim (fp8) code bytes per
  // row and dst2 dim/32 scale bytes; all four strides in bytes
  uint8_t* dst2;
  int64_t dst2_bstride, dst2_tstride;
  // FQ_FP8_PACK: one scale byte per 32 channels covers `srb` consecutive cache rows (1 or 32);
  // with 32, a row that opens a block sets the block's scale and the block's later rows are
  // quantized with it. Such a write runs in two launches: phase 0 the rows that open a block,
  // phase 1 the others (which read the scales phase 0 or an earlier call stored).
  int srb, phase;
};

// N (a multiple of 8) consecutive elements, 16-byte aligned
template <typename T, int N> __device__ __forceinline__ void loadn(const T* p, float* v) {
  if constexpr (sizeof(T) == 4) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      float4 t = q[i];
      v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
  } else {
    const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      uint4 t = q[i];
      uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
        v[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
      }
    }
  }
}
template <typename T, int N> __device__ __forceinline__ void storen(T* p, const float* v) {
  if constexpr (sizeof(T) == 4) {
    float4* q = reinterpret_cast<float4*>(p);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) q[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  } else {
    uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)f2bf(v[8 * i + 2 * j]) | ((uint32_t)f2bf(v[8 * i + 2 * j + 1]) << 16);
      q[i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// One fake-quant block of BLK values, N of them in this thread at v[0..N): N = BLK, or N < BLK
// with the block's other values in the BLK/N neighbouring lanes (an aligned lane group), whose
// maxima are combined. Rounded back to T.
template <typename T, int FQ, int BLK, int N>
__device__ __forceinline__ void fake_quant_block(float* v) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) amax = fmaxf(amax, fabsf(v[i]));
  if constexpr (BLK > N) amax = group_max(amax, BLK / N);
  if (FQ == FQ_FP8_UE8M0) {
    amax = fmaxf(amax, 1e-4f);
    const float s = pow2_ceil_log2(amax * (float)(1.0 / 448.0));
    const float inv = __fdiv_rn(1.0f, s);   // s is a power of two: x * (1/s) rounds as x / s does
#pragma unroll
    for (int i = 0; i < N; ++i)
      v[i] = io<T>::rnd(e4m3_round(fminf(fmaxf(v[i] * inv, -448.0f), 448.0f)) * s);
  } else if (FQ == FQ_FP4_UE8M0) {
    amax = fmaxf(amax, (float)(6.0 * 1.1754943508222875e-38));  // 6 * 2^-126
    const float s = pow2_ceil_log2(amax * (float)(1.0 / 6.0));
    const float inv = __fdiv_rn(1.0f, s);   // s is a power of two: x * (1/s) rounds as x / s does
#pragma unroll
    for (int i = 0; i < N; ++i)
      v[i] = io<T>::rnd(e2m1_round(fminf(fmaxf(v[i] * inv, -6.0f), 6.0f)) * s);
  } else if (FQ == FQ_FP4_E4M3) {
    amax = fmaxf(amax, 0.01171875f);                             // 6 * 2^-9
    const float s = e4m3_round(__fdiv_rn(amax, 6.0f));
#pragma unroll
    for (int i = 0; i < N; ++i)
      v[i] = io<T>::rnd(e2m1_round(fminf(fmaxf(__fdiv_rn(v[i], s), -6.0f), 6.0f)) * s);
  }
}

// Row coordinates of thread gid with `upr` threads per row: (row, unit u within the row, head h,
// token s, batch row b). Launches with fewer than 2^32 threads (the common case) use 32-bit
// division, a short sequence where the 64-bit one is a long software routine.
struct RowPos {
  int64_t row, b;
  int u, h, s;
};

template <bool WIDE>
__device__ __forceinline__ RowPos row_pos(const RowArgs& a, int upr) {
  RowPos p;
  if (WIDE) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    p.row = gid / upr;
    p.u = (int)(gid - p.row * upr);
    p.h = (int)(p.row % a.H);
    const int64_t t = p.row / a.H;
    p.s = (int)(t % a.S);
    p.b = t / a.S;
  } else {
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t row = gid / (uint32_t)upr;
    p.u = (int)(gid - row * (uint32_t)upr);
    const uint32_t t = row / (uint32_t)a.H;
    p.h = (int)(row - t * (uint32_t)a.H);
    const uint32_t bb = t / (uint32_t)a.S;
    p.s = (int)(t - bb * (uint32_t)a.S);
    p.row = row;
    p.b = bb;
  }
  return p;
}

// EPT elements per thread: 32 / EPT lanes per 32-element chunk, lane `sub` of a chunk holding
// elements sub * EPT .. +EPT of it.
template <typename T, bool NORM, bool ROPE, int FQ, int BLK, int EPT, bool WIDE>
__global__ __launch_bounds__(256) void row_pipeline_kernel(RowArgs a) {
  constexpr int L = 32 / EPT;
  static_assert(EPT % 8 == 0 && 32 % EPT == 0, "8, 16 or 32 elements per thread");
  const RowPos rp = row_pos<WIDE>(a, a.cpr * L);
  const int64_t row = rp.row, b = rp.b;
  const int c = rp.u / L, sub = rp.u - (rp.u / L) * L, h = rp.h, s = rp.s;
  const int e0 = c * 32 + sub * EPT;       // this thread's first element of the row
  if (row >= a.rows) return;  // whole rows leave together, so every lane group stays complete
  if (FQ == FQ_FP8_PACK && a.srb > 1 && (((a.tok_base + s) % a.srb == 0) != (a.phase == 0))) return;

  // rope factors of this thread's pairs, requested before the row itself so the two loads
  // overlap (a pair ahead of the tail reads the first entry and is left unrotated)
  const int first = a.dim - a.rd;
  const bool rope = ROPE && a.rd > 0 && e0 + EPT > first;   // the thread meets the rope tail
  float cs[EPT / 2], sn[EPT / 2];
  if (rope) {
    const int half = a.rd >> 1;
    const int64_t pos = (int64_t)a.pos_base + (int64_t)s * a.pos_step;
    const float* ct = a.cos_tab + pos * half;
    const float* st = a.sin_tab + pos * half;
#pragma unroll
    for (int j = 0; j < EPT / 2; ++j) {
      const int p = max(e0 + 2 * j - first, 0) >> 1;
      cs[j] = ct[p];
      sn[j] = st[p];
    }
  }
  float v[EPT];
  loadn<T, EPT>(reinterpret_cast<const T*>(a.src) + row * a.dim + e0, v);

  if (NORM) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) ss += v[i] * v[i];
    ss = group_sum(ss, a.cpr * L);
    const float inv = 1.0f / sqrtf(ss / (float)a.dim + a.eps);
    const float* w = a.norm_w + e0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) v[i] = io<T>::rnd(w[i] * (v[i] * inv));
  }
  if (rope) {
#pragma unroll
    for (int j = 0; j < EPT / 2; ++j) {
      if (e0 + 2 * j >= first) {
        rotate_pair(v[2 * j], v[2 * j + 1], cs[j], a.inverse ? -sn[j] : sn[j]);
        v[2 * j] = io<T>::rnd(v[2 * j]);
        v[2 * j + 1] = io<T>::rnd(v[2 * j + 1]);
      }
    }
  }
  if (FQ == FQ_FP4_MX) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) amax = fmaxf(amax, fabsf(v[i]));
    if constexpr (L > 1) amax = group_max(amax, L);
    uint32_t cw[EPT / 8];
    const uint32_t sc = mxfp4_encode<EPT>(v, amax, cw);
    uint8_t* cdst = reinterpret_cast<uint8_t*>(a.dst) + b * a.dst_bstride + (int64_t)(a.tok_base + s) * a.dst_tstride +
                    (int64_t)h * (a.dim / 2) + e0 / 2;
#pragma unroll
    for (int w = 0; w < EPT / 8; ++w) reinterpret_cast<uint32_t*>(cdst)[w] = cw[w];
    if (sub == 0)
      a.dst2[b * a.dst2_bstride + (int64_t)(a.tok_base + s) * a.dst2_tstride + (int64_t)h * (a.dim / 32) + c] =
          (uint8_t)sc;
    return;
  }
  if (FQ == FQ_FP8_PACK) {
    // fake_quant_fp8_ue8m0's scale and rounding (fake_quant_block, FQ_FP8_UE8M0), stored as codes
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) amax = fmaxf(amax, fabsf(v[i]));
    if constexpr (L > 1) amax = group_max(amax, L);
    amax = fmaxf(amax, 1e-4f);
    const int crow = a.tok_base + s;         // the cache row written
    uint8_t* sdst = a.dst2 + b * a.dst2_bstride + (int64_t)(a.srb > 1 ? crow / a.srb : crow) * a.dst2_tstride +
                    (int64_t)h * (a.dim / 32) + c;
    const bool opens = a.srb <= 1 || crow % a.srb == 0;
    const float sc = opens ? pow2_ceil_log2(amax * (float)(1.0 / 448.0)) : e8m0_to_float(*sdst);
    const float inv = __fdiv_rn(1.0f, sc);   // exact: sc is a power of two
    uint32_t cw[EPT / 4];
#pragma unroll
    for (int w = 0; w < EPT / 4; ++w) {
      uint32_t word = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        word |= (uint32_t)e4m3_encode(e4m3_round(fminf(fmaxf(v[4 * w + i] * inv, -448.0f), 448.0f))) << (8 * i);
      cw[w] = word;
    }
    uint8_t* cdst = reinterpret_cast<uint8_t*>(a.dst) + b * a.dst_bstride + (int64_t)(a.tok_base + s) * a.dst_tstride +
                    (int64_t)h * a.dim + e0;
#pragma unroll
    for (int w = 0; w < EPT / 8; ++w) reinterpret_cast<uint2*>(cdst)[w] = make_uint2(cw[2 * w], cw[2 * w + 1]);
    if (sub == 0 && opens) *sdst = (uint8_t)((__float_as_uint(sc) >> 23) & 0xFFu);
    return;
  }
  if (FQ == FQ_FP4_E4M3_PACK) {
    // fake_quant_fp4_e4m3's scale and rounding (fake_quant_block, FQ_FP4_E4M3) per 16 values,
    // stored as e2m1 codes (channel 2p in the low nibble of byte p) and the block's e4m3 scale
    constexpr int NB = EPT < 16 ? EPT : 16;  // this thread's values of one block
    uint8_t* rowp = reinterpret_cast<uint8_t*>(a.dst) + b * a.dst_bstride + (int64_t)(a.tok_base + s) * a.dst_tstride;
    uint32_t cw[EPT / 8];
#pragma unroll
    for (int w = 0; w < EPT / 8; ++w) cw[w] = 0u;
#pragma unroll
    for (int b0 = 0; b0 < EPT; b0 += NB) {
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < NB; ++i) amax = fmaxf(amax, fabsf(v[b0 + i]));
      if constexpr (NB < 16) amax = group_max(amax, 16 / NB);
      amax = fmaxf(amax, 0.01171875f);                           // 6 * 2^-9
      const float sc = e4m3_round(__fdiv_rn(amax, 6.0f));
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int e = b0 + i;
        cw[e / 8] |= e2m1_code(fminf(fmaxf(__fdiv_rn(v[e], sc), -6.0f), 6.0f)) << (4 * (e % 8));
      }
      if (NB == 16 || sub % (16 / NB) == 0) rowp[a.dim / 2 + (e0 + b0) / 16] = e4m3_encode(sc);
    }
    if constexpr (EPT == 8) {
      *reinterpret_cast<uint32_t*>(rowp + e0 / 2) = cw[0];
    } else {
#pragma unroll
      for (int w = 0; w < EPT / 8; w += 2) *reinterpret_cast<uint2*>(rowp + e0 / 2 + 4 * w) = make_uint2(cw[w], cw[w + 1]);
    }
    return;
  }
  if (FQ != FQ_NONE) {
    constexpr int NB = BLK < EPT ? BLK : EPT;  // this thread's values of one block
#pragma unroll
    for (int b0 = 0; b0 < EPT; b0 += NB) fake_quant_block<T, FQ, BLK, NB>(v + b0);
  }
  T* dst = reinterpret_cast<T*>(a.dst) + b * a.dst_bstride + (int64_t)(a.tok_base + s) * a.dst_tstride +
           (int64_t)h * a.dim + e0;
  storen<T, EPT>(dst, v);
}

template <typename T, bool NORM, bool ROPE, int FQ, int BLK, int EPT>
static int launch_rows_ept(const RowArgs& a, hipStream_t stream, const char* what) {
  const int64_t threads = a.rows * a.cpr * (32 / EPT);
  if (threads == 0) return 0;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks * 256 <= (int64_t)UINT32_MAX)
    hipLaunchKernelGGL((row_pipeline_kernel<T, NORM, ROPE, FQ, BLK, EPT, false>), dim3((unsigned)blocks), dim3(256),
                       0, stream, a);
  else
    hipLaunchKernelGGL((row_pipeline_kernel<T, NORM, ROPE, FQ, BLK, EPT, true>), dim3((unsigned)blocks), dim3(256),
                       0, stream, a);
  return check_launch(what);
}

// 8 elements per thread, unless a fused norm would need more than 64 lanes for one row
template <typename T, bool NORM, bool ROPE, int FQ, int BLK>
static int launch_rows(const RowArgs& a, hipStream_t stream, const char* what) {
  if (!NORM || a.cpr * 4 <= 64) return launch_rows_ept<T, NORM, ROPE, FQ, BLK, 8>(a, stream, what);
  return launch_rows_ept<T, NORM, ROPE, FQ, BLK, 32>(a, stream, what);
}

template <bool NORM, bool ROPE, int FQ, int BLK>
static int dispatch_rows(int dtype, const RowArgs& a, hipStream_t stream, const char* what) {
  if (dtype == DSV41_F32) return launch_rows<float, NORM, ROPE, FQ, BLK>(a, stream, what);
  if (dtype == DSV41_BF16) return launch_rows<bf16_t, NORM, ROPE, FQ, BLK>(a, stream, what);
  return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported (F32 or BF16)", what, dtype);
}

// Common shape checks. NORM needs the row's chunks in one power-of-two lane group.
static int check_rows(const char* what, const void* src, const void* dst, int64_t rows, int dim,
                      bool norm) {
  DSV41_REQUIRE(src && dst, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(aligned16(src) && aligned16(dst), DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  DSV41_REQUIRE(rows >= 0, DSV41_E_ARG, "%s: rows < 0", what);
  DSV41_REQUIRE(dim > 0 && dim % 32 == 0, DSV41_E_SHAPE, "%s: dim %d must be a positive multiple of 32", what, dim);
  if (norm)
    DSV41_REQUIRE(is_pow2(dim / 32) && dim / 32 <= 64, DSV41_E_SHAPE,
                  "%s: dim %d must be 32 * 2^k <= 2048 for the fused norm", what, dim);
  return 0;
}

static RowArgs plain_rows(const void* x, void* y, int64_t rows, int dim) {
  RowArgs a{};
  a.src = x; a.dst = y; a.rows = rows; a.dim = dim; a.cpr = dim / 32;
  a.S = 1; a.H = 1; a.dst_bstride = 0; a.dst_tstride = dim; a.tok_base = 0;
  // with S = H = 1 every row is its own batch row: b = row, so the batch stride is the row
  a.dst_bstride = dim;
  return a;
}

template <int FQ>
static int fq_entry(const char* what, const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                    int32_t dtype, hipStream_t stream) {
  int rc = check_rows(what, x, y, rows, cols, false);
  if (rc) return rc;
  DSV41_REQUIRE(block == 16 || block == 32, DSV41_E_SHAPE, "%s: block %d must be 16 or 32", what, block);
  // blocks never cross 32-element chunks, so the tensor is treated as chunks of one row each
  RowArgs a = plain_rows(x, y, rows * (cols / 32), 32);
  if (block == 32) return dispatch_rows<false, false, FQ, 32>(dtype, a, stream, what);
  return dispatch_rows<false, false, FQ, 16>(dtype, a, stream, what);
}

// ------------------------------------------------------------------ RMSNorm (any dim)

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* x, T* y, const float* w, int dim, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  x += row * dim;
  y += row * dim;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < dim; i += 256) {
    const float v = io<T>::ld(x + i);
    ss += v * v;
  }
  ss = group_sum(ss, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += 256) io<T>::st(y + i, w[i] * (io<T>::ld(x + i) * inv));
}

// Rows held in registers: one workgroup per row, thread t holding 16-byte chunks t, t + 256, ...
// (at most C of them), so the row is read once with full-width loads and scaled from registers.
// ADD: the residual add of a block first -- h <- cast(h + delta), stored back -- and the norm of
// the rounded sum, as the two separate ops compute it. The sum of squares is fp32, per thread,
// then the wave's xor tree and the four waves in a fixed order.
template <typename T, int C, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(T* x, const T* delta, T* y, const float* w, int dim,
                                                           float eps) {
  constexpr int E = 16 / (int)sizeof(T);       // elements per chunk
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int nch = dim / E;
  uint4* xr = reinterpret_cast<uint4*>(x + row * dim);
  float v[C][E];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      const uint4 u = xr[ch];
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int i = 0; i < E; ++i) v[c][i] = io<T>::ld(e + i);
      if constexpr (ADD) {
        const uint4 du = reinterpret_cast<const uint4*>(delta + row * dim)[ch];
        const T* de = reinterpret_cast<const T*>(&du);
        uint4 out;
        T* oe = reinterpret_cast<T*>(&out);
#pragma unroll
        for (int i = 0; i < E; ++i) {
          v[c][i] = io<T>::rnd(v[c][i] + io<T>::ld(de + i));
          io<T>::st(oe + i, v[c][i]);
        }
        xr[ch] = out;
      }
#pragma unroll
      for (int i = 0; i < E; ++i) ss += v[c][i] * v[c][i];
    }
  }
  ss = group_sum(ss, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
  uint4* yr = reinterpret_cast<uint4*>(y + row * dim);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      uint4 out;
      T* oe = reinterpret_cast<T*>(&out);
#pragma unroll
      for (int i = 0; i < E; ++i) io<T>::st(oe + i, w[ch * E + i] * (v[c][i] * inv));
      yr[ch] = out;
    }
  }
}

template <typename T, bool ADD>
static bool launch_rows_norm(T* x, const T* delta, T* y, const float* w, int64_t rows, int dim, float eps,
                             hipStream_t stream) {
  constexpr int E = 16 / (int)sizeof(T);
  if (dim % E || !aligned16(x) || !aligned16(y) || (ADD && !aligned16(delta))) return false;
  const int per = (dim / E + 255) / 256;     // chunks per thread
  const dim3 grid((unsigned)rows), block(256);
  switch (per) {
    case 1: hipLaunchKernelGGL((rmsnorm_rows_kernel<T, 1, ADD>), grid, block, 0, stream, x, delta, y, w, dim, eps); break;
    case 2: hipLaunchKernelGGL((rmsnorm_rows_kernel<T, 2, ADD>), grid, block, 0, stream, x, delta, y, w, dim, eps); break;
    case 3: hipLaunchKernelGGL((rmsnorm_rows_kernel<T, 3, ADD>), grid, block, 0, stream, x, delta, y, w, dim, eps); break;
    case 4: hipLaunchKernelGGL((rmsnorm_rows_kernel<T, 4, ADD>), grid, block, 0, stream, x, delta, y, w, dim, eps); break;
    default: return false;
  }
  return true;
}

// ------------------------------------------------------------------ rope table, ring, window idx

__global__ void rope_table_kernel(float* cs, float* sn, const float* freqs, int seqlen, int half) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)seqlen * half) return;
  const int t = (int)(i / half), j = (int)(i % half);
  const float ang = (float)t * freqs[j];
  cs[i] = cosf(ang);
  sn[i] = sinf(ang);
}

template <typename T>
__global__ void window_write_kernel(T* win, const T* kv, int n, int dim, int window, int start_pos, int keep,
                                    int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // over bsz*keep*dim
  if (i >= total) return;
  const int64_t per_b = (int64_t)keep * dim;
  const int64_t b = i / per_b;
  const int64_t r = i - b * per_b;
  const int t = (int)(r / dim), d = (int)(r % dim);
  const int slot = (int)(((int64_t)start_pos + n - keep + t) % window);
  win[(b * window + slot) * dim + d] = kv[(b * n + (n - keep + t)) * dim + d];
}

// window_write into an MXFP8 ring (rows of dim e4m3fn codes, then dim/32 ue8m0 scale bytes):
// 8 channels per thread, a 32-channel block per 4 consecutive lanes, quantized by
// fake_quant_fp8_ue8m0's formula -- exact for window KV that already holds that QAT's values.
template <typename T>
__global__ void window_write_mxfp8_kernel(uint8_t* ring, int64_t ring_bstride, const T* kv, int n, int dim, int window,
                                          int start_pos, int keep, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // over bsz*keep*(dim/8)
  if (i >= total) return;                       // total is a multiple of 4: block lanes stay together
  const int cpr = dim / 8;
  const int64_t row = i / cpr;
  const int c = (int)(i - row * cpr);
  const int64_t b = row / keep;
  const int t = (int)(row - b * keep);
  const int slot = (int)(((int64_t)start_pos + n - keep + t) % window);
  const T* src = kv + (b * n + (n - keep + t)) * (int64_t)dim + c * 8;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = io<T>::ld(src + j);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = fmaxf(group_max(amax, 4), 1e-4f);
  const float sc = pow2_ceil_log2(amax * (float)(1.0 / 448.0));
  const float inv = __fdiv_rn(1.0f, sc);        // exact: sc is a power of two
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; ++j)
    w[j / 4] |= (uint32_t)e4m3_encode(e4m3_round(fminf(fmaxf(v[j] * inv, -448.0f), 448.0f))) << (8 * (j % 4));
  uint8_t* dst = ring + b * ring_bstride + (int64_t)slot * (dim + dim / 32);
  *reinterpret_cast<uint2*>(dst + c * 8) = make_uint2(w[0], w[1]);
  if ((c & 3) == 0) dst[dim + c / 4] = (uint8_t)((__float_as_uint(sc) >> 23) & 0xFFu);
}

__global__ void window_idx_kernel(int32_t* out, int wp, int n, int window, int weff) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)n * weff) return;
  const int q = (int)(i / weff), j = (int)(i % weff);
  const int end = q + wp;
  const int start = max(end - window + 1, 0);
  const int idx = start + j;
  out[i] = idx > end ? -1 : idx;
}

}  // namespace dsv41

using namespace dsv41;

// ------------------------------------------------------------------ C ABI

extern "C" int dsv41_fq_fp8_ue8m0(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                                  int32_t dtype, hipStream_t stream) {
  return fq_entry<FQ_FP8_UE8M0>("dsv41_fq_fp8_ue8m0", x, y, rows, cols, block, dtype, stream);
}

extern "C" int dsv41_fq_fp4_ue8m0(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                                  int32_t dtype, hipStream_t stream) {
  return fq_entry<FQ_FP4_UE8M0>("dsv41_fq_fp4_ue8m0", x, y, rows, cols, block, dtype, stream);
}

extern "C" int dsv41_fq_fp4_e4m3(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                                 int32_t dtype, hipStream_t stream) {
  return fq_entry<FQ_FP4_E4M3>("dsv41_fq_fp4_e4m3", x, y, rows, cols, block, dtype, stream);
}

extern "C" int dsv41_rope_table(float* cos_out, float* sin_out, const float* freqs, int32_t seqlen,
                                int32_t half, hipStream_t stream) {
  const char* what = "dsv41_rope_table";
  DSV41_REQUIRE(cos_out && sin_out && freqs, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(seqlen >= 0 && half > 0, DSV41_E_ARG, "%s: bad sizes seqlen=%d half=%d", what, seqlen, half);
  const int64_t total = (int64_t)seqlen * half;
  if (total == 0) return 0;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, cos_out,
                     sin_out, freqs, seqlen, half);
  return check_launch(what);
}

extern "C" int dsv41_rope_tail(const void* x, void* y, int32_t bsz, int32_t seqlen, int32_t heads, int32_t dim,
                               int32_t rd, const float* cos_tab, const float* sin_tab, int32_t pos_base,
                               int32_t pos_step, int32_t inverse, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_rope_tail";
  DSV41_REQUIRE(bsz >= 0 && seqlen >= 0 && heads > 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, x, y, (int64_t)bsz * seqlen * heads, dim, false);
  if (rc) return rc;
  DSV41_REQUIRE(cos_tab && sin_tab, DSV41_E_ARG, "%s: null rope table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: rd %d must be even and <= dim", what, rd);
  DSV41_REQUIRE(pos_base >= 0 && (seqlen == 0 || (int64_t)pos_base + (int64_t)(seqlen - 1) * pos_step >= 0),
                DSV41_E_ARG, "%s: negative position", what);
  RowArgs a{};
  a.src = x; a.dst = y; a.rows = (int64_t)bsz * seqlen * heads; a.dim = dim; a.cpr = dim / 32;
  a.S = seqlen; a.H = heads; a.dst_bstride = (int64_t)seqlen * heads * dim; a.dst_tstride = (int64_t)heads * dim;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.pos_base = pos_base; a.pos_step = pos_step;
  a.inverse = inverse ? 1 : 0;
  return dispatch_rows<false, true, FQ_NONE, 32>(dtype, a, stream, what);
}

extern "C" int dsv41_rmsnorm(const void* x, void* y, const float* weight, int64_t rows, int32_t dim, float eps,
                             int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_rmsnorm";
  DSV41_REQUIRE(x && y && weight, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && dim > 0, DSV41_E_ARG, "%s: bad sizes", what);
  if (rows == 0) return 0;
  DSV41_REQUIRE(rows < (1ll << 31), DSV41_E_ARG, "%s: too many rows", what);
  // rows of up to 4 chunks of 16 bytes per thread take the register kernel (bf16 up to 8,192
  // channels, fp32 up to 4,096); others the strided one
  if (dtype == DSV41_F32) {
    if (!launch_rows_norm<float, false>((float*)const_cast<void*>(x), nullptr, (float*)y, weight, rows, dim, eps, stream))
      hipLaunchKernelGGL(rmsnorm_kernel<float>, dim3((unsigned)rows), dim3(256), 0, stream, (const float*)x,
                         (float*)y, weight, dim, eps);
  } else if (dtype == DSV41_BF16) {
    if (!launch_rows_norm<bf16_t, false>((bf16_t*)const_cast<void*>(x), nullptr, (bf16_t*)y, weight, rows, dim, eps,
                                         stream))
      hipLaunchKernelGGL(rmsnorm_kernel<bf16_t>, dim3((unsigned)rows), dim3(256), 0, stream, (const bf16_t*)x,
                         (bf16_t*)y, weight, dim, eps);
  } else {
    return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  }
  return check_launch(what);
}

extern "C" int dsv41_add_rmsnorm(void* h, const void* delta, void* y, const float* weight, int64_t rows, int32_t dim,
                                 float eps, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_add_rmsnorm";
  DSV41_REQUIRE(h && delta && y && weight, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && dim > 0, DSV41_E_ARG, "%s: bad sizes", what);
  if (rows == 0) return 0;
  DSV41_REQUIRE(rows < (1ll << 31), DSV41_E_ARG, "%s: too many rows", what);
  DSV41_REQUIRE(h != y && delta != y, DSV41_E_ARG, "%s: the output must not alias h or delta", what);
  bool ok;
  if (dtype == DSV41_F32)
    ok = launch_rows_norm<float, true>((float*)h, (const float*)delta, (float*)y, weight, rows, dim, eps, stream);
  else if (dtype == DSV41_BF16)
    ok = launch_rows_norm<bf16_t, true>((bf16_t*)h, (const bf16_t*)delta, (bf16_t*)y, weight, rows, dim, eps, stream);
  else
    return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  DSV41_REQUIRE(ok, DSV41_E_SHAPE, "%s: rows of %d elements (16-byte aligned, at most 1,024 16-byte chunks) required",
                what, dim);
  return check_launch(what);
}

extern "C" int dsv41_kv_window_prep(void* kv, const float* norm_w, const float* cos_tab, const float* sin_tab,
                                    int32_t bsz, int32_t n, int32_t dim, int32_t rd, int32_t start_pos, float eps,
                                    int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_kv_window_prep";
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, kv, kv, (int64_t)bsz * n, dim, true);
  if (rc) return rc;
  DSV41_REQUIRE(norm_w && cos_tab && sin_tab, DSV41_E_ARG, "%s: null weight/table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = kv; a.dst = kv; a.rows = (int64_t)bsz * n; a.dim = dim; a.cpr = dim / 32;
  a.S = n; a.H = 1; a.dst_bstride = (int64_t)n * dim; a.dst_tstride = dim;
  a.norm_w = norm_w; a.eps = eps; a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd;
  a.pos_base = start_pos; a.pos_step = 1;
  return dispatch_rows<true, true, FQ_FP8_UE8M0, 32>(dtype, a, stream, what);
}

extern "C" int dsv41_window_write(void* win_kv, const void* kv, int32_t bsz, int32_t n, int32_t dim,
                                  int32_t window, int32_t start_pos, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_window_write";
  DSV41_REQUIRE(win_kv && kv, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && dim > 0 && window > 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  const int keep = n < window ? n : window;
  const int64_t total = (int64_t)bsz * keep * dim;
  if (total == 0) return 0;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (dtype == DSV41_F32)
    hipLaunchKernelGGL(window_write_kernel<float>, dim3(blocks), dim3(256), 0, stream, (float*)win_kv,
                       (const float*)kv, n, dim, window, start_pos, keep, total);
  else if (dtype == DSV41_BF16)
    hipLaunchKernelGGL(window_write_kernel<bf16_t>, dim3(blocks), dim3(256), 0, stream, (bf16_t*)win_kv,
                       (const bf16_t*)kv, n, dim, window, start_pos, keep, total);
  else
    return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  return check_launch(what);
}

extern "C" int dsv41_window_write_mxfp8(uint8_t* win_kv8, int64_t ring_bstride, const void* kv, int32_t bsz,
                                        int32_t n, int32_t dim, int32_t window, int32_t start_pos, int32_t dtype,
                                        hipStream_t stream) {
  const char* what = "dsv41_window_write_mxfp8";
  DSV41_REQUIRE(win_kv8 && kv, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && window > 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dim > 0 && dim % 32 == 0, DSV41_E_SHAPE, "%s: dim %d must be a positive multiple of 32", what, dim);
  DSV41_REQUIRE(ring_bstride >= (int64_t)window * (dim + dim / 32), DSV41_E_ARG, "%s: ring too small", what);
  DSV41_REQUIRE(ring_bstride % 8 == 0 && (dim + dim / 32) % 8 == 0, DSV41_E_ARG,
                "%s: rows and the batch stride must be multiples of 8 bytes", what);
  DSV41_REQUIRE((reinterpret_cast<uintptr_t>(win_kv8) & 7u) == 0 && aligned16(kv), DSV41_E_ARG,
                "%s: misaligned tensor", what);
  const int keep = n < window ? n : window;
  const int64_t total = (int64_t)bsz * keep * (dim / 8);
  if (total == 0) return 0;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (dtype == DSV41_F32)
    hipLaunchKernelGGL(window_write_mxfp8_kernel<float>, dim3(blocks), dim3(256), 0, stream, win_kv8, ring_bstride,
                       (const float*)kv, n, dim, window, start_pos, keep, total);
  else if (dtype == DSV41_BF16)
    hipLaunchKernelGGL(window_write_mxfp8_kernel<bf16_t>, dim3(blocks), dim3(256), 0, stream, win_kv8, ring_bstride,
                       (const bf16_t*)kv, n, dim, window, start_pos, keep, total);
  else
    return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  return check_launch(what);
}

extern "C" int dsv41_window_idx(int32_t* out, int32_t wp, int32_t n, int32_t window, hipStream_t stream) {
  const char* what = "dsv41_window_idx";
  DSV41_REQUIRE(out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(wp >= 0 && n >= 0 && window > 0, DSV41_E_ARG, "%s: bad sizes", what);
  const int weff = window < wp + n ? window : wp + n;
  const int64_t total = (int64_t)n * weff;
  if (total == 0) return 0;
  hipLaunchKernelGGL(window_idx_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, out, wp, n,
                     window, weff);
  return check_launch(what);
}

// The compressed-cache write (attention.py:157-163) stored packed: rope(latent), then
// fake_quant_fp4_e4m3's e2m1 codes and e4m3 scales per 16 channels, one row of dim/2 + dim/16
// bytes per group (codes first), cache_bstride bytes per batch row.
extern "C" int dsv41_comp_write_fp4(const void* latents, uint8_t* comp_kv4, int64_t cache_bstride,
                                    const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g, int32_t dim,
                                    int32_t rd, int32_t g0, int32_t ratio, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_comp_write_fp4";
  DSV41_REQUIRE(bsz >= 0 && g >= 0 && g0 >= 0 && ratio > 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, latents, comp_kv4, (int64_t)bsz * g, dim, false);
  if (rc) return rc;
  const int64_t row = dim / 2 + dim / 16;
  DSV41_REQUIRE(cache_bstride >= (int64_t)(g0 + g) * row, DSV41_E_ARG, "%s: cache too small", what);
  DSV41_REQUIRE(cache_bstride % 16 == 0 && row % 16 == 0, DSV41_E_ARG,
                "%s: rows and the batch stride must be multiples of 16 bytes", what);
  DSV41_REQUIRE(cos_tab && sin_tab, DSV41_E_ARG, "%s: null rope table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = latents; a.dst = comp_kv4; a.rows = (int64_t)bsz * g; a.dim = dim; a.cpr = dim / 32;
  a.S = g; a.H = 1; a.dst_bstride = cache_bstride; a.dst_tstride = row; a.tok_base = g0;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.pos_base = g0 * ratio; a.pos_step = ratio;
  return dispatch_rows<false, true, FQ_FP4_E4M3_PACK, 16>(dtype, a, stream, what);
}

extern "C" int dsv41_comp_write(const void* latents, void* comp_kv, int64_t cache_bstride, const float* cos_tab,
                                const float* sin_tab, int32_t bsz, int32_t g, int32_t dim, int32_t rd, int32_t g0,
                                int32_t ratio, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_comp_write";
  DSV41_REQUIRE(bsz >= 0 && g >= 0 && g0 >= 0 && ratio > 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, latents, comp_kv, (int64_t)bsz * g, dim, false);
  if (rc) return rc;
  DSV41_REQUIRE(cache_bstride >= (int64_t)(g0 + g) * dim, DSV41_E_ARG, "%s: cache too small", what);
  DSV41_REQUIRE(cos_tab && sin_tab, DSV41_E_ARG, "%s: null rope table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = latents; a.dst = comp_kv; a.rows = (int64_t)bsz * g; a.dim = dim; a.cpr = dim / 32;
  a.S = g; a.H = 1; a.dst_bstride = cache_bstride; a.dst_tstride = dim; a.tok_base = g0;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.pos_base = g0 * ratio; a.pos_step = ratio;
  return dispatch_rows<false, true, FQ_FP4_E4M3, 16>(dtype, a, stream, what);
}

extern "C" int dsv41_index_key_publish(const void* k_raw, void* index_k, int64_t cache_bstride, const float* norm_w,
                                       const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                                       int32_t dim, int32_t rd, int32_t g0, int32_t ratio, float eps,
                                       int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_index_key_publish";
  DSV41_REQUIRE(bsz >= 0 && g >= 0 && g0 >= 0 && ratio > 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, k_raw, index_k, (int64_t)bsz * g, dim, true);
  if (rc) return rc;
  DSV41_REQUIRE(cache_bstride >= (int64_t)(g0 + g) * dim, DSV41_E_ARG, "%s: cache too small", what);
  DSV41_REQUIRE(norm_w && cos_tab && sin_tab, DSV41_E_ARG, "%s: null weight/table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = k_raw; a.dst = index_k; a.rows = (int64_t)bsz * g; a.dim = dim; a.cpr = dim / 32;
  a.S = g; a.H = 1; a.dst_bstride = cache_bstride; a.dst_tstride = dim; a.tok_base = g0;
  a.norm_w = norm_w; a.eps = eps; a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd;
  a.pos_base = g0 * ratio; a.pos_step = ratio;
  return dispatch_rows<true, true, FQ_FP4_UE8M0, 32>(dtype, a, stream, what);
}

extern "C" int dsv41_index_key_publish_mxfp4(const void* k_raw, uint8_t* k_codes, int64_t kc_bstride,
                                             uint8_t* k_scales, int64_t ks_bstride, const float* norm_w,
                                             const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                                             int32_t dim, int32_t rd, int32_t g0, int32_t ratio, float eps,
                                             int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_index_key_publish_mxfp4";
  DSV41_REQUIRE(bsz >= 0 && g >= 0 && g0 >= 0 && ratio > 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, k_raw, k_codes, (int64_t)bsz * g, dim, true);
  if (rc) return rc;
  DSV41_REQUIRE(k_scales, DSV41_E_ARG, "%s: null scale cache", what);
  DSV41_REQUIRE(kc_bstride >= (int64_t)(g0 + g) * (dim / 2) && ks_bstride >= (int64_t)(g0 + g) * (dim / 32),
                DSV41_E_ARG, "%s: cache too small", what);
  DSV41_REQUIRE(kc_bstride % 16 == 0, DSV41_E_ARG, "%s: kc_bstride must be a multiple of 16 bytes", what);
  DSV41_REQUIRE(norm_w && cos_tab && sin_tab, DSV41_E_ARG, "%s: null weight/table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = k_raw; a.dst = k_codes; a.rows = (int64_t)bsz * g; a.dim = dim; a.cpr = dim / 32;
  a.S = g; a.H = 1; a.dst_bstride = kc_bstride; a.dst_tstride = dim / 2; a.tok_base = g0;
  a.dst2 = k_scales; a.dst2_bstride = ks_bstride; a.dst2_tstride = dim / 32;
  a.norm_w = norm_w; a.eps = eps; a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd;
  a.pos_base = g0 * ratio; a.pos_step = ratio;
  return dispatch_rows<true, true, FQ_FP4_MX, 32>(dtype, a, stream, what);
}

// Shared checks and set-up of the packed fp8 writers: codes [bsz, >=g0+g, dim] and scales
// [bsz, >=ceil((g0+g)/scale_rb), dim/32] bytes, batch strides in bytes, one scale per 32 channels
// of every scale_rb rows. With scale_rb = 32 a row that opens a 32-row block sets the block's
// scale and the block's later rows are rounded with it.
static int fp8_rows(const char* what, const void* src, uint8_t* codes, int64_t c_bstride, uint8_t* scales,
                    int64_t s_bstride, int32_t scale_rb, int32_t bsz, int32_t g, int32_t dim, int32_t rd, int32_t g0,
                    int32_t ratio, bool norm, RowArgs* a) {
  DSV41_REQUIRE(bsz >= 0 && g >= 0 && g0 >= 0 && ratio > 0, DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(scale_rb == 1 || scale_rb == 32, DSV41_E_ARG, "%s: scale row block must be 1 or 32", what);
  int rc = check_rows(what, src, codes, (int64_t)bsz * g, dim, norm);
  if (rc) return rc;
  DSV41_REQUIRE(scales, DSV41_E_ARG, "%s: null scale cache", what);
  DSV41_REQUIRE(c_bstride >= (int64_t)(g0 + g) * dim &&
                    s_bstride >= (int64_t)((g0 + g + scale_rb - 1) / scale_rb) * (dim / 32),
                DSV41_E_ARG, "%s: cache too small", what);
  DSV41_REQUIRE(c_bstride % 16 == 0, DSV41_E_ARG, "%s: code batch stride must be a multiple of 16 bytes", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  a->src = src; a->dst = codes; a->rows = (int64_t)bsz * g; a->dim = dim; a->cpr = dim / 32;
  a->S = g; a->H = 1; a->dst_bstride = c_bstride; a->dst_tstride = dim; a->tok_base = g0;
  a->dst2 = scales; a->dst2_bstride = s_bstride; a->dst2_tstride = dim / 32; a->srb = scale_rb;
  a->rd = rd; a->pos_base = g0 * ratio; a->pos_step = ratio;
  return 0;
}

// The packed fp8 store of rows [g0, g0+g): one launch with per-row scales; with 32-row scale
// blocks the rows that open a block first (they set its scale), then the others.
template <bool NORM>
static int fp8_store(const char* what, RowArgs a, int32_t g0, int32_t g, int32_t dtype, hipStream_t stream) {
  if (a.srb <= 1) return dispatch_rows<NORM, true, FQ_FP8_PACK, 32>(dtype, a, stream, what);
  const int first_open = (g0 + a.srb - 1) / a.srb, last_open = (g0 + g - 1) / a.srb;   // blocks opened here
  const int openers = g > 0 ? last_open - first_open + 1 : 0;
  if (openers > 0) {
    a.phase = 0;
    const int rc = dispatch_rows<NORM, true, FQ_FP8_PACK, 32>(dtype, a, stream, what);
    if (rc) return rc;
  }
  if (g > openers) {
    a.phase = 1;
    return dispatch_rows<NORM, true, FQ_FP8_PACK, 32>(dtype, a, stream, what);
  }
  return 0;
}

extern "C" int dsv41_comp_write_fp8(const void* latents, uint8_t* codes, int64_t c_bstride, uint8_t* scales,
                                    int64_t s_bstride, int32_t scale_rb, const float* cos_tab, const float* sin_tab,
                                    int32_t bsz, int32_t g, int32_t dim, int32_t rd, int32_t g0, int32_t ratio,
                                    int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_comp_write_fp8";
  RowArgs a{};
  int rc = fp8_rows(what, latents, codes, c_bstride, scales, s_bstride, scale_rb, bsz, g, dim, rd, g0, ratio, false,
                    &a);
  if (rc) return rc;
  DSV41_REQUIRE(cos_tab && sin_tab, DSV41_E_ARG, "%s: null rope table", what);
  a.cos_tab = cos_tab; a.sin_tab = sin_tab;
  return fp8_store<false>(what, a, g0, g, dtype, stream);
}

extern "C" int dsv41_index_key_publish_fp8(const void* k_raw, uint8_t* codes, int64_t c_bstride, uint8_t* scales,
                                           int64_t s_bstride, int32_t scale_rb, const float* norm_w,
                                           const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                                           int32_t dim, int32_t rd, int32_t g0, int32_t ratio, float eps,
                                           int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_index_key_publish_fp8";
  RowArgs a{};
  int rc = fp8_rows(what, k_raw, codes, c_bstride, scales, s_bstride, scale_rb, bsz, g, dim, rd, g0, ratio, true,
                    &a);
  if (rc) return rc;
  DSV41_REQUIRE(norm_w && cos_tab && sin_tab, DSV41_E_ARG, "%s: null weight/table", what);
  a.norm_w = norm_w; a.eps = eps; a.cos_tab = cos_tab; a.sin_tab = sin_tab;
  return fp8_store<true>(what, a, g0, g, dtype, stream);
}

extern "C" int dsv41_index_q_prep_mxfp4(const void* q, uint8_t* q_codes, uint8_t* q_scales, const float* cos_tab,
                                        const float* sin_tab, int32_t bsz, int32_t n, int32_t heads, int32_t dim,
                                        int32_t rd, int32_t start_pos, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_index_q_prep_mxfp4";
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, q, q_codes, (int64_t)bsz * n * heads, dim, false);
  if (rc) return rc;
  DSV41_REQUIRE(q_scales && cos_tab && sin_tab, DSV41_E_ARG, "%s: null scales or rope table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = q; a.dst = q_codes; a.rows = (int64_t)bsz * n * heads; a.dim = dim; a.cpr = dim / 32;
  a.S = n; a.H = heads;
  a.dst_bstride = (int64_t)n * heads * (dim / 2); a.dst_tstride = (int64_t)heads * (dim / 2);
  a.dst2 = q_scales; a.dst2_bstride = (int64_t)n * heads * (dim / 32); a.dst2_tstride = (int64_t)heads * (dim / 32);
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.pos_base = start_pos; a.pos_step = 1;
  return dispatch_rows<false, true, FQ_FP4_MX, 32>(dtype, a, stream, what);
}

extern "C" int dsv41_index_q_prep(void* q, const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t n,
                                  int32_t heads, int32_t dim, int32_t rd, int32_t start_pos, int32_t dtype,
                                  hipStream_t stream) {
  const char* what = "dsv41_index_q_prep";
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && start_pos >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  int rc = check_rows(what, q, q, (int64_t)bsz * n * heads, dim, false);
  if (rc) return rc;
  DSV41_REQUIRE(cos_tab && sin_tab, DSV41_E_ARG, "%s: null rope table", what);
  DSV41_REQUIRE(rd > 0 && rd % 2 == 0 && rd <= dim, DSV41_E_SHAPE, "%s: bad rd %d", what, rd);
  RowArgs a{};
  a.src = q; a.dst = q; a.rows = (int64_t)bsz * n * heads; a.dim = dim; a.cpr = dim / 32;
  a.S = n; a.H = heads; a.dst_bstride = (int64_t)n * heads * dim; a.dst_tstride = (int64_t)heads * dim;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.pos_base = start_pos; a.pos_step = 1;
  return dispatch_rows<false, true, FQ_FP4_UE8M0, 32>(dtype, a, stream, what);
}
