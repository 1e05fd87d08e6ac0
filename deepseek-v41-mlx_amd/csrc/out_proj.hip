// The grouped block-diagonal output LoRA of Attention.__call__ (attention.py:176-179):
//
//   out[m, g*r + j] = sum_k o[m, g*d + k] * wo_a[g*r + j, k]
//
// o is the attention output [rows, groups*d] (bf16, inverse rope applied), wo_a the Linear weight
// [groups*r, d] (bf16, unquantized), out [rows, groups*r]. The reference computes the einsum on
// fp32 copies of both and casts the result to the activation dtype before wo_b. Here every
// product of two bf16 values is exact in the MFMA and the sums are fp32 (the MFMA's own
// accumulation over the channels in order), so the result differs from the reference's only in the
// order of the fp32 additions; the bf16 output is the fp32 value rounded to nearest even once, as
// astype does.
//
// Launch shapes (bf16 o and wo_a with d a multiple of 64 and r of 128 -- the release's 4096 and
// 1024 -- take the MFMA kernel; other shapes and fp32 activations take a plain fp32 kernel). Both
// operand tiles are copied global -> LDS (global_load_lds_dwordx4) over 64-channel steps in an
// XOR-swizzled layout that the MFMA fragment reads take without bank conflicts:
//   decode (rows <= 128): the weight is streamed from HBM once. A workgroup owns 32 weight rows
//     of one group and every query row (32-row tiles); its four waves each own a 16 x 32 or
//     16 x 16 block of the output, and the copies run eight steps ahead (a 64-128 KB ring), which
//     is what keeps enough of the stream in flight: 256 workgroups for 8 x 1024, one per CU, the
//     workgroups of one group on one XCD so that they share its L2 copy of o.
//   prefill: 256 x 256 output tiles (weight rows x query rows), double-buffered; eight waves of
//     128 x 64 each, two per SIMD (128 x 128 tiles of four 64 x 64 waves when r is not a
//     multiple of 256).
#include "mfma.h"

namespace dsv41 {

struct WoaArgs {
  const bf16_t* o;     // [rows, groups * d]
  const bf16_t* w;     // [groups * r, d]; split: [r, groups * d]
  void* out;           // [rows, groups * r], bf16 or fp32
  int rows, groups, d, r;
  int split;           // 1: one dense weight whose contraction is cut into `groups` ranges of d
  const bf16_t* w1;    // split only: weight rows [r0, r) come from w1 [r - r0, groups * d]
  int r0;              // (two weights applied to the same rows; r0 a multiple of the tile's rows)
};

// ------------------------------------------------------------------ any shape

// One thread per output: the d products of one row of o and one weight row, summed in fp32 in
// channel order (products of bf16 values are exact; fp32 ones round). For the shapes and dtypes
// the MFMA kernels do not take (small test configurations, fp32 activations).
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void wo_a_plain_kernel(const TI* o, const TI* w, TO* out, int rows, int groups,
                                                          int d, int r) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;      // over rows * groups * r
  if (i >= (int64_t)rows * groups * r) return;
  const int64_t gr = (int64_t)groups * r;
  const int64_t m = i / gr;
  const int gj = (int)(i - m * gr), grp = gj / r;
  const TI* op = o + m * groups * d + (int64_t)grp * d;
  const TI* wp = w + (int64_t)gj * d;
  float acc = 0.0f;
  for (int k = 0; k < d; ++k) acc += io<TI>::ld(op + k) * io<TI>::ld(wp + k);
  io<TO>::st(out + i, acc);
}

// Four consecutive outputs of one query row.
template <typename TO>
__device__ __forceinline__ void store4(TO* p, f32x4 v);
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* p, f32x4 v) {
  uint2 s;
  s.x = pack2_bf16(v[0], v[1]);
  s.y = pack2_bf16(v[2], v[3]);
  *reinterpret_cast<uint2*>(p) = s;
}
template <>
__device__ __forceinline__ void store4<float>(float* p, f32x4 v) {
  *reinterpret_cast<f32x4*>(p) = v;
}

// ------------------------------------------------------------------ tiled (every row count)

constexpr int kTileR = 128;   // weight rows of the smallest output tile (r is a multiple of it)
constexpr int kWideR = 256;   // weight rows of the large tile

// 16-byte chunk c of tile row `row` (rows of BK bf16: BK / 8 chunks) sits at slot c ^ swz(row).
// A fragment read takes one chunk of 16 consecutive rows; with these slots no two of those lanes
// share a bank, whether the banks serve 8 lanes of 16 bytes (128 bytes) per cycle or 16 lanes
// (256 bytes).
template <int BK>
__device__ __forceinline__ int tile_swz(int row) {
  if constexpr (BK == 64) return (row & 7) ^ ((row >> 3) & 1);
  else return ((row >> 1) & 3) ^ ((row >> 3) & 1);
}

// Output tile of 16 WR GR weight rows x 16 WM GM query rows: a GR x GM grid of waves, each
// 16 WR x 16 WM (WR x WM MFMA tiles). BK channels per step; NS steps of both operand tiles in LDS
// at once (NS - 1 in flight while one is multiplied).
template <int WR, int WM, int GR, int GM, int BK, int NS>
struct TileCfg {
  static constexpr int NWV = GR * GM, NT = 64 * NWV;
  static constexpr int TR = 16 * WR * GR, TM = 16 * WM * GM;
  static constexpr int RB = BK * 2;                 // bytes per tile row
  static constexpr int CPR = BK / 8;                // 16-byte chunks per row
  static constexpr int RPI = 1024 / RB;             // rows per copy instruction
  static constexpr int NW = TR * RB / (1024 * NWV), NO = TM * RB / (1024 * NWV);   // copies per wave per step
  static constexpr int STAGE = (TR + TM) * RB;
  static constexpr int LDS = NS * STAGE;
  static_assert(BK == 32 || BK == 64, "32- or 64-channel steps");
  static_assert(NW * 1024 * NWV == TR * RB && NO * 1024 * NWV == TM * RB, "whole copy instructions per wave");
};

// The same for deep rings: at most `pending` (clamped to P) later steps of N copies each may
// stay in flight; N * P stays within the 6-bit vmcnt field.
template <int N, int P>
__device__ __forceinline__ void wait_copies_deep(int pending) {
  static_assert(N * P <= 63, "vmcnt holds 6 bits");
  if constexpr (P > 0) {
    if (pending >= P) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N * P) : "memory");
      return;
    }
    wait_copies_deep<N, P - 1>(pending);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

template <int N>
__device__ __forceinline__ void wait_copies(int pending) {
  // at most `pending` later steps of per_step copies each may stay in flight
  if constexpr (N >= 3) {
    if (pending >= 3) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * N) : "memory");
      return;
    }
  }
  if constexpr (N >= 2) {
    if (pending == 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * N) : "memory");
      return;
    }
  }
  if (pending >= 1) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
    return;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int WR, int WM, int GR, int GM, int BK, int NS, typename TO>
__global__ __launch_bounds__(64 * GR * GM, (TileCfg<WR, WM, GR, GM, BK, NS>::LDS <= 80 * 1024) ? 2 : 1) void wo_a_tiles_kernel(
    WoaArgs a) {
  using C = TileCfg<WR, WM, GR, GM, BK, NS>;
  __shared__ __align__(16) uint8_t lds[C::LDS];   // NS x [weight tile][query tile]
  const int mtiles = (a.rows + C::TM - 1) / C::TM, rtiles = a.r / C::TR;
  // consecutive tiles on one XCD, the weight tile fastest: the rtiles workgroups that read one
  // query tile share that XCD's L2
  const int total = (int)gridDim.x;
  const int tile = total % 8 ? (int)blockIdx.x : ((int)blockIdx.x % 8) * (total / 8) + (int)blockIdx.x / 8;
  const int rt = tile % rtiles, mt = (tile / rtiles) % mtiles, grp = tile / (rtiles * mtiles);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const int wr = (wave % GR) * 16 * WR, wm = (wave / GR) * 16 * WM;   // this wave's block

  // copy sources: wave w fills rows [w TR/NWV, (w+1) TR/NWV) of the weight tile and [w TM/NWV, ..)
  // of the query tile, RPI rows per instruction; lane l writes slot l % CPR of row l / CPR of its
  // instruction's rows, i.e. chunk slot ^ swz(row) of that row
  uint64_t wsrc[C::NW], osrc[C::NO];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    const int row = wave * (C::TR / C::NWV) + j * C::RPI + lane / C::CPR;
    const int chunk = (lane % C::CPR) ^ tile_swz<BK>(row);
    // grouped: group grp's weight rows; split: range grp of every weight row (row stride groups * d),
    // rows from r0 on in w1 when it is given
    const int wr_all = rt * C::TR + row;
    const bool second = a.w1 != nullptr && wr_all >= a.r0;
    const bf16_t* wbase = second ? a.w1 : a.w;
    const int64_t wrow = a.split ? (int64_t)(second ? wr_all - a.r0 : wr_all) * ((int64_t)a.groups * a.d) + (int64_t)grp * a.d
                                 : ((int64_t)grp * a.r + wr_all) * a.d;
    wsrc[j] = reinterpret_cast<uint64_t>(wbase + wrow + 8 * chunk);
  }
#pragma unroll
  for (int j = 0; j < C::NO; ++j) {
    const int row = wave * (C::TM / C::NWV) + j * C::RPI + lane / C::CPR;
    const int chunk = (lane % C::CPR) ^ tile_swz<BK>(row);
    const int64_t orow = min(mt * C::TM + row, a.rows - 1);   // rows past the end: not stored
    osrc[j] = reinterpret_cast<uint64_t>(a.o + orow * a.groups * a.d + (int64_t)grp * a.d + 8 * chunk);
  }
  const uint32_t lds0 = lds_offset(lds);
  auto issue = [&](int buf, int k) {
    const uint32_t wdst = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(lds0 + (uint32_t)(buf * C::STAGE) + (uint32_t)(wave * (C::TR / C::NWV) * C::RB)));   // wave-uniform: M0
    const uint32_t odst = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(lds0 + (uint32_t)(buf * C::STAGE + C::TR * C::RB) + (uint32_t)(wave * (C::TM / C::NWV) * C::RB)));
    const uint64_t kb = (uint64_t)k * 2;
#pragma unroll
    for (int j = 0; j < C::NW; ++j) dma16_vaddr(wsrc[j] + kb, wdst + j * 1024);
#pragma unroll
    for (int j = 0; j < C::NO; ++j) dma16_vaddr(osrc[j] + kb, odst + j * 1024);
  };
  auto frag = [&](const uint8_t* t, int row, int chunk) {
    return as_bf16x8(*reinterpret_cast<const uint4*>(t + row * C::RB + ((chunk ^ tile_swz<BK>(row)) << 4)));
  };

  f32x4 acc[WR][WM];
#pragma unroll
  for (int i = 0; i < WR; ++i)
#pragma unroll
    for (int j = 0; j < WM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One barrier per step: after it, step kt is in LDS for every wave and every wave is done with
  // step kt - 1, whose buffer then takes step kt + NS - 1.
  const int nk = a.d / BK;
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nk) issue(p, p * BK);
  for (int kt = 0; kt < nk; ++kt) {
    if constexpr (NS <= 4) wait_copies<C::NW + C::NO>(min(NS - 2, nk - 1 - kt));   // this wave's copies of step kt landed
    else wait_copies_deep<C::NW + C::NO, NS - 2>(min(NS - 2, nk - 1 - kt));
    __syncthreads();
    if (kt + NS - 1 < nk) issue((kt + NS - 1) % NS, (kt + NS - 1) * BK);
    const uint8_t* wt = lds + (kt % NS) * C::STAGE;
    const uint8_t* qt = wt + C::TR * C::RB;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[WR], bf[WM];
#pragma unroll
      for (int i = 0; i < WR; ++i) af[i] = frag(wt, wr + 16 * i + l16, 4 * ks + g);
#pragma unroll
      for (int j = 0; j < WM; ++j) bf[j] = frag(qt, wm + 16 * j + l16, 4 * ks + g);
#pragma unroll
      for (int i = 0; i < WR; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
    }
  }

  const int64_t ostride = (int64_t)a.groups * a.r;
  TO* out = reinterpret_cast<TO*>(a.out);
#pragma unroll
  for (int j = 0; j < WM; ++j) {
    const int m = mt * C::TM + wm + 16 * j + l16;
    if (m >= a.rows) continue;
#pragma unroll
    for (int i = 0; i < WR; ++i)
      store4<TO>(out + m * ostride + (int64_t)grp * a.r + rt * C::TR + wr + 16 * i + 4 * g, acc[i][j]);
  }
}

template <int WR, int WM, int GR, int GM, int BK, int NS, typename TO>
static void launch_tiles(const WoaArgs& a, hipStream_t stream) {
  using C = TileCfg<WR, WM, GR, GM, BK, NS>;
  const int64_t tiles = (int64_t)a.groups * (a.r / C::TR) * ((a.rows + C::TM - 1) / C::TM);
  hipLaunchKernelGGL((wo_a_tiles_kernel<WR, WM, GR, GM, BK, NS, TO>), dim3((unsigned)tiles), dim3(C::NT), 0, stream, a);
}

// Split contraction at 33-64 query rows: 128- or 160-row weight tiles where each range is long
// (>= 1024 channels) and the tiles fill the chip once (128-256 workgroups; of the two, the one with
// more workgroups). A 32-row tile reads the 64 query rows from L2 for every 32 weight rows it
// streams, twice the weight's bytes; a 128-row one half of them (measured at 64 rows: wq_b
// 1280 -> 32768 19.1 us against 21.5 for hipBLASLt; wo_b 8192 -> 5120 in 4 ranges on 128-row tiles
// 26.5 us, 160 workgroups, and in 8 ranges on 160-row tiles 23.4-23.8 us, 256 workgroups, against
// 29.6-30.1 for hipBLASLt; 32-row tiles 32.8 us). Returns the tile's weight rows, 0 for none.
__host__ __device__ inline int wide_split_tile(int rows, int d, int n, int ranges) {
  if (rows <= 32 || rows > 64 || d < 1024) return 0;
  int best = 0;
  int64_t best_t = 0;
  for (int tr = 128; tr <= 160; tr += 32) {
    const int64_t t = (int64_t)(n / tr) * ranges;
    if (n % tr == 0 && t >= 128 && t <= 256 && t > best_t) {
      best = tr;
      best_t = t;
    }
  }
  return best;
}

template <typename TO>
static void launch_wo_a(const WoaArgs& a, hipStream_t stream) {
  // decode: 32 weight rows x every query row per workgroup (groups * r / 32 workgroups), an
  // eight-stage copy ring (four at 128 rows, whose stage is 20 KB)
  if (a.rows <= 128) {
    const int64_t tiles = (int64_t)a.groups * (a.r / 32);
    const int wide = a.split ? wide_split_tile(a.rows, a.d, a.r, a.groups) : 0;
    if (wide && (a.w1 == nullptr || a.r0 % wide == 0)) {
      if (wide == 160) launch_tiles<5, 2, 2, 2, 64, 4, TO>(a, stream);   // 160 x 64 tiles, 112 KB
      else launch_tiles<4, 2, 2, 2, 64, 4, TO>(a, stream);               // 128 x 64 tiles, 96 KB
      return;
    }
    switch ((a.rows + 31) / 32) {
      case 1: launch_tiles<1, 1, 2, 2, 64, 8, TO>(a, stream); break;
      case 2:
        if (tiles > 256) launch_tiles<1, 2, 2, 2, 64, 6, TO>(a, stream);   // 72 KB: two per CU
        else launch_tiles<1, 2, 2, 2, 64, 8, TO>(a, stream);
        break;
      case 3: launch_tiles<1, 3, 2, 2, 64, 8, TO>(a, stream); break;
      default: launch_tiles<1, 4, 2, 2, 64, 4, TO>(a, stream); break;
    }
    return;
  }
  if (a.r % kWideR == 0) launch_tiles<8, 4, 2, 4, 64, 2, TO>(a, stream);
  else launch_tiles<4, 4, 2, 2, 64, 2, TO>(a, stream);
}

}  // namespace dsv41

using namespace dsv41;

template <typename TI>
static int launch_wo_a_plain(const void* o, const void* w, void* out, int rows, int groups, int d, int r,
                             int out_dtype, hipStream_t stream) {
  const int64_t n = (int64_t)rows * groups * r;
  const dim3 grid((unsigned)((n + 255) / 256));
  const TI* oi = static_cast<const TI*>(o);
  const TI* wi = static_cast<const TI*>(w);
  if (out_dtype == DSV41_BF16)
    hipLaunchKernelGGL((wo_a_plain_kernel<TI, bf16_t>), grid, dim3(256), 0, stream, oi, wi,
                       static_cast<bf16_t*>(out), rows, groups, d, r);
  else
    hipLaunchKernelGGL((wo_a_plain_kernel<TI, float>), grid, dim3(256), 0, stream, oi, wi, static_cast<float*>(out),
                       rows, groups, d, r);
  return 0;
}

extern "C" int dsv41_wo_a_grouped(const void* o, const void* wo_a, void* out, int32_t rows, int32_t groups,
                                  int32_t d, int32_t r, int32_t dtype, int32_t out_dtype, hipStream_t stream) {
  const char* what = "dsv41_wo_a_grouped";
  DSV41_REQUIRE(o && wo_a && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && groups > 0 && d > 0 && r > 0, DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dtype == DSV41_BF16 || dtype == DSV41_F32, DSV41_E_DTYPE, "%s: dtype %d not supported (BF16 or F32)",
                what, dtype);
  DSV41_REQUIRE(out_dtype == DSV41_BF16 || out_dtype == DSV41_F32, DSV41_E_DTYPE,
                "%s: out dtype %d not supported (BF16 or F32)", what, out_dtype);
  DSV41_REQUIRE(aligned16(o) && aligned16(wo_a) && aligned16(out), DSV41_E_ARG, "%s: tensors must be 16-byte aligned",
                what);
  DSV41_REQUIRE((int64_t)groups * r * d < (1ll << 40) && (int64_t)rows * groups * (d > r ? d : r) < (1ll << 40),
                DSV41_E_ARG, "%s: tensors too large", what);
  if (rows == 0) return 0;
  const bool mfma = dtype == DSV41_BF16 && d % 64 == 0 && r % kTileR == 0;   // every tile shape's multiples
  if (!mfma) {
    DSV41_REQUIRE(((int64_t)rows * groups * r + 255) / 256 < (1ll << 32), DSV41_E_ARG, "%s: too many outputs", what);
    if (dtype == DSV41_BF16) launch_wo_a_plain<bf16_t>(o, wo_a, out, rows, groups, d, r, out_dtype, stream);
    else launch_wo_a_plain<float>(o, wo_a, out, rows, groups, d, r, out_dtype, stream);
    return check_launch(what);
  }
  DSV41_REQUIRE((int64_t)groups * (r / kTileR) * ((rows + 127) / 128) < (1ll << 31), DSV41_E_ARG,
                "%s: too many tiles", what);
  WoaArgs a{static_cast<const bf16_t*>(o), static_cast<const bf16_t*>(wo_a), out, rows, groups, d, r, 0};
  if (out_dtype == DSV41_BF16) launch_wo_a<bf16_t>(a, stream);
  else launch_wo_a<float>(a, stream);
  return check_launch(what);
}

// ------------------------------------------------------------------ split-contraction rows

namespace dsv41 {
// y[m, j] = sum over the ranges s (in order) of part[m, s * n + j], rounded to bf16 once; four
// consecutive outputs per thread. With y1, columns j >= n0 go to y1 [rows, n - n0] and the rest to
// y [rows, n0] (n0 a multiple of 4).
__global__ __launch_bounds__(256) void linear_reduce_kernel(const float* __restrict__ part, bf16_t* __restrict__ y,
                                                            bf16_t* __restrict__ y1, int rows, int n, int n0,
                                                            int splits) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;   // over rows * n
  if (i >= (int64_t)rows * n) return;
  const int64_t m = i / n;
  const int j = (int)(i - m * n);
  bf16_t* dst = y1 == nullptr ? y + i : (j < n0 ? y + m * n0 + j : y1 + m * (n - n0) + (j - n0));
  const float* p = part + m * (int64_t)splits * n + j;
  f32x4 acc = *reinterpret_cast<const f32x4*>(p);
  for (int sidx = 1; sidx < splits; ++sidx) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + (int64_t)sidx * n);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = acc[e] + v[e];
  }
  uint2 st;
  st.x = pack2_bf16(acc[0], acc[1]);
  st.y = pack2_bf16(acc[2], acc[3]);
  *reinterpret_cast<uint2*>(dst) = st;
}
}  // namespace dsv41

extern "C" size_t dsv41_linear_rows_workspace_bytes(int32_t rows, int32_t n, int32_t splits) {
  if (rows <= 0 || n <= 0 || splits <= 1) return 0;
  return (size_t)rows * (size_t)splits * (size_t)n * sizeof(float);
}

// y = x w^T (or, with w1, y = x w^T and y1 = x w1^T in one launch) at decode row counts; n is the
// total width n0 + n1 of the two outputs.
static int run_linear_rows(const char* what, const void* x, const void* w, const void* w1, void* y, void* y1,
                           void* workspace, size_t workspace_bytes, int32_t rows, int32_t k, int32_t n0, int32_t n1,
                           int32_t splits, int32_t dtype, hipStream_t stream) {
  const bool pair = w1 != nullptr;
  DSV41_REQUIRE(x && w && y && (!pair || y1), DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(dtype == DSV41_BF16, DSV41_E_DTYPE, "%s: bf16 only (dtype %d)", what, dtype);
  DSV41_REQUIRE(rows >= 0 && rows <= 128 && k > 0 && n0 > 0 && n1 >= 0 && (int64_t)n0 + n1 < (1 << 30), DSV41_E_ARG,
                "%s: rows %d (at most 128), k %d, n %d + %d", what, rows, k, n0, n1);
  DSV41_REQUIRE(splits >= 1 && splits <= 64 && k % (64 * splits) == 0, DSV41_E_SHAPE,
                "%s: k = %d must split into %d ranges of whole 64-channel steps", what, k, splits);
  DSV41_REQUIRE(!pair || splits >= 2, DSV41_E_SHAPE, "%s: two weights need at least 2 contraction ranges", what);
  DSV41_REQUIRE(n0 % 32 == 0 && n1 % 32 == 0, DSV41_E_SHAPE, "%s: n = %d (+ %d) must be multiples of 32", what, n0,
                n1);
  DSV41_REQUIRE(aligned16(x) && aligned16(w) && aligned16(y) && (!pair || (aligned16(w1) && aligned16(y1))),
                DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  if (rows == 0) return 0;
  const int n = n0 + n1;
  const size_t need = dsv41_linear_rows_workspace_bytes(rows, n, splits);
  DSV41_REQUIRE(workspace_bytes >= need && (need == 0 || (workspace && aligned16(workspace))), DSV41_E_WORKSPACE,
                "%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
  WoaArgs a{static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w), splits > 1 ? workspace : y, rows, splits,
            k / splits, n, 1, static_cast<const bf16_t*>(w1), n0};
  if (splits > 1) launch_wo_a<float>(a, stream);
  else launch_wo_a<bf16_t>(a, stream);
  int rc = check_launch(what);
  if (rc || splits <= 1) return rc;
  const int64_t quads = ((int64_t)rows * n) / 4;
  hipLaunchKernelGGL(linear_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const float*>(workspace), static_cast<bf16_t*>(y), static_cast<bf16_t*>(y1), rows,
                     n, n0, splits);
  return check_launch(what);
}

extern "C" int dsv41_linear_rows(const void* x, const void* w, void* y, void* workspace, size_t workspace_bytes,
                                 int32_t rows, int32_t k, int32_t n, int32_t splits, int32_t dtype,
                                 hipStream_t stream) {
  return run_linear_rows("dsv41_linear_rows", x, w, nullptr, y, nullptr, workspace, workspace_bytes, rows, k, n, 0,
                         splits, dtype, stream);
}

extern "C" int dsv41_linear_rows_pair(const void* x, const void* w0, const void* w1, void* y0, void* y1,
                                      void* workspace, size_t workspace_bytes, int32_t rows, int32_t k, int32_t n0,
                                      int32_t n1, int32_t splits, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_linear_rows_pair";
  DSV41_REQUIRE(w1 != nullptr && n1 > 0, DSV41_E_ARG, "%s: the second weight is missing", what);
  return run_linear_rows(what, x, w0, w1, y0, y1, workspace, workspace_bytes, rows, k, n0, n1, splits, dtype, stream);
}
