// Top-k selection of the indexer, deepseek_v41_mlx/indexer.py:200-204, and the block-level
// candidate pre-filter, indexer.py:38-64.
//
// Order: the k best scores, ties broken by the lowest position (the rule the reference leaves
// to mx.argpartition, tests/test_parity.py:17-21), -0.0 equal to +0.0. Output positions are
// ascending, mapped to idx + offset when idx < lens and -1 otherwise.
//
// One 1024-thread workgroup per score row. A 4-pass, 8-bit MSD radix select over
// order-preserving 32-bit keys finds the k-th best key T and how many T-valued keys to keep
// (per-wave histograms in LDS keep atomics uncontended); one ordered compaction pass then
// writes every key > T plus the first `need` keys == T, in position order (wave ballots and
// popcounts give each selected key its rank) -- so the output comes out sorted and ties
// resolve to the lowest positions by construction. Rows up to 32k scores keep their keys in
// registers for the whole selection.
#include "common.h"

namespace dsv41 {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;

__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u << 1) == 0u) u = 0u;                       // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelShared {
  uint32_t hist[kSelWaves][256];
  uint32_t tot[256];
  uint32_t wsum[kSelWaves];
  uint32_t pick[2];
};

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// Finds the k-th largest key among key(0..count) (1 <= k <= count). Returns T and sets
// *need = number of T-valued keys to take after all keys > T. All threads must call it.
template <typename KeyFn>
__device__ uint32_t radix_select(SelShared& sh, KeyFn key, int count, int k, int* need) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0u, pmask = 0u;
  int kk = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&sh.hist[0][0])[i] = 0u;
    if (tid == 0) sh.pick[0] = sh.pick[1] = 0u;
    __syncthreads();
    for (int i = tid; i < count; i += kSelThreads) {
      const uint32_t kv = key(i);
      if ((kv & pmask) == prefix) atomicAdd(&sh.hist[wave][(kv >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 256) {
      uint32_t c = 0u;
#pragma unroll
      for (int w = 0; w < kSelWaves; ++w) c += sh.hist[w][tid];
      sh.tot[tid] = c;
    }
    __syncthreads();
    uint32_t incl = 0u, mine = 0u;
    if (tid < 256) {
      // suffix sums over digits: thread t handles digit 255 - t
      mine = sh.tot[255 - tid];
      incl = wave_incl_scan(mine, lane);
      if (lane == 63) sh.wsum[wave] = incl;
    }
    __syncthreads();
    if (tid < 256) {
      for (int w = 0; w < wave; ++w) incl += sh.wsum[w];
      const uint32_t above = incl - mine;               // keys whose digit is > d
      if (above < (uint32_t)kk && (uint32_t)kk <= incl) {
        sh.pick[0] = 255u - (uint32_t)tid;
        sh.pick[1] = above;
      }
    }
    __syncthreads();
    prefix |= sh.pick[0] << shift;
    pmask |= 255u << shift;
    kk -= (int)sh.pick[1];
    __syncthreads();
  }
  *need = kk;
  return prefix;
}

// Ordered compaction: calls emit(i, rank) for each selected i in increasing i, where rank is
// its position among the selected. Selection: key > T, or key == T among the first `need`.
template <typename KeyFn, typename EmitFn>
__device__ void ordered_select(SelShared& sh, KeyFn key, int count, uint32_t T, int need, EmitFn emit) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t gt_base = 0u, eq_base = 0u;
  for (int c0 = 0; c0 < count; c0 += kSelThreads) {
    const int i = c0 + tid;
    const uint32_t kv = i < count ? key(i) : 0u;
    const uint32_t gt = (i < count && kv > T) ? 1u : 0u;
    const uint32_t eq = (i < count && kv == T) ? 1u : 0u;
    const uint32_t packed = (gt << 16) | eq;
    const uint32_t incl = wave_incl_scan(packed, lane);
    if (lane == 63) sh.wsum[wave] = incl;
    __syncthreads();
    uint32_t wbase = 0u, total = 0u;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
      const uint32_t ws = sh.wsum[w];
      if (w < wave) wbase += ws;
      total += ws;
    }
    const uint32_t excl = wbase + incl - packed;
    const uint32_t gt_before = gt_base + (excl >> 16);
    const uint32_t eq_before = eq_base + (excl & 0xFFFFu);
    if (gt || (eq && eq_before < (uint32_t)need))
      emit(i, (int)(gt_before + min(eq_before, (uint32_t)need)));
    gt_base += total >> 16;
    eq_base += total & 0xFFFFu;
    __syncthreads();
  }
}

// Histogram add where many lanes share a digit (the leading radix passes see most keys in a
// few bins): the two most common digits of the wave are added with one atomic each, the
// remaining lanes individually, so no LDS address takes more than a few atomics per instruction.
__device__ __forceinline__ void hist_add(uint32_t* h, uint32_t digit, bool active, int lane) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const uint64_t act = __ballot(active);
    if (act == 0ull) return;
    const int leader = __ffsll((unsigned long long)act) - 1;
    const uint32_t ld = (uint32_t)__shfl((int)digit, leader, 64);
    const uint64_t peers = __ballot(active && digit == ld);
    if (lane == leader) atomicAdd(&h[ld], (uint32_t)__popcll(peers));
    if (digit == ld) active = false;
  }
  if (active) atomicAdd(&h[digit], 1u);
}

// Rows of up to J*1024 scores: every thread holds its J keys in registers (one batched
// load), so the four radix passes and the compaction touch memory only for histograms.
template <int J>
__global__ __launch_bounds__(kSelThreads) void topk_reg_kernel(const float* __restrict__ scores,
                                                               int32_t* __restrict__ out, int n, int nb, int k,
                                                               int start_pos, int ratio, int offset) {
  constexpr int E = J * kSelWaves;               // (chunk, wave) count entries
  constexpr int EL = (E + 63) / 64;              // entries per lane of wave 0 in the base scan
  __shared__ uint32_t hist[kSelWaves][256];
  __shared__ uint32_t cnt[2][E];                 // gt / eq counts, then exclusive bases
  __shared__ uint32_t pick[2];
  const int64_t row = blockIdx.x;
  const float* x = scores + row * nb;
  int32_t* o = out + row * k;
  const int s = (int)(row % n);
  const int lens = (start_pos + s + 1) / ratio;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  uint32_t key[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = tid + j * kSelThreads;
    key[j] = i < nb ? order_key(x[i]) : 0u;
  }
  uint32_t T = 0u;
  int need = k;
  if (k < nb) {
    uint32_t prefix = 0u, pmask = 0u;
    int kk = k;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      // a wave clears and fills only its own histogram row: no barrier before the atomics
      for (int d = lane; d < 256; d += 64) hist[wave][d] = 0u;
#pragma unroll
      for (int j = 0; j < J; ++j)
        hist_add(hist[wave], (key[j] >> shift) & 255u, tid + j * kSelThreads < nb && (key[j] & pmask) == prefix,
                 lane);
      __syncthreads();
      if (wave == 0) {
        // lane l owns digits 255-4l .. 252-4l; scan from the highest digit down
        uint32_t c[4], sum = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int d = 255 - 4 * lane - q;
          uint32_t t = 0u;
#pragma unroll
          for (int w = 0; w < kSelWaves; ++w) t += hist[w][d];
          c[q] = t;
          sum += t;
        }
        uint32_t above = wave_incl_scan(sum, lane) - sum;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (above < (uint32_t)kk && (uint32_t)kk <= above + c[q]) {
            pick[0] = (uint32_t)(255 - 4 * lane - q);
            pick[1] = above;
          }
          above += c[q];
        }
      }
      __syncthreads();
      prefix |= pick[0] << shift;
      pmask |= 255u << shift;
      kk -= (int)pick[1];
    }
    T = prefix;
    need = kk;
  }
  // ordered compaction: keys > T, then the first `need` keys == T, in position order
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = tid + j * kSelThreads;
    const bool ok = i < nb && k < nb;
    const uint64_t bg = __ballot(ok && key[j] > T);
    const uint64_t be = __ballot(ok && key[j] == T);
    if (lane == 0) {
      cnt[0][j * kSelWaves + wave] = (uint32_t)__popcll(bg);
      cnt[1][j * kSelWaves + wave] = (uint32_t)__popcll(be);
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      uint32_t v[EL], sum = 0u;
#pragma unroll
      for (int q = 0; q < EL; ++q) {
        const int e = lane * EL + q;
        v[q] = e < E ? cnt[f][e] : 0u;
        sum += v[q];
      }
      uint32_t base = wave_incl_scan(sum, lane) - sum;
#pragma unroll
      for (int q = 0; q < EL; ++q) {
        const int e = lane * EL + q;
        if (e < E) cnt[f][e] = base;
        base += v[q];
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = tid + j * kSelThreads;
    if (k >= nb) {                       // everything selected, in order
      if (i < nb) o[i] = i < lens ? i + offset : -1;
      continue;
    }
    const bool ok = i < nb;
    const bool gt = ok && key[j] > T, eq = ok && key[j] == T;
    const uint64_t bg = __ballot(gt), be = __ballot(eq);
    const uint32_t gt_before = cnt[0][j * kSelWaves + wave] + (uint32_t)__popcll(bg & below);
    const uint32_t eq_before = cnt[1][j * kSelWaves + wave] + (uint32_t)__popcll(be & below);
    if (gt || (eq && eq_before < (uint32_t)need)) {
      const uint32_t pos = gt_before + min(eq_before, (uint32_t)need);
      if (pos < (uint32_t)k) o[pos] = i < lens ? i + offset : -1;
    }
  }
}

// Rows longer than 32k scores: keys are re-read from memory in every pass.
__global__ __launch_bounds__(kSelThreads) void topk_kernel(const float* __restrict__ scores, int32_t* __restrict__ out,
                                                           int n, int nb, int k, int start_pos, int ratio,
                                                           int offset) {
  __shared__ SelShared sh;
  const int64_t row = blockIdx.x;
  const float* x = scores + row * nb;
  int32_t* o = out + row * k;
  const int s = (int)(row % n);
  const int lens = (start_pos + s + 1) / ratio;
  auto key = [&](int i) { return order_key(x[i]); };
  auto emit = [&](int i, int rank) {
    if (rank < k) o[rank] = i < lens ? i + offset : -1;
  };
  if (k >= nb) {  // everything is selected (k == nb)
    for (int i = threadIdx.x; i < nb; i += kSelThreads) emit(i, i);
    return;
  }
  int need = 0;
  const uint32_t T = radix_select(sh, key, nb, k, &need);
  ordered_select(sh, key, nb, T, need, emit);
}

constexpr int kMaxCandBlocks = 8192;

__global__ __launch_bounds__(kSelThreads) void candidate_kernel(const float* __restrict__ scores,
                                                                uint8_t* __restrict__ keep, int n, int nb,
                                                                int topk_blocks, int bs, const int32_t* lens_v,
                                                                int start_pos, int ratio) {
  __shared__ SelShared sh;
  __shared__ float bmax[kMaxCandBlocks];
  __shared__ uint8_t bkeep[kMaxCandBlocks];
  const int64_t row = blockIdx.x;
  const float* x = scores + row * nb;
  const int s = (int)(row % n);
  const int lens = lens_v ? lens_v[s] : (start_pos + s + 1) / ratio;
  const int nblk = (nb + bs - 1) / bs;
  const int last = lens > 0 ? (lens - 1) / bs : -1;  // floor((lens - 1) / bs)
  for (int j = threadIdx.x; j < nblk; j += kSelThreads) {
    float m = -INFINITY;
    const int e = min(nb, (j + 1) * bs);
    for (int t = j * bs; t < e; ++t) m = fmaxf(m, x[t]);
    bmax[j] = j == last ? INFINITY : m;
    bkeep[j] = 0;
  }
  __syncthreads();
  const int kb = min(topk_blocks, nblk);
  if (kb >= nblk) {
    for (int j = threadIdx.x; j < nblk; j += kSelThreads) bkeep[j] = bmax[j] > -INFINITY ? 1 : 0;
  } else if (kb > 0) {
    auto key = [&](int j) { return order_key(bmax[j]); };
    int need = 0;
    const uint32_t T = radix_select(sh, key, nblk, kb, &need);
    ordered_select(sh, key, nblk, T, need, [&](int j, int) { bkeep[j] = bmax[j] > -INFINITY ? 1 : 0; });
  }
  __syncthreads();
  uint8_t* kr = keep + row * nb;
  for (int t = threadIdx.x; t < nb; t += kSelThreads) kr[t] = bkeep[t / bs];
}

}  // namespace dsv41

using namespace dsv41;

extern "C" int dsv41_topk_select(const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                                 int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset, hipStream_t stream) {
  const char* what = "dsv41_topk_select";
  DSV41_REQUIRE(scores && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && n > 0 && nb >= 0 && topk >= 0 && start_pos >= 0 && ratio > 0, DSV41_E_ARG,
                "%s: bad sizes", what);
  DSV41_REQUIRE(nb <= (1 << 22), DSV41_E_SHAPE, "%s: nb %d > 2^22", what, nb);
  DSV41_REQUIRE(rows < (1ll << 31), DSV41_E_ARG, "%s: too many rows", what);
  const int k = topk < nb ? topk : nb;
  if (rows == 0 || k == 0) return 0;
  const dim3 grid((unsigned)rows), block(kSelThreads);
  if (nb <= 4 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<4>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  else if (nb <= 8 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<8>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  else if (nb <= 16 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<16>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  else if (nb <= 32 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<32>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  else
    hipLaunchKernelGGL(topk_kernel, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  return check_launch(what);
}

extern "C" int dsv41_candidate_blocks(const float* scores, uint8_t* keep, int64_t rows, int32_t n, int32_t nb,
                                      int32_t topk_blocks, int32_t block_size, const int32_t* lens,
                                      int32_t start_pos, int32_t ratio, hipStream_t stream) {
  const char* what = "dsv41_candidate_blocks";
  DSV41_REQUIRE(scores && keep, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && n > 0 && nb >= 0 && topk_blocks >= 0 && block_size > 0 && start_pos >= 0 && ratio > 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE((nb + block_size - 1) / block_size <= kMaxCandBlocks, DSV41_E_SHAPE, "%s: more than %d blocks",
                what, kMaxCandBlocks);
  DSV41_REQUIRE(rows < (1ll << 31), DSV41_E_ARG, "%s: too many rows", what);
  if (rows == 0 || nb == 0) return 0;
  hipLaunchKernelGGL(candidate_kernel, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, scores, keep, n, nb,
                     topk_blocks, block_size, lens, start_pos, ratio);
  return check_launch(what);
}
