// Top-k selection of the indexer, deepseek_v41_mlx/indexer.py:140-144, and the block-level
// candidate pre-filter, indexer.py:38-64.
//
// Order: the k best scores, ties broken by the lowest position (the rule the reference leaves
// to mx.argpartition, tests/test_parity.py:17-21), -0.0 equal to +0.0. Output positions are
// ascending, mapped to idx + offset when idx < lens and -1 otherwise.
//
// One 1024-thread workgroup per score row. Rows of up to 32K scores (topk_reg_kernel) keep
// their keys in registers, J consecutive positions per thread, as order-preserving 32-bit keys;
// an MSD radix select over digits of 11, 11 and 10 bits finds the k-th best key T and how many
// T-valued keys to take, then one block scan of per-thread (greater, equal) counts gives each
// thread the rank of its first selection and it writes its selections in position order -- the
// output comes out sorted and ties resolve to the lowest positions by construction. Rows over
// 16K scores with k <= 2048 can go in two stages through a workspace (per-chunk lists of the
// chunk's best k, then a merge); candidate blocks run the same register core over block maxima.
// Longer rows fall back to topk_kernel (4-pass, 8-bit digits, keys re-read from memory).
#include "select.h"

namespace dsv41 {

struct SelShared {
  uint32_t hist[kSelWaves][256];
  uint32_t tot[256];
  uint32_t wsum[kSelWaves];
  uint32_t pick[2];
};

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

// Rows of up to J*1024 scores: thread t holds the J consecutive positions t*J .. t*J+J-1 in
// registers (float4 loads), so the radix passes and the compaction touch memory only for
// histograms and the output. Digits are 11, 11 and 10 bits wide: an 11-bit leading digit (sign,
// exponent, two mantissa bits) spreads realistic score rows over enough bins that plain LDS
// atomics stay cheap, and the later passes count only keys sharing the chosen prefix.
// Histograms alternate between two buffers, so clearing the next one needs no extra barrier.
// Compaction: one block scan of the packed per-thread (greater, equal) counts gives every thread
// the number of selected positions before its own; it then walks its keys in position order.
// J keys of entries i0 .. i0+J-1 of a score row as order keys (float4 loads when `vec`: the row
// 16-byte aligned and i0 a multiple of 4), valid for j < nvalid.
template <int J>
__device__ __forceinline__ void load_keys(const float* x, int i0, int nvalid, int vec, uint32_t (&key)[J]) {
  static_assert(J % 4 == 0, "keys are loaded as float4");
  if (vec) {
#pragma unroll
    for (int q = 0; q < J / 4; ++q) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (4 * q < nvalid) v = *reinterpret_cast<const float4*>(x + i0 + 4 * q);
      key[4 * q + 0] = order_key(v.x);
      key[4 * q + 1] = order_key(v.y);
      key[4 * q + 2] = order_key(v.z);
      key[4 * q + 3] = order_key(v.w);
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j) key[j] = j < nvalid ? order_key(x[i0 + j]) : 0u;
  }
}

template <int J>
__global__ __launch_bounds__(kSelThreads) void topk_reg_kernel(const float* __restrict__ scores,
                                                               int32_t* __restrict__ out, int n, int nb, int k,
                                                               int start_pos, int ratio, int offset, int vec) {
  __shared__ RegSelShared sh;
  const int64_t row = blockIdx.x;
  const float* x = scores + row * nb;
  int32_t* o = out + row * k;
  const int s = (int)(row % n);
  const int lens = (start_pos + s + 1) / ratio;
  const int i0 = threadIdx.x * J;
  const int nvalid = min(max(nb - i0, 0), J);   // keys j < nvalid are real positions
  if (k >= nb) {                                 // everything is selected, in order
    for (int j = 0; j < nvalid; ++j) o[i0 + j] = i0 + j < lens ? i0 + j + offset : -1;
    return;
  }
  uint32_t key[J];
  load_keys<J>(x, i0, nvalid, vec, key);
  select_top<J>(key, nvalid, k, sh, [&](uint32_t rank, int j) {
    const int i = i0 + j;
    o[rank] = i < lens ? i + offset : -1;
  });
}

// Long rows in two stages (the workspace form). Stage 1: each kTopkChunk-entry chunk of a row
// selects its own best min(k, chunk) entries under the same order and writes them, in position
// order, as (order key, position) at cand[row][chunk][rank] -- every entry of the row's best k
// is among its chunk's best k, so the chunk lists hold the answer. Stage 2 selects the row's k
// best from the concatenated lists (still in position order, so ties still resolve to the lowest
// positions), one workgroup per row, keys in registers. Stage 1 spreads a row over
// ceil(nb / chunk) workgroups instead of one; chunks are kTopkChunk entries, or twice that where
// k is above an eighth of kTopkChunk (the lists then stay at 4,096 entries per 32K-score row).
constexpr int kTopkChunk = 4096;

template <int J>   // chunk = J * kSelThreads entries
__global__ __launch_bounds__(kSelThreads) void topk_chunk_kernel(const float* __restrict__ scores,
                                                                 uint32_t* __restrict__ ckey,
                                                                 int32_t* __restrict__ cpos, int nb, int k,
                                                                 int chunks, int vec) {
  constexpr int CH = J * kSelThreads;
  __shared__ RegSelShared sh;
  const int64_t row = blockIdx.x / chunks;
  const int ch = (int)(blockIdx.x - row * chunks);
  const int base = ch * CH;
  const int count = min(CH, nb - base);
  const int kc = min(k, count);
  const float* x = scores + row * nb + base;
  const int64_t cbase = (row * chunks + ch) * (int64_t)k;
  const int i0 = threadIdx.x * J;
  const int nvalid = min(max(count - i0, 0), J);
  uint32_t key[J];
  load_keys<J>(x, i0, nvalid, vec, key);
  select_top<J>(key, nvalid, kc, sh, [&](uint32_t rank, int j) {
    ckey[cbase + rank] = order_key(x[i0 + j]);     // re-read: j is a run-time index
    cpos[cbase + rank] = base + i0 + j;
  });
}

template <int J>
__global__ __launch_bounds__(kSelThreads) void topk_merge_kernel(const uint32_t* __restrict__ ckey,
                                                                  const int32_t* __restrict__ cpos,
                                                                  int32_t* __restrict__ out, int n, int nb, int k,
                                                                  int chunks, int chunk, int start_pos, int ratio,
                                                                  int offset) {
  __shared__ RegSelShared sh;
  const int64_t row = blockIdx.x;
  // the lists of chunks 0..chunks-2 are full (k entries: chunk >= k), the last one holds
  // min(k, its count): the valid entries are the first m of the row's concatenation
  const int m = (chunks - 1) * k + min(k, nb - (chunks - 1) * chunk);
  const uint32_t* kr = ckey + row * (int64_t)chunks * k;
  const int32_t* pr = cpos + row * (int64_t)chunks * k;
  int32_t* o = out + row * k;
  const int s = (int)(row % n);
  const int lens = (start_pos + s + 1) / ratio;
  const int i0 = threadIdx.x * J;
  const int nvalid = min(max(m - i0, 0), J);
  // keys and positions are loaded together: the selection's output step then reads no memory
  uint32_t key[J];
  int32_t pos[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    key[j] = j < nvalid ? kr[i0 + j] : 0u;
    pos[j] = j < nvalid ? pr[i0 + j] : 0;
  }
  select_top<J>(key, nvalid, k, sh, [&](uint32_t rank, int j) {
    int32_t i = 0;
#pragma unroll
    for (int t = 0; t < J; ++t) i = t == j ? pos[t] : i;   // j is a run-time index
    o[rank] = i < lens ? i + offset : -1;
  });
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

// select_candidate_blocks on the register core: thread t holds the maxima of blocks t*J ..
// t*J+J-1 as order keys (the pinned block (lens-1)/bs as +inf); the best min(topk_blocks, nblk)
// blocks (ties -> lowest block) are marked, and a marked block is kept when its maximum is
// > -inf. Each thread then writes the keep bytes of its own blocks.
template <int J>
__global__ __launch_bounds__(kSelThreads) void candidate_kernel(const float* __restrict__ scores,
                                                                uint8_t* __restrict__ keep, int n, int nb,
                                                                int topk_blocks, int bs, const int32_t* lens_v,
                                                                int start_pos, int ratio, int vec8) {
  __shared__ RegSelShared sh;
  __shared__ uint8_t marked[kMaxCandBlocks];
  const int64_t row = blockIdx.x;
  const float* x = scores + row * nb;
  const int s = (int)(row % n);
  const int lens = lens_v ? lens_v[s] : (start_pos + s + 1) / ratio;
  const int nblk = (nb + bs - 1) / bs;
  const int last = lens > 0 ? (lens - 1) / bs : -1;  // floor((lens - 1) / bs)
  const int j0 = threadIdx.x * J;
  const int nvalid = min(max(nblk - j0, 0), J);
  float bm[J];
  uint32_t key[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    float m = -INFINITY;
    const int blk = j0 + j;
    if (j < nvalid) {
      if (vec8 && blk * 8 + 8 <= nb) {                 // 8-score block, 16-byte aligned
        const float4 u = *reinterpret_cast<const float4*>(x + blk * 8);
        const float4 v = *reinterpret_cast<const float4*>(x + blk * 8 + 4);
        m = fmaxf(fmaxf(fmaxf(u.x, u.y), fmaxf(u.z, u.w)), fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
      } else {
        const int e = min(nb, (blk + 1) * bs);
        for (int t = blk * bs; t < e; ++t) m = fmaxf(m, x[t]);
      }
    }
    bm[j] = blk == last ? INFINITY : m;
    key[j] = order_key(bm[j]);
    if (j < nvalid) marked[blk] = 0;
  }
  const int kb = min(topk_blocks, nblk);
  if (kb >= nblk) {
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (j < nvalid) marked[j0 + j] = 1;
  } else if (kb > 0) {
    select_top<J>(key, nvalid, kb, sh, [&](uint32_t, int j) { marked[j0 + j] = 1; });
  }
  __syncthreads();
  uint8_t* kr = keep + row * nb;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (j >= nvalid) continue;
    const int blk = j0 + j;
    const uint8_t v = (marked[blk] && bm[j] > -INFINITY) ? 1 : 0;
    if (vec8 && blk * 8 + 8 <= nb) {
      const uint32_t w = v ? 0x01010101u : 0u;
      *reinterpret_cast<uint2*>(kr + blk * 8) = make_uint2(w, w);
    } else {
      const int e = min(nb, (blk + 1) * bs);
      for (int t = blk * bs; t < e; ++t) kr[t] = v;
    }
  }
}

}  // namespace dsv41

using namespace dsv41;

namespace dsv41 {
// Stage 2 of a two-stage selection over per-chunk lists of k (key, position) entries, `chunk`
// scores per chunk (>= k); also used by the indexer's fused decode form. chunks * k <= 32768.
int topk_merge_launch(const char* what, const uint32_t* ckey, const int32_t* cpos, int32_t* out, int64_t rows, int n,
                      int nb, int k, int chunks, int chunk, int start_pos, int ratio, int offset, hipStream_t stream) {
  const int64_t m = (int64_t)chunks * k;
  DSV41_REQUIRE(m <= 32 * kSelThreads && rows < (1ll << 31), DSV41_E_SHAPE, "%s: %lld candidates per row", what,
                (long long)m);
  const dim3 grid((unsigned)rows), block(kSelThreads);
#define DSV41_MERGE_CASE(J_)                                                                                  \
  if (m <= J_ * kSelThreads) {                                                                                \
    hipLaunchKernelGGL(topk_merge_kernel<J_>, grid, block, 0, stream, ckey, cpos, out, n, nb, k, chunks, chunk, \
                       start_pos, ratio, offset);                                                            \
    return check_launch(what);                                                                              \
  }
  DSV41_MERGE_CASE(4)
  DSV41_MERGE_CASE(8)
  DSV41_MERGE_CASE(16)
  DSV41_MERGE_CASE(32)
#undef DSV41_MERGE_CASE
  return set_error(DSV41_E_SHAPE, "%s: too many candidates", what);
}
}  // namespace dsv41

// The two-stage form for a row of nb scores: rows longer than one 16-keys-per-thread workgroup
// holds, k at most half a chunk, and the chunk lists small enough for one register workgroup.
// For 16 rows of 32,768 scores and k = 1,024 one 32-keys-per-thread workgroup per row is faster
// on scores already in cache (17.5-19.3 against 19.4-20.2 us), but inside a decode step, reading
// the scores the scoring kernel has just written, the two stages spread that read over 8
// workgroups per row and win: the 40-layer fp8 step took 1.163-1.166 ms against 1.190-1.195 ms.
static bool topk_two_stage(int nb, int k, int* chunks, int* jm, int* chunk) {
  if (nb <= 16 * kSelThreads || 2 * k > kTopkChunk) return false;
  // lists of more than 4,096 entries per row with 4,096-entry chunks: 8,192-entry chunks halve them
  const int ch = (int64_t)((nb + kTopkChunk - 1) / kTopkChunk) * k > 4 * kSelThreads ? 2 * kTopkChunk : kTopkChunk;
  const int c = (nb + ch - 1) / ch;
  const int64_t m = (int64_t)c * k;
  if (m > 32 * kSelThreads) return false;
  *chunks = c;
  *chunk = ch;
  *jm = m <= 4 * kSelThreads ? 4 : (m <= 8 * kSelThreads ? 8 : (m <= 16 * kSelThreads ? 16 : 32));
  return true;
}

static size_t topk_ws_bytes(int64_t rows, int chunks, int k) {
  const size_t list = ((size_t)rows * chunks * k * sizeof(uint32_t) + 255) & ~(size_t)255;
  return 2 * list;                               // order keys, then positions
}

static int topk_launch(const char* what, const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                       int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset, void* workspace,
                       size_t workspace_bytes, bool allow_two_stage, hipStream_t stream) {
  DSV41_REQUIRE(scores && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(rows >= 0 && n > 0 && nb >= 0 && topk >= 0 && start_pos >= 0 && ratio > 0, DSV41_E_ARG,
                "%s: bad sizes", what);
  DSV41_REQUIRE(nb <= (1 << 22), DSV41_E_SHAPE, "%s: nb %d > 2^22", what, nb);
  DSV41_REQUIRE(rows < (1ll << 31), DSV41_E_ARG, "%s: too many rows", what);
  const int k = topk < nb ? topk : nb;
  if (rows == 0 || k == 0) return 0;
  const dim3 grid((unsigned)rows), block(kSelThreads);
  const int vec = (nb % 4 == 0 && aligned16(scores)) ? 1 : 0;
  int chunks = 0, jm = 0, chunk = 0;
  if (allow_two_stage && topk_two_stage(nb, k, &chunks, &jm, &chunk)) {
    const size_t need = topk_ws_bytes(rows, chunks, k);
    DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed", what,
                  need);
    DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
    DSV41_REQUIRE(rows * chunks < (1ll << 31), DSV41_E_ARG, "%s: too many row chunks", what);
    uint32_t* ckey = reinterpret_cast<uint32_t*>(workspace);
    int32_t* cpos = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(workspace) + need / 2);
    if (chunk == kTopkChunk)
      hipLaunchKernelGGL(topk_chunk_kernel<kTopkChunk / kSelThreads>, dim3((unsigned)(rows * chunks)), block, 0, stream,
                         scores, ckey, cpos, nb, k, chunks, vec);
    else
      hipLaunchKernelGGL(topk_chunk_kernel<2 * kTopkChunk / kSelThreads>, dim3((unsigned)(rows * chunks)), block, 0,
                         stream, scores, ckey, cpos, nb, k, chunks, vec);
    int rc = check_launch(what);
    if (rc) return rc;
    return topk_merge_launch(what, ckey, cpos, out, rows, n, nb, k, chunks, chunk, start_pos, ratio, offset, stream);
  }
  if (nb <= 4 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<4>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset, vec);
  else if (nb <= 8 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<8>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset, vec);
  else if (nb <= 16 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<16>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset,
                       vec);
  else if (nb <= 32 * kSelThreads)
    hipLaunchKernelGGL(topk_reg_kernel<32>, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset,
                       vec);
  else
    hipLaunchKernelGGL(topk_kernel, grid, block, 0, stream, scores, out, n, nb, k, start_pos, ratio, offset);
  return check_launch(what);
}

extern "C" int dsv41_topk_select(const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                                 int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset, hipStream_t stream) {
  return topk_launch("dsv41_topk_select", scores, out, rows, n, nb, topk, start_pos, ratio, offset, nullptr, 0, false,
                     stream);
}

extern "C" size_t dsv41_topk_workspace_bytes(int64_t rows, int32_t nb, int32_t topk) {
  if (rows <= 0 || nb <= 0 || topk <= 0) return 0;
  const int k = topk < nb ? topk : nb;
  int chunks = 0, jm = 0, chunk = 0;
  return topk_two_stage(nb, k, &chunks, &jm, &chunk) ? topk_ws_bytes(rows, chunks, k) : 0;
}

extern "C" int dsv41_topk_select_ws(const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                                    int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  return topk_launch("dsv41_topk_select_ws", scores, out, rows, n, nb, topk, start_pos, ratio, offset, workspace,
                     workspace_bytes, true, stream);
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
  const int nblk = (nb + block_size - 1) / block_size;
  // 8-score blocks read as two float4 and written as 8 keep bytes: rows 16-byte aligned
  const int vec8 = (block_size == 8 && nb % 4 == 0 && aligned16(scores) &&
                    (reinterpret_cast<uintptr_t>(keep) & 7u) == 0 && nb % 8 == 0) ? 1 : 0;
  if (nblk <= 4 * kSelThreads)
    hipLaunchKernelGGL(candidate_kernel<4>, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, scores, keep, n, nb,
                       topk_blocks, block_size, lens, start_pos, ratio, vec8);
  else
    hipLaunchKernelGGL(candidate_kernel<8>, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, scores, keep, n, nb,
                       topk_blocks, block_size, lens, start_pos, ratio, vec8);
  return check_launch(what);
}
