// Exact top-k selection core shared by the top-k kernels (topk.hip) and the indexer's fused
// decode form (indexer.hip): order-preserving keys, a wave scan, and the register radix select
// with ordered compaction (ties -> lowest entry).
#pragma once
#include "common.h"

namespace dsv41 {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;

__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u << 1) == 0u) u = 0u;                       // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive scan over the 64 lanes of a wave with DPP moves (no LDS round trips): shifts by 1,
// 2, 4, 8 within each 16-lane row, then row 15 -> row 1 and 3, lane 31 -> rows 2 and 3.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

struct RegSelShared {
  uint32_t hist[2][2048];
  uint32_t wsum[kSelWaves];
  uint32_t pick[3];
};

// The selection core of the register kernels: thread t holds the keys of entries t*J .. t*J+J-1
// (consecutive, in position order), valid for j < nvalid; 1 <= k <= the number of valid entries.
// Finds the k-th best key T and how many T-valued entries to take -- or, once the digit bin
// that holds the k-th best has exactly as many entries as are still to take (after one or two of
// the three digit passes), the resolved top bits P of every selected key: the selection is then
// every key whose top bits are >= P, with no tie left to break -- then calls emit(rank, j) for
// each selected entry j of this thread, rank = its place among the selected in entry order (so
// ties resolve to the lowest entries); j is a run-time index, so emit must not index register
// arrays with it. All threads of the workgroup must call it.
template <int J, int NT = kSelThreads, typename Emit>
__device__ __forceinline__ void select_top(const uint32_t (&key)[J], int nvalid, int k, RegSelShared& sh, Emit emit) {
  constexpr int NBIN = 2048;
  constexpr int BPT = NBIN / NT;                 // suffix-scan bins per thread
  constexpr int NWV = NT / 64;
  static_assert(NBIN % NT == 0 && NWV <= kSelWaves, "512 or 1024 threads");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int b = 0; b < BPT; ++b) sh.hist[bi][tid + b * NT] = 0u;
  __syncthreads();

  // exclusive prefix of the per-wave totals in wsum, for wave `wave` (all reads in flight)
  auto wave_base = [&]() {
    uint32_t base = 0u;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      const uint32_t v = sh.wsum[w];
      base += w < wave ? v : 0u;
    }
    return base;
  };

  uint32_t prefix = 0u, pmask = 0u;
  int kk = k;
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 2 ? 1023u : 2047u;
    uint32_t* h = sh.hist[pass & 1];
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (j < nvalid && (key[j] & pmask) == prefix) atomicAdd(&h[(key[j] >> shift) & dmask], 1u);
    __syncthreads();                             // histogram complete
    if (pass < 2) {                              // the other buffer was last read before the previous barrier
#pragma unroll
      for (int b = 0; b < BPT; ++b) sh.hist[(pass & 1) ^ 1][tid + b * NT] = 0u;
    }
    // suffix scan from the highest digit down: thread t owns digits 2047-BPT*t .. 2048-BPT*(t+1)
    uint32_t c[BPT], tot = 0u;
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      c[b] = h[NBIN - 1 - BPT * tid - b];
      tot += c[b];
    }
    const uint32_t incl = wave_incl_scan(tot, lane);
    if (lane == 63) sh.wsum[wave] = incl;
    __syncthreads();
    uint32_t above = wave_base() + incl - tot;
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      if (above < (uint32_t)kk && (uint32_t)kk <= above + c[b]) {
        sh.pick[0] = (uint32_t)(NBIN - 1 - BPT * tid - b);
        sh.pick[1] = above;
        sh.pick[2] = above + c[b] == (uint32_t)kk ? 1u : 0u;   // the whole bin is taken
      }
      above += c[b];
    }
    __syncthreads();
    prefix |= sh.pick[0] << shift;
    pmask |= dmask << shift;
    kk -= (int)sh.pick[1];
    // uniform: every thread read the same pick; the next pass's writes to pick follow a barrier
    // that every thread passes after these reads
    if (pass < 2 && sh.pick[2] != 0u) break;
  }
  // compare the resolved top bits only (all 32 after three passes)
  const uint32_t T = prefix;
  const uint32_t need = (uint32_t)kk;            // keys == T to take, lowest entries first
  uint32_t mk[J];
#pragma unroll
  for (int j = 0; j < J; ++j) mk[j] = key[j] & pmask;

  uint32_t cg = 0u, ce = 0u;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    cg += (j < nvalid && mk[j] > T) ? 1u : 0u;
    ce += (j < nvalid && mk[j] == T) ? 1u : 0u;
  }
  const uint32_t packed = (cg << 16) | ce;       // counts <= 32768: no carry between halves
  const uint32_t incl = wave_incl_scan(packed, lane);
  if (lane == 63) sh.wsum[wave] = incl;          // last read before the final pass barrier
  __syncthreads();
  const uint32_t excl = wave_base() + incl - packed;
  const uint32_t gt_before = excl >> 16;
  uint32_t eq_before = excl & 0xFFFFu;
  // Every key > T is taken, and a key == T while fewer than `need` equal keys precede it; each
  // taken entry occupies the next rank, so this thread's m-th taken entry has rank
  // gt_before + min(eq_before, need) + m. The take mask is formed branch-free, then only its set
  // bits are visited (a thread takes few entries).
  const uint32_t base = gt_before + min(eq_before, need);
  uint32_t tmask = 0u;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool ok = j < nvalid;
    const bool gt = ok && mk[j] > T, eq = ok && mk[j] == T;
    tmask |= (gt || (eq && eq_before < need)) ? (1u << j) : 0u;
    eq_before += eq ? 1u : 0u;
  }
  for (uint32_t m = 0u; tmask != 0u; ++m) {
    const int j = __builtin_ctz(tmask);
    emit(base + m, j);
    tmask &= tmask - 1u;
  }
}

// Host: stage 2 of a two-stage selection (topk.hip). ckey/cpos hold, per row, `chunks` lists of k
// (order key, position) entries in position order, each list the best min(k, chunk count) of its
// `chunk`-score chunk; writes the row's k best as top-k output (positions < lens -> + offset,
// else -1, lens = (start_pos + s + 1) / ratio, s = row % n).
int topk_merge_launch(const char* what, const uint32_t* ckey, const int32_t* cpos, int32_t* out, int64_t rows, int n,
                      int nb, int k, int chunks, int chunk, int start_pos, int ratio, int offset, hipStream_t stream);

}  // namespace dsv41
