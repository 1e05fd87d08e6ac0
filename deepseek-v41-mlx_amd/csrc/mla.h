// Definitions shared by the sparse-MLA kernels: the argument block, the unified KV position map
// of a query's list, the rope steps applied around the attention, and small wave helpers.
#pragma once

#include "mfma.h"

namespace dsv41 {

struct KvSrc {
  const void* ring;  int64_t ring_bstride;  int window, wp, ring_first;
  const void* chunk; int64_t chunk_bstride; int n_chunk;
  const void* comp;  int64_t comp_bstride;  int n_comp;
  // fp8 compressed cache (F8 kernels): e4m3 rows, one ue8m0 byte per 32 channels for every
  // block of comp_scale_rb rows (1 or 32), comp_scale_bstride bytes per batch row
  const uint8_t* comp_scale; int64_t comp_scale_bstride; int comp_scale_rb;
  const int32_t* idx; int k;
  int win_implicit;
};

struct MlaArgs {
  const void* q;
  void* o;
  const float* sink;
  KvSrc src;
  int m, heads, dim;
  float scale;
  const float* cos_tab;
  const float* sin_tab;
  int rd, start_pos;
  int q_rd;           // > 0: apply q's forward rope tail of this width while loading q
  int hgroups, splits, per_split;
  bf16_t* part_o;     // split partials: numerator / denominator, rounded to bf16, in 16 x 16 tiles
                      // (part_tile: [unit][split][head tile][dim / 16][16 heads][16 channels])
  float* part_ml;     // split partials: (log2-domain max, denominator) [unit][split][head][2]
  void* ring_w;       // one-token decode: also store the token's KV row in its ring slot (or null)
};

// Workgroups are dispatched to the 8 XCDs round-robin by linear id and each XCD has its own L2.
// Renumber so that consecutive logical tiles run on one XCD: the head groups of one query (and
// neighbouring queries of a prefill chunk) gather the same KV rows and then share that L2.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_tile(int bid, int total) {
  if (total % kXcds) return bid;
  return (bid % kXcds) * (total / kXcds) + bid / kXcds;
}

// Entry e of query qs's list -> unified position (-1 = none). wc = window entries of qs.
__device__ __forceinline__ int list_pos(const KvSrc& s, int b, int m, int qs, int e, int wc) {
  if (s.win_implicit) {
    if (e < wc) return s.wp + qs - wc + 1 + e;
    e -= wc;
  }
  if (e < s.k) return s.idx[((int64_t)b * m + qs) * s.k + e];
  return -1;
}

// Element offset of split partial (unit, split sp, head h, channel d): 16-head x 16-channel tiles
// of 512 contiguous bytes, so the 64 lanes of one MFMA accumulator tile store one full block and
// a combine lane's 8 channels of one head are 16 contiguous bytes.
__device__ __forceinline__ int64_t part_tile(const MlaArgs& a, int unit, int sp, int h, int d) {
  const int htiles = (a.heads + 15) >> 4;
  return ((((int64_t)unit * a.splits + sp) * htiles + (h >> 4)) * (a.dim >> 4) + (d >> 4)) * 256 + (h & 15) * 16 +
         (d & 15);
}

template <typename T>
__device__ __forceinline__ const T* row_ptr(const KvSrc& s, int b, int u, int dim) {
  if (u < 0) return nullptr;
  if (u < s.wp)
    return reinterpret_cast<const T*>(s.ring) + b * s.ring_bstride + (int64_t)((s.ring_first + u) % s.window) * dim;
  u -= s.wp;
  if (u < s.n_chunk) return reinterpret_cast<const T*>(s.chunk) + b * s.chunk_bstride + (int64_t)u * dim;
  u -= s.n_chunk;
  if (u < s.n_comp) return reinterpret_cast<const T*>(s.comp) + b * s.comp_bstride + (int64_t)u * dim;
  return nullptr;
}

__device__ __forceinline__ int window_count(const KvSrc& s, int qs) {
  return s.win_implicit ? min(s.window, s.wp + qs + 1) : 0;
}

// inverse rope: rotate the adjacent pair (x0, x1) by the conjugate of (cs, sn)
__device__ __forceinline__ void rope_inv_apply(float cs, float sn_neg, float& x0, float& x1) {
  rotate_pair(x0, x1, cs, sn_neg);
}

__device__ __forceinline__ bool in_rope_tail(const MlaArgs& a, int D, int d) { return a.rd > 0 && d >= D - a.rd; }

// (cos, -sin) of the pair at channel d (even) of query qs, when d lies in the rope tail
__device__ __forceinline__ void rope_inv_load(const MlaArgs& a, int D, int qs, int d, float& cs, float& sn_neg) {
  const int half = a.rd >> 1;
  const int p = (d - (D - a.rd)) >> 1;
  const int64_t pos = (int64_t)a.start_pos + qs;
  cs = a.cos_tab[pos * half + p];
  sn_neg = -a.sin_tab[pos * half + p];
}

// inverse rope of one adjacent pair at channel d (even) of a head_dim-D row
__device__ __forceinline__ void rope_inv_pair(const MlaArgs& a, int D, int qs, int d, float& x0, float& x1,
                                              bool round) {
  if (!in_rope_tail(a, D, d)) return;
  float cs, sn;
  rope_inv_load(a, D, qs, d, cs, sn);
  rope_inv_apply(cs, sn, x0, x1);
  if (round) {
    x0 = round_bf16(x0);
    x1 = round_bf16(x1);
  }
}

// Forward rope of the query tail (rope_tail(q, rd, cos, sin), attention.py:117) applied as q is
// loaded: the adjacent pair at channel d (even) of query qs, when d lies in the last q_rd
// channels, turns by (cos, sin) at position start_pos + qs with dsv41_rope_tail's arithmetic
// (rotate_pair).
__device__ __forceinline__ void rope_q_pair(const MlaArgs& a, int D, int qs, int d, float& x0, float& x1) {
  if (a.q_rd <= 0 || d < D - a.q_rd) return;
  const int half = a.q_rd >> 1;
  const int p = (d - (D - a.q_rd)) >> 1;
  const int64_t pos = (int64_t)a.start_pos + qs;
  rotate_pair(x0, x1, a.cos_tab[pos * half + p], a.sin_tab[pos * half + p]);
}

// The same on 8 consecutive bf16 channels c0.. of one query head (c0 a multiple of 8), each
// rotated value rounded to bf16 (channels outside the tail convert back unchanged).
__device__ __forceinline__ bf16x8 rope_q8(const MlaArgs& a, int D, int qs, int c0, bf16x8 x) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
#pragma unroll
  for (int j = 0; j < 4; ++j) rope_q_pair(a, D, qs, c0 + 2 * j, v[2 * j], v[2 * j + 1]);
  return cvt_bf16x8(v);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegFloor = -1e30f;

constexpr float kRescale = 8.0f;       // lazy softmax rescaling threshold (log2 units)
constexpr int kStepRows = 32;          // rows per pipeline step (two 16-row MFMA tiles)
constexpr int kMaxList = 2304;         // list entries one workgroup stages in LDS
constexpr int kLdsBudget = 160 * 1024;
constexpr int kPairList = 256;         // list entries of the two-per-CU decode instance (half the LDS)
constexpr int kMaxRing = 4;            // ring slots: steps in flight + the one computed


// Wait until at most `after` steps of NL copies each are still in flight (after < kMaxRing).
template <int NL>
__device__ __forceinline__ void wait_steps(int after) {
  if (after >= 3) wait_vmcnt<3 * NL>();
  else if (after == 2) wait_vmcnt<2 * NL>();
  else if (after == 1) wait_vmcnt<NL>();
  else wait_vmcnt<0>();
}

__device__ __forceinline__ bf16x8 join_bf16x8(i16x4 lo, i16x4 hi) {
  struct P { i16x4 a, b; } p{lo, hi};
  return __builtin_bit_cast(bf16x8, p);
}

// The 64-bit value lane `r` holds as (lo, hi). readlane returns a signed int: both halves are
// widened through uint32_t so the low word never sign-extends into the high one.
__device__ __forceinline__ uint64_t lane_u64(uint32_t lo, uint32_t hi, int r) {
  const uint32_t l = (uint32_t)__builtin_amdgcn_readlane((int)lo, r);
  const uint32_t h = (uint32_t)__builtin_amdgcn_readlane((int)hi, r);
  return ((uint64_t)h << 32) | (uint64_t)l;
}

// Store 4 consecutive output channels d0..d0+3 of one head: divide, round to bf16 (the
// reference's cast at the end of sparse_attn), inverse rope, round again, 8-byte store.
__device__ __forceinline__ void store_out4(const MlaArgs& a, int D, int qs, bf16_t* orow, int d0, f32x4 o, float den) {
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round_bf16(o[i] / den);
  rope_inv_pair(a, D, qs, d0, v[0], v[1], true);
  rope_inv_pair(a, D, qs, d0 + 2, v[2], v[3], true);
  uint2 st;
  st.x = pack2_bf16(v[0], v[1]);
  st.y = pack2_bf16(v[2], v[3]);
  *reinterpret_cast<uint2*>(orow + d0) = st;
}

}  // namespace dsv41
