// Sparse MLA, deepseek_v41_mlx/sparse_attention.py:34-60 (TileLang sparse_attn_kernel,
// docs/reference/kernel.py:310-403) and the attention core of attention.py:124-175.
//
// K = V: one shared [dim] row per selected position serves all heads of a query, so a query is
// a small GEMM of its [heads x dim] q block against the gathered [rows x dim] block.
//
// bf16 kernel (MFMA 16x16x32, fp32 accumulate), one workgroup = one query x (NHT*16) heads x one
// split of its index list; 4 waves share every gathered 32-row tile through LDS and split the
// head dimension between them:
//   S^T[rows x heads] = K[rows x d] Q^T[d x heads]: each wave contracts a quarter of d; the four
//     partial tiles meet in LDS and every wave sums them in the same order;
//   online softmax in log2 units, the sink seeding the running max and denominator of split 0
//     (sink in the denominator only, no value row); masked rows contribute nothing;
//   O^T[d x heads] += V^T P^T: each wave owns a quarter of d; P^T comes straight from the S^T
//     accumulators (same lane layout), V^T is read from the row-major LDS tile.
// Rows are gathered with one 1 KB coalesced read per wave per row (d = 512) and the next tile's
// reads are in flight while the current one is computed. Queries with too little parallelism
// (decode) split their index list across workgroups and a combine kernel merges the partial
// (max, denominator, numerator) triples. The epilogue divides, rounds to bf16 as the reference
// does, then applies the inverse rope to the last rd channels (attention.py:174-175).
//
// fp32 kernel: a plain FMA implementation for the 1e-5 parity configs.
#include "mfma.h"

namespace dsv41 {

struct KvSrc {
  const void* ring;  int64_t ring_bstride;  int window, wp, ring_first;
  const void* chunk; int64_t chunk_bstride; int n_chunk;
  const void* comp;  int64_t comp_bstride;  int n_comp;
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
  int splits, per_split;
  float* part_o;
  float* part_ml;
};

// Entry e of query qs's list -> unified position (-1 = none). wc = window entries of qs.
__device__ __forceinline__ int list_pos(const KvSrc& s, int b, int m, int qs, int e, int wc) {
  if (s.win_implicit) {
    if (e < wc) return s.wp + qs - wc + 1 + e;
    e -= wc;
  }
  if (e < s.k) return s.idx[((int64_t)b * m + qs) * s.k + e];
  return -1;
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

// inverse rope of one adjacent pair at channel d (even) of a head_dim-D row
__device__ __forceinline__ void rope_inv_pair(const MlaArgs& a, int D, int qs, int d, float& x0, float& x1,
                                              bool round) {
  if (a.rd <= 0 || d < D - a.rd) return;
  const int half = a.rd >> 1;
  const int p = (d - (D - a.rd)) >> 1;
  const int64_t pos = (int64_t)a.start_pos + qs;
  const float cs = a.cos_tab[pos * half + p];
  const float sn = -a.sin_tab[pos * half + p];
  const float xr = x0, xi = x1;
  x0 = __fsub_rn(__fmul_rn(xr, cs), __fmul_rn(xi, sn));
  x1 = __fadd_rn(__fmul_rn(xr, sn), __fmul_rn(xi, cs));
  if (round) {
    x0 = round_bf16(x0);
    x1 = round_bf16(x1);
  }
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegFloor = -1e30f;

template <int D, int NHT>
__global__ __launch_bounds__(256) void mla_bf16_kernel(MlaArgs a) {
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int KSW = (KS + 3) / 4, DTW = (DT + 3) / 4;
  constexpr int RS = D * 2 + 16;   // padded LDS row stride, bytes
  constexpr int CPR = D / 8;       // 16-byte chunks per row
  constexpr int CPT = D / 64;      // chunks per thread per 32-row tile
  __shared__ __align__(16) uint8_t kv_lds[32 * RS];
  __shared__ __align__(16) f32x4 xch[4][NHT][2][64];
  __shared__ uint32_t vmask_sh;

  const KvSrc& S = a.src;
  const int unit = blockIdx.x, hg = blockIdx.y, sp = blockIdx.z;
  const int b = unit / a.m, qs = unit - (unit / a.m) * a.m;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int wc = window_count(S, qs);
  const int L = wc + S.k;
  const int e_begin = sp * a.per_split;
  const int e_end = min(e_begin + a.per_split, L);
  const int ks0 = (KS * wave) / 4, ks1 = (KS * (wave + 1)) / 4;
  const int dt0 = (DT * wave) / 4, dt1 = (DT * (wave + 1)) / 4;
  const int hbase = hg * NHT * 16;
  const float sl2 = a.scale * kLog2e;

  // Q^T as the MFMA B operand: lane -> head (hbase + ht*16 + l16), k-chunk 8g of k-step ks
  bf16x8 qb[NHT][KSW];
  const bf16_t* qrow = reinterpret_cast<const bf16_t*>(a.q) + (int64_t)unit * a.heads * D;
  float m_run[NHT], l_run[NHT];
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
    const int h = hbase + ht * 16 + l16;
#pragma unroll
    for (int kk = 0; kk < KSW; ++kk) {
      const int ks = ks0 + kk;
      qb[ht][kk] = (h < a.heads && ks < ks1) ? ld_bf16x8(qrow + (int64_t)h * D + ks * 32 + 8 * g) : zero_bf16x8();
    }
    if (sp == 0 && h < a.heads) {
      const float s2 = a.sink[h] * kLog2e;
      m_run[ht] = fmaxf(s2, kNegFloor);
      l_run[ht] = exp2f(s2 - m_run[ht]);
    } else {
      m_run[ht] = kNegFloor;
      l_run[ht] = 0.0f;
    }
  }
  f32x4 acc_o[NHT][DTW];
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
    for (int dd = 0; dd < DTW; ++dd) acc_o[ht][dd] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 pf[CPT];
  auto load_tile = [&](int e0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ci = tid + 256 * c;
      const int r = ci / CPR, col = ci - (ci / CPR) * CPR;
      const int e = e0 + r;
      const bf16_t* p = e < e_end ? row_ptr<bf16_t>(S, b, list_pos(S, b, a.m, qs, e, wc), D) : nullptr;
      pf[c] = p ? *reinterpret_cast<const uint4*>(p + col * 8) : make_uint4(0, 0, 0, 0);
    }
  };

  if (e_begin < e_end) load_tile(e_begin);
  for (int e0 = e_begin; e0 < e_end; e0 += 32) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ci = tid + 256 * c;
      const int r = ci / CPR, col = ci - (ci / CPR) * CPR;
      *reinterpret_cast<uint4*>(kv_lds + r * RS + col * 16) = pf[c];
    }
    if (wave == 0) {
      bool v = false;
      if (lane < 32) {
        const int e = e0 + lane;
        v = e < e_end && row_ptr<bf16_t>(S, b, list_pos(S, b, a.m, qs, e, wc), D) != nullptr;
      }
      const uint64_t bal = __ballot(v);
      if (lane == 0) vmask_sh = (uint32_t)bal;
    }
    __syncthreads();
    const uint32_t vmask = vmask_sh;
    if (e0 + 32 < e_end) load_tile(e0 + 32);

    // partial S^T over this wave's share of d
    f32x4 sacc[NHT][2];
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) sacc[ht][0] = sacc[ht][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KSW; ++kk) {
      const int ks = ks0 + kk;
      if (ks < ks1) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const bf16x8 A = ld_bf16x8(kv_lds + (rt * 16 + l16) * RS + (ks * 32 + 8 * g) * 2);
#pragma unroll
          for (int ht = 0; ht < NHT; ++ht) sacc[ht][rt] = mfma16x16x32(A, qb[ht][kk], sacc[ht][rt]);
        }
      }
    }
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      xch[wave][ht][0][lane] = sacc[ht][0];
      xch[wave][ht][1][lane] = sacc[ht][1];
    }
    __syncthreads();

    bf16x8 pb[NHT];
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      float p[8];
      float tmax = kNegFloor;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const f32x4 s4 = ((xch[0][ht][rt][lane] + xch[1][ht][rt][lane]) + xch[2][ht][rt][lane]) + xch[3][ht][rt][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rt * 16 + 4 * g + i;
          const bool ok = (vmask >> r) & 1u;
          const float l2 = s4[i] * sl2;
          p[rt * 4 + i] = ok ? l2 : -INFINITY;
          if (ok) tmax = fmaxf(tmax, l2);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mnew = fmaxf(m_run[ht], tmax);
      const float alpha = exp2f(m_run[ht] - mnew);
      float psum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = exp2f(p[e] - mnew);
        psum += p[e];
      }
      psum += __shfl_xor(psum, 16, 64);
      psum += __shfl_xor(psum, 32, 64);
      l_run[ht] = l_run[ht] * alpha + psum;
      m_run[ht] = mnew;
#pragma unroll
      for (int dd = 0; dd < DTW; ++dd) acc_o[ht][dd] *= alpha;
      pb[ht] = pack_bf16x8(p);
    }

    // O^T += V^T P^T over this wave's share of d
#pragma unroll
    for (int dd = 0; dd < DTW; ++dd) {
      const int dt = dt0 + dd;
      if (dt < dt1) {
        const uint8_t* col = kv_lds + (dt * 16 + l16) * 2;
        uint32_t w4[4];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int r = rt * 16 + 4 * g;
          const uint32_t v0 = *reinterpret_cast<const uint16_t*>(col + (r + 0) * RS);
          const uint32_t v1 = *reinterpret_cast<const uint16_t*>(col + (r + 1) * RS);
          const uint32_t v2 = *reinterpret_cast<const uint16_t*>(col + (r + 2) * RS);
          const uint32_t v3 = *reinterpret_cast<const uint16_t*>(col + (r + 3) * RS);
          w4[rt * 2 + 0] = v0 | (v1 << 16);
          w4[rt * 2 + 1] = v2 | (v3 << 16);
        }
        const bf16x8 A = as_bf16x8(make_uint4(w4[0], w4[1], w4[2], w4[3]));
#pragma unroll
        for (int ht = 0; ht < NHT; ++ht) acc_o[ht][dd] = mfma16x16x32(A, pb[ht], acc_o[ht][dd]);
      }
    }
    __syncthreads();
  }

  if (a.splits == 1) {
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      const int h = hbase + ht * 16 + l16;
      if (h >= a.heads) continue;
      const float den = l_run[ht];
      bf16_t* orow = reinterpret_cast<bf16_t*>(a.o) + ((int64_t)unit * a.heads + h) * D;
#pragma unroll
      for (int dd = 0; dd < DTW; ++dd) {
        const int dt = dt0 + dd;
        if (dt >= dt1) continue;
        const int d0 = dt * 16 + 4 * g;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = round_bf16(acc_o[ht][dd][i] / den);
        rope_inv_pair(a, D, qs, d0, v[0], v[1], true);
        rope_inv_pair(a, D, qs, d0 + 2, v[2], v[3], true);
        uint2 st;
        st.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
        st.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
        *reinterpret_cast<uint2*>(orow + d0) = st;
      }
    }
  } else {
    const int64_t slot = ((int64_t)unit * a.splits + sp) * a.heads;
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      const int h = hbase + ht * 16 + l16;
      if (h >= a.heads) continue;
      float* po = a.part_o + (slot + h) * D;
#pragma unroll
      for (int dd = 0; dd < DTW; ++dd) {
        const int dt = dt0 + dd;
        if (dt < dt1) *reinterpret_cast<f32x4*>(po + dt * 16 + 4 * g) = acc_o[ht][dd];
      }
      if (wave == 0 && g == 0) {
        a.part_ml[(slot + h) * 2 + 0] = m_run[ht];
        a.part_ml[(slot + h) * 2 + 1] = l_run[ht];
      }
    }
  }
}

// Merges split partials (log2-domain max, denominator, numerator) of one (query, head).
template <typename T>
__global__ __launch_bounds__(128) void mla_combine_kernel(MlaArgs a) {
  const int unit = blockIdx.x, h = blockIdx.y;
  const int D = a.dim;
  const int qs = unit % a.m;
  const int64_t slot0 = (int64_t)unit * a.splits * a.heads;
  float M = kNegFloor;
  for (int sp = 0; sp < a.splits; ++sp) M = fmaxf(M, a.part_ml[(slot0 + (int64_t)sp * a.heads + h) * 2]);
  float den = 0.0f;
  for (int sp = 0; sp < a.splits; ++sp) {
    const float* ml = a.part_ml + (slot0 + (int64_t)sp * a.heads + h) * 2;
    den += ml[1] * exp2f(ml[0] - M);
  }
  T* orow = reinterpret_cast<T*>(a.o) + ((int64_t)unit * a.heads + h) * D;
  for (int p = threadIdx.x; p < D / 2; p += 128) {
    float x0 = 0.0f, x1 = 0.0f;
    for (int sp = 0; sp < a.splits; ++sp) {
      const int64_t slot = slot0 + (int64_t)sp * a.heads + h;
      const float wgt = exp2f(a.part_ml[slot * 2] - M);
      const float* po = a.part_o + slot * D + 2 * p;
      x0 += po[0] * wgt;
      x1 += po[1] * wgt;
    }
    x0 = io<T>::rnd(x0 / den);
    x1 = io<T>::rnd(x1 / den);
    rope_inv_pair(a, D, qs, 2 * p, x0, x1, false);
    io<T>::st(orow + 2 * p, x0);
    io<T>::st(orow + 2 * p + 1, x1);
  }
}

// fp32: 4 heads x 16 rows per step, plain FMA, natural-log softmax with the reference's form.
constexpr int kF32Heads = 4;
constexpr int kF32Rows = 16;
constexpr int kF32MaxDim = 768;

__global__ __launch_bounds__(256) void mla_f32_kernel(MlaArgs a) {
  extern __shared__ float smf[];
  const int D = a.dim;
  float* q_l = smf;                        // [4][D]
  float* kv_l = smf + kF32Heads * D;       // [16][D]
  __shared__ float lg[kF32Heads][kF32Rows];
  __shared__ float mrun[kF32Heads], lrun[kF32Heads], alph[kF32Heads];
  __shared__ const float* rp[kF32Rows];
  const KvSrc& S = a.src;
  const int unit = blockIdx.x, hbase = blockIdx.y * kF32Heads;
  const int b = unit / a.m, qs = unit - (unit / a.m) * a.m;
  const int tid = threadIdx.x;
  const int wc = window_count(S, qs);
  const int L = wc + S.k;
  const float* qrow = reinterpret_cast<const float*>(a.q) + (int64_t)unit * a.heads * D;
  for (int i = tid; i < kF32Heads * D; i += 256) {
    const int h = hbase + i / D;
    q_l[i] = h < a.heads ? qrow[(int64_t)h * D + i % D] : 0.0f;
  }
  if (tid < kF32Heads) {
    const int h = hbase + tid;
    const float sk = h < a.heads ? a.sink[h] : -INFINITY;
    mrun[tid] = fmaxf(sk, kNegFloor);
    lrun[tid] = expf(sk - mrun[tid]);
  }
  constexpr int PJ = (kF32MaxDim / 2 + 255) / 256;
  float o[kF32Heads][PJ][2];
#pragma unroll
  for (int h = 0; h < kF32Heads; ++h)
#pragma unroll
    for (int j = 0; j < PJ; ++j) o[h][j][0] = o[h][j][1] = 0.0f;

  for (int e0 = 0; e0 < L; e0 += kF32Rows) {
    __syncthreads();
    if (tid < kF32Rows) {
      const int e = e0 + tid;
      rp[tid] = e < L ? row_ptr<float>(S, b, list_pos(S, b, a.m, qs, e, wc), D) : nullptr;
    }
    __syncthreads();
    for (int i = tid; i < kF32Rows * D; i += 256) {
      const float* p = rp[i / D];
      kv_l[i] = p ? p[i % D] : 0.0f;
    }
    __syncthreads();
    {
      const int di = tid >> 2, part = tid & 3;
      const int h = di >> 4, r = di & 15;
      const int q4 = D / 4;
      float acc = 0.0f;
      for (int d = part * q4; d < (part + 1) * q4; ++d) acc += q_l[h * D + d] * kv_l[r * D + d];
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      if (part == 0) lg[h][r] = rp[r] ? acc * a.scale : kNegFloor;
    }
    __syncthreads();
    if (tid < kF32Heads) {
      float tmax = kNegFloor;
      for (int r = 0; r < kF32Rows; ++r)
        if (rp[r]) tmax = fmaxf(tmax, lg[tid][r]);
      const float mnew = fmaxf(mrun[tid], tmax);
      const float al = expf(mrun[tid] - mnew);
      float ps = 0.0f;
      for (int r = 0; r < kF32Rows; ++r) {
        const float pv = rp[r] ? expf(lg[tid][r] - mnew) : 0.0f;
        lg[tid][r] = pv;
        ps += pv;
      }
      lrun[tid] = lrun[tid] * al + ps;
      mrun[tid] = mnew;
      alph[tid] = al;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int d = 2 * (tid + 256 * j);
      if (d >= D) continue;
#pragma unroll
      for (int h = 0; h < kF32Heads; ++h) {
        float x0 = o[h][j][0] * alph[h], x1 = o[h][j][1] * alph[h];
        for (int r = 0; r < kF32Rows; ++r) {
          x0 += lg[h][r] * kv_l[r * D + d];
          x1 += lg[h][r] * kv_l[r * D + d + 1];
        }
        o[h][j][0] = x0;
        o[h][j][1] = x1;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < kF32Heads; ++h) {
    const int hh = hbase + h;
    if (hh >= a.heads) continue;
    float* orow = reinterpret_cast<float*>(a.o) + ((int64_t)unit * a.heads + hh) * D;
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int d = 2 * (tid + 256 * j);
      if (d >= D) continue;
      float x0 = o[h][j][0] / lrun[h], x1 = o[h][j][1] / lrun[h];
      rope_inv_pair(a, D, qs, d, x0, x1, false);
      orow[d] = x0;
      orow[d + 1] = x1;
    }
  }
}

// ------------------------------------------------------------------ host planning

struct MlaPlan {
  int nht, hgroups, splits, per_split;
};

static MlaPlan plan_bf16(int64_t units, int heads, int list_max) {
  const int hg16 = (heads + 15) / 16;
  MlaPlan p{};
  p.nht = hg16 >= 4 ? 4 : (hg16 >= 2 ? 2 : 1);
  p.hgroups = (hg16 + p.nht - 1) / p.nht;
  p.splits = 1;
  if (units * p.hgroups < 256) {
    p.nht = 1;
    p.hgroups = hg16;
    const int64_t wgs = units * p.hgroups;
    if (wgs < 256) {
      int want = (int)((256 + wgs - 1) / wgs);
      int cap = list_max / 64;
      if (cap < 1) cap = 1;
      if (want > cap) want = cap;
      if (want > 16) want = 16;
      p.splits = want;
    }
  }
  const int lm = list_max > 0 ? list_max : 1;
  p.per_split = ((lm + p.splits - 1) / p.splits + 31) / 32 * 32;
  p.splits = (lm + p.per_split - 1) / p.per_split;
  return p;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t workspace_for(const MlaPlan& p, int64_t units, int heads, int dim) {
  if (p.splits <= 1) return 0;
  const size_t slots = (size_t)units * p.splits * heads;
  return align256(slots * dim * sizeof(float)) + align256(slots * 2 * sizeof(float));
}

static bool bf16_dim_supported(int d) { return d == 64 || d == 128 || d == 256 || d == 512 || d == 576; }

template <int D>
static void launch_bf16_d(const MlaArgs& a, const MlaPlan& p, int64_t units, hipStream_t stream) {
  dim3 grid((unsigned)units, (unsigned)p.hgroups, (unsigned)p.splits);
  if (p.nht == 4) hipLaunchKernelGGL((mla_bf16_kernel<D, 4>), grid, dim3(256), 0, stream, a);
  else if (p.nht == 2) hipLaunchKernelGGL((mla_bf16_kernel<D, 2>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((mla_bf16_kernel<D, 1>), grid, dim3(256), 0, stream, a);
}

static int run_mla(const char* what, MlaArgs a, int64_t units, int list_max, int dtype, void* workspace,
                   size_t workspace_bytes, hipStream_t stream) {
  if (units == 0) return 0;
  DSV41_REQUIRE(units < (1ll << 31), DSV41_E_ARG, "%s: too many queries", what);
  if (dtype == DSV41_F32) {
    DSV41_REQUIRE(a.dim % 4 == 0 && a.dim <= kF32MaxDim, DSV41_E_SHAPE, "%s: fp32 path needs dim %% 4 == 0, <= %d",
                  what, kF32MaxDim);
    a.splits = 1;
    a.per_split = list_max;
    const size_t smem = (size_t)(kF32Heads + kF32Rows) * a.dim * sizeof(float);
    dim3 grid((unsigned)units, (unsigned)((a.heads + kF32Heads - 1) / kF32Heads), 1);
    hipLaunchKernelGGL(mla_f32_kernel, grid, dim3(256), smem, stream, a);
    return check_launch(what);
  }
  if (dtype != DSV41_BF16) return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  DSV41_REQUIRE(bf16_dim_supported(a.dim), DSV41_E_SHAPE, "%s: bf16 path supports dim 64/128/256/512/576, got %d",
                what, a.dim);
  const MlaPlan p = plan_bf16(units, a.heads, list_max);
  a.splits = p.splits;
  a.per_split = p.per_split;
  const size_t need = workspace_for(p, units, a.heads, a.dim);
  if (need) {
    DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed",
                  what, need);
    DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
    const size_t slots = (size_t)units * p.splits * a.heads;
    a.part_o = reinterpret_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + align256(slots * a.dim * sizeof(float)));
  }
  switch (a.dim) {
    case 64: launch_bf16_d<64>(a, p, units, stream); break;
    case 128: launch_bf16_d<128>(a, p, units, stream); break;
    case 256: launch_bf16_d<256>(a, p, units, stream); break;
    case 512: launch_bf16_d<512>(a, p, units, stream); break;
    default: launch_bf16_d<576>(a, p, units, stream); break;
  }
  int rc = check_launch(what);
  if (rc || p.splits == 1) return rc;
  hipLaunchKernelGGL(mla_combine_kernel<bf16_t>, dim3((unsigned)units, (unsigned)a.heads), dim3(128), 0, stream, a);
  return check_launch(what);
}

}  // namespace dsv41

using namespace dsv41;

extern "C" size_t dsv41_sparse_mla_workspace_bytes(int32_t bsz, int32_t m, int32_t heads, int32_t dim,
                                                   int32_t rows_per_query, int32_t dtype) {
  if (dtype != DSV41_BF16 || bsz <= 0 || m <= 0 || heads <= 0 || dim <= 0) return 0;
  const int64_t units = (int64_t)bsz * m;
  return workspace_for(plan_bf16(units, heads, rows_per_query), units, heads, dim);
}

extern "C" int dsv41_sparse_attn(const void* q, const void* kv, const float* sink, const int32_t* idx, void* o,
                                 int32_t bsz, int32_t m, int32_t heads, int32_t dim, int32_t nkv, int32_t k,
                                 float scale, int32_t dtype, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  const char* what = "dsv41_sparse_attn";
  DSV41_REQUIRE(q && kv && sink && o && (idx || k == 0), DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && m >= 0 && heads > 0 && dim > 0 && nkv >= 0 && k >= 0, DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dim % 32 == 0, DSV41_E_SHAPE, "%s: dim %d must be a multiple of 32", what, dim);
  DSV41_REQUIRE(aligned16(q) && aligned16(kv) && aligned16(o), DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  MlaArgs a{};
  a.q = q; a.o = o; a.sink = sink;
  a.src.chunk = kv; a.src.chunk_bstride = (int64_t)nkv * dim; a.src.n_chunk = nkv;
  a.src.window = 1; a.src.wp = 0; a.src.ring_first = 0;
  a.src.idx = idx; a.src.k = k; a.src.win_implicit = 0;
  a.m = m; a.heads = heads; a.dim = dim; a.scale = scale; a.rd = 0;
  return run_mla(what, a, (int64_t)bsz * m, k, dtype, workspace, workspace_bytes, stream);
}

extern "C" int dsv41_sparse_mla(const void* q, const void* win_kv, const void* chunk_kv, const void* comp_kv,
                                int64_t comp_bstride, int32_t n_comp, const float* sink, const int32_t* idx, int32_t k,
                                void* o, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t window,
                                int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab, int32_t rd,
                                int32_t dtype, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* what = "dsv41_sparse_mla";
  const int wp = start_pos < window ? start_pos : window;
  DSV41_REQUIRE(q && chunk_kv && sink && o && (idx || k == 0) && (win_kv || wp == 0) && (comp_kv || n_comp == 0),
                DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && dim > 0 && window > 0 && start_pos >= 0 && k >= 0 && n_comp >= 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dim % 32 == 0, DSV41_E_SHAPE, "%s: dim %d must be a multiple of 32", what, dim);
  DSV41_REQUIRE(n_comp == 0 || comp_bstride >= (int64_t)n_comp * dim, DSV41_E_ARG, "%s: comp_bstride too small", what);
  DSV41_REQUIRE(aligned16(q) && aligned16(chunk_kv) && aligned16(o) && (!win_kv || aligned16(win_kv)) &&
                    (!comp_kv || aligned16(comp_kv)),
                DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  DSV41_REQUIRE(comp_bstride % 8 == 0, DSV41_E_ARG, "%s: comp_bstride must be a multiple of 8", what);
  DSV41_REQUIRE(rd == 0 || (cos_tab && sin_tab && rd % 2 == 0 && rd <= dim), DSV41_E_ARG, "%s: bad rope tail", what);
  MlaArgs a{};
  a.q = q; a.o = o; a.sink = sink;
  a.src.ring = win_kv; a.src.ring_bstride = (int64_t)window * dim; a.src.window = window; a.src.wp = wp;
  a.src.ring_first = (start_pos - wp) % window;
  a.src.chunk = chunk_kv; a.src.chunk_bstride = (int64_t)n * dim; a.src.n_chunk = n;
  a.src.comp = comp_kv; a.src.comp_bstride = comp_bstride; a.src.n_comp = n_comp;
  a.src.idx = idx; a.src.k = k; a.src.win_implicit = 1;
  a.m = n; a.heads = heads; a.dim = dim; a.scale = scale;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.start_pos = start_pos;
  const int weff = window < wp + n ? window : wp + n;
  return run_mla(what, a, (int64_t)bsz * n, weff + k, dtype, workspace, workspace_bytes, stream);
}
