// Indexer scoring, deepseek_v41_mlx/indexer.py:123-138:
//   S[b,s,t] = sum_h relu(q[b,s,h,:] . k[b,t,:]) * w[b,s,h],  t >= lens_s -> -inf,
//   candidate-masked -> -inf, with w = round_dtype(w_raw * w_scale).
//
// Kernels (bf16 MFMA with fp32 accumulation unless noted; heads = MFMA M, cache rows = N; each
// lane ends with 4 heads x 1 row, ReLU * w and the head sum run on the accumulators):
//   indexer_decode_kernel     few queries, 128-channel bf16 or fp8 keys: key tiles move by
//                             non-temporal LDS copies into per-wave rings (the decode path);
//   indexer_prefill_kernel    chunked prefill: 8 queries per workgroup share 64-row key chunks
//                             staged once in a swizzled LDS ring;
//   indexer_score_mx_kernel   MXFP4 keys and query: block-scaled fp4 MFMA, operands loaded
//                             straight into registers;
//   indexer_score_bf16_kernel the register kernel for the remaining shapes (other head counts
//                             and key widths, unaligned fp8 scale rows): keys stream straight
//                             from HBM into VGPRs, two batches of four tiles in flight;
//   indexer_score_f32_kernel  the fp32 parity path.
// Rows past a query's visibility are written as -inf without touching the cache (causal
// prefill skips about half the bytes).
#include "mfma.h"
#include "select.h"

namespace dsv41 {

constexpr int kIdxThreads = 512;  // 8 waves

// One batch of U 16-row key tiles in the MFMA B-operand layout: bf16 rows, or (F8) e4m3 codes
// with the row block's ue8m0 scale bytes (one per 32 channels), dequantized to bf16 at use.
template <bool F8, int U, int KS> struct KeyBatch;
template <int U, int KS> struct KeyBatch<false, U, KS> {
  bf16x8 k[U][KS];
  uint32_t cf[U];
  __device__ __forceinline__ bf16x8 op(int u, int ks) const { return k[u][ks]; }
};
template <int U, int KS> struct KeyBatch<true, U, KS> {
  uint2 k[U][KS];
  uint32_t sc[U];
  uint32_t cf[U];
  __device__ __forceinline__ bf16x8 op(int u, int ks) const {
    return dequant_e4m3x8(k[u][ks].x, k[u][ks].y, e8m0_to_float((sc[u] >> (8 * ks)) & 255u));
  }
};

template <int HT, int KS, bool F8>
__global__ __launch_bounds__(kIdxThreads) void indexer_score_bf16_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ w_raw, float w_scale,
    const void* __restrict__ kcache, int64_t k_bstride, const uint8_t* __restrict__ kscale, int64_t ks_bstride,
    int ks_rb, const uint8_t* __restrict__ cand, float* __restrict__ scores, int n, int nb, int start_pos, int ratio,
    int rows_per_wg, int heads) {
  static_assert(!F8 || KS == 4, "fp8 keys: 128 channels (four scale bytes per row block)");
  // H = the head tiles' rows; heads <= H are real. The rows past `heads` hold a zero query and a
  // zero weight, so each adds exactly +0 to the score.
  constexpr int H = HT * 16;
  constexpr int DIM = KS * 32;
  constexpr int QROW = DIM * 2 + 16;       // padded LDS row stride in bytes
  __shared__ __align__(16) uint8_t q_lds[H * QROW];

  const int qi = blockIdx.y;               // b * n + s
  const int b = qi / n, s = qi - (qi / n) * n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int lens = (start_pos + s + 1) / ratio;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(r0 + rows_per_wg, nb);
  const int vis_end = max(r0, min(r1, lens));
  float* out = scores + (int64_t)qi * nb;
  for (int t = vis_end + tid; t < r1; t += kIdxThreads) out[t] = -INFINITY;
  if (vis_end <= r0) return;               // uniform: nothing visible in this row range

  bf16x8 qa[HT][KS];                       // the query block as the MFMA A operand (heads = M)
  float wv[HT][4];                         // head weights of this lane's 4 heads per head tile

  // natural MFMA k order (k = 32 ks + 8 g + i): one load instruction reads a contiguous 64-byte
  // (fp8: 32-byte) span of each of its 16 rows
  const bf16_t* kb = reinterpret_cast<const bf16_t*>(kcache) + (int64_t)b * k_bstride + g * 8;
  const uint8_t* kb8 = reinterpret_cast<const uint8_t*>(kcache) + (int64_t)b * k_bstride + g * 8;
  const uint8_t* ksb = F8 ? kscale + (int64_t)b * ks_bstride : nullptr;
  const uint8_t* cb = cand ? cand + (int64_t)qi * nb : nullptr;
  constexpr int NW = kIdxThreads / 64;

  // Four 16-row tiles per batch; the next batch is always in flight while the current one is
  // computed (two register sets). Loads are unconditional -- rows past the visible range are
  // clamped onto its last row -- so every batch issues the same number of loads and the
  // compiler's wait counts stay exact across iterations.
  constexpr int U = HT >= 8 ? 2 : 4;       // 128 heads: the query block alone takes 128 VGPRs
  constexpr int STRIDE = 16 * U * NW;
  // candidate flags of a batch travel with its key loads, so no load is issued behind the batch
  // that is waited on before it
  using Batch = KeyBatch<F8, U, KS>;
  auto load = [&](Batch& kk, int t0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = min(t0 + 16 * u + l16, vis_end - 1);   // clamp: loads stay inside the cache
      if constexpr (F8) {
        const uint8_t* kr = kb8 + (int64_t)row * DIM;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kk.k[u][ks] = *reinterpret_cast<const uint2*>(kr + ks * 32);
        kk.sc[u] = *reinterpret_cast<const uint32_t*>(ksb + (int64_t)(row / ks_rb) * 4);
      } else {
        const bf16_t* kr = kb + (int64_t)row * DIM;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kk.k[u][ks] = ld_bf16x8(kr + ks * 32);
      }
      kk.cf[u] = cb ? (uint32_t)cb[row] : 1u;
    }
  };
  auto compute = [&](const Batch& kk, int t0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tb = t0 + 16 * u;
      f32x4 acc[HT];
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kop = kk.op(u, ks);
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma16x16x32(qa[ht][ks], kop, acc[ht]);
      }
      float part = 0.0f;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int i = 0; i < 4; ++i) part += relu_bits(acc[ht][i]) * wv[ht][i];
      part = sum_rows4(part);
      const int row = tb + l16;
      if (g == 0 && row < vis_end) {
        out[row] = kk.cf[u] ? part : -INFINITY;
      }
    }
  };
  int t0 = r0 + 16 * U * wave;
  // Stage q[b, s] ([H, DIM] bf16) through LDS, with the first key batch already in flight: the
  // query's global loads go out first, then every wave's first batch (unconditional and clamped,
  // so the wait counts stay exact), then the LDS store and the barrier.
  constexpr int QN = (H * DIM / 8 + kIdxThreads - 1) / kIdxThreads;
  const uint4* qrow = reinterpret_cast<const uint4*>(q + (int64_t)qi * heads * DIM);
  uint4 qv[QN];
#pragma unroll
  for (int c = 0; c < QN; ++c) {
    const int e = tid + c * kIdxThreads;
    qv[c] = e < heads * DIM / 8 ? qrow[e] : make_uint4(0u, 0u, 0u, 0u);
  }
  Batch ka, kb2;
  load(ka, min(t0, vis_end - 1));
#pragma unroll
  for (int c = 0; c < QN; ++c) {
    const int e = tid + c * kIdxThreads;
    if (e < H * DIM / 8) {
      const int h = e / (DIM / 8), d8 = e - h * (DIM / 8);
      *reinterpret_cast<uint4*>(q_lds + h * QROW + d8 * 16) = qv[c];
    }
  }
  __syncthreads();
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qa[ht][ks] = ld_bf16x8(q_lds + (ht * 16 + l16) * QROW + (ks * 32 + g * 8) * 2);
  {
    const bf16_t* wrow = w_raw + (int64_t)qi * heads;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = ht * 16 + 4 * g + i;
        wv[ht][i] = h < heads ? round_bf16(bf2f(wrow[h]) * w_scale) : 0.0f;
      }
  }
  if (t0 >= vis_end) return;
  for (;;) {
    load(kb2, t0 + STRIDE);
    compute(ka, t0);
    t0 += STRIDE;
    if (t0 >= vis_end) break;
    load(ka, t0 + STRIDE);
    compute(kb2, t0);
    t0 += STRIDE;
    if (t0 >= vis_end) break;
  }
}

// 128-channel keys, the decode shape (few queries, long cache): the same scores as
// indexer_score_bf16_kernel, with the key stream moved by LDS copies. Wave w of the workgroup
// takes 16-row tiles w, w + 8, w + 16, ... of the row range; each tile is 1 KB global_load_lds
// copies of whole rows (non-temporal) into the wave's private ring of kDecSlots tiles, read back
// in the MFMA operand layout. A copy's lane lands at tile row (rows per copy) * k + lane / (chunks
// per row) and fetches a column chunk XOR-swizzled by that row, so that the operand reads of 16
// rows hit disjoint bank groups. bf16 rows (256 B): 4 copies per tile, chunk ^ row. fp8 rows
// (e4m3 codes, 128 B): 2 copies per tile, chunk ^ ((row >> 1) & 7); the row block's ue8m0 scale
// words (one byte per 32 channels, one word per `rb` rows) are staged for the whole row range
// up front, and each operand is dequantized on the way to the MFMA (exact in bf16), in the same
// channel order as the bf16 kernel, so both forms give the same bits. The query block and the
// head weights arrive by copies too, the scores collect in LDS and leave in one coalesced pass at
// the end (candidate mask and -inf past visibility applied there): between the first copy and
// the last wait a wave issues no other vector-memory operation, so its vmcnt waits count exactly
// its own copies.
constexpr int kIdxMaxRows = 4096;        // rows per workgroup (idx_grid's bound)
constexpr int kDecWaves = 8;

template <bool F8> struct DecKeys {
  static constexpr int ROW = F8 ? 128 : 256;   // bytes per key row
  static constexpr int TILE = 16 * ROW;        // one 16-row tile
  static constexpr int CPT = TILE / 1024;      // 1 KB copies per tile
  static constexpr int CPR = ROW / 16;         // 16-byte chunks per row
  static constexpr int SLOTS = F8 ? 3 : 2;     // ring depth per wave: tiles in flight + the one scored
  static constexpr int SCALES = F8 ? kIdxMaxRows * 4 : 0;   // staged scale bytes (rb = 1 at most rows)
  __device__ static int swz(int rloc) { return F8 ? ((rloc >> 1) & 7) : (rloc & 15); }
};

// TJ > 0: the fused top-k form (decode). Instead of writing its scores, the workgroup selects
// the best min(topk, rows) of its row range (TJ scores per thread, ties -> lowest position) and
// writes them in position order as (order key, position) at ckey/cpos[(qi * chunks + range) *
// topk ...]; topk_merge_launch then selects each query's topk from those lists. The range's
// best topk contain every entry of the row's best topk, so the result is the top-k of the
// scores exactly.
template <int HT, int NW, bool F8, int TJ>
__global__ __launch_bounds__(NW * 64) void indexer_decode_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ w_raw, float w_scale, const void* __restrict__ kcache,
    int64_t k_bstride, const uint8_t* __restrict__ kscale, int64_t ks_bstride, int ks_rb,
    const uint8_t* __restrict__ cand, float* __restrict__ scores, int n, int nb, int start_pos, int ratio,
    int rows_per_wg, int topk, uint32_t* __restrict__ ckey, int32_t* __restrict__ cpos) {
  using K = DecKeys<F8>;
  constexpr int H = HT * 16, DIM = 128, KS = 4, QROW = DIM * 2;
  constexpr int QCOPIES = H * QROW / 1024;                 // 1 KB copies of the query block
  constexpr int QPW = (QCOPIES + NW - 1) / NW;             // per wave (waves past the block issue none)
  constexpr int QSC = H * QROW > kIdxMaxRows * 4 ? H * QROW : kIdxMaxRows * 4;
  static_assert(H * 2 % 16 == 0, "the head-weight row is whole 16-byte chunks");
  __shared__ __align__(16) uint8_t ring[NW * K::SLOTS * K::TILE];
  __shared__ __align__(16) uint8_t q_lds[QSC];   // the query block; then, once every wave holds it, the scores
  __shared__ __align__(16) uint8_t s_lds[K::SCALES > 0 ? K::SCALES : 16];
  // the head-weight row lands in the last wave's last ring slot, which no tile uses before the loop
  const uint8_t* w_lds = ring + ((NW - 1) * K::SLOTS + K::SLOTS - 1) * K::TILE;
  float* sc_lds = reinterpret_cast<float*>(q_lds);

  const int qi = blockIdx.y;               // b * n + s
  const int b = qi / n, s = qi - (qi / n) * n;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lens = (start_pos + s + 1) / ratio;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(r0 + rows_per_wg, nb);
  const int vis_end = max(r0, min(r1, lens));
  float* out = TJ ? nullptr : scores + (int64_t)qi * nb;
  const int64_t cbase = ((int64_t)qi * gridDim.x + blockIdx.x) * topk;   // this range's list (TJ > 0)
  if (vis_end <= r0) {                     // uniform: nothing visible in this row range
    if constexpr (TJ > 0) {                // all -inf: the lowest positions are the best
      for (int t = tid; t < min(topk, r1 - r0); t += NW * 64) {
        ckey[cbase + t] = order_key(-INFINITY);
        cpos[cbase + t] = r0 + t;
      }
    } else {
      for (int t = r0 + tid; t < r1; t += NW * 64) out[t] = -INFINITY;
    }
    return;
  }
  const int nt = (vis_end - r0 + 16 * NW - 1) / (16 * NW);   // tiles per wave (the last ones clamped)
  const uint8_t* kb = reinterpret_cast<const uint8_t*>(kcache) + (int64_t)b * k_bstride * (F8 ? 1 : 2);
  const uint32_t ring_w = lds_offset(ring) + (uint32_t)(wave * K::SLOTS * K::TILE);
  auto issue = [&](int i) {                // tile i of this wave into slot i % SLOTS
    const int ti = min(i, nt - 1);
    const int slot = i % K::SLOTS;
#pragma unroll
    for (int k = 0; k < K::CPT; ++k) {
      const int rloc = (1024 / K::ROW) * k + lane / K::CPR;
      const int row = min(r0 + 16 * (NW * ti + wave) + rloc, vis_end - 1);   // clamp: stays in the cache
      const int col = (lane % K::CPR) ^ K::swz(rloc);
      const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(ring_w + (uint32_t)(slot * K::TILE + k * 1024));
      dma16_vaddr_nt(reinterpret_cast<uint64_t>(kb + (int64_t)row * K::ROW + col * 16), dst);
    }
  };
  const int ssh = ks_rb == 32 ? 5 : 0;     // rows per scale word: 32 or 1
  {
    const uint8_t* qb = reinterpret_cast<const uint8_t*>(q + (int64_t)qi * H * DIM);
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      const int c = wave * QPW + j;        // uniform
      if (c < QCOPIES) {
        const int rloc = c * 4 + (lane >> 4);
        const int col = (lane & 15) ^ (rloc & 15);
        dma16_vaddr(reinterpret_cast<uint64_t>(qb + rloc * QROW + col * 16),
                    (uint32_t)__builtin_amdgcn_readfirstlane(lds_offset(q_lds) + (uint32_t)(c * 1024)));
      }
    }
    if (wave == NW - 1) {                  // the H-entry weight row: lanes past it re-read its last chunk
      const uint8_t* wb = reinterpret_cast<const uint8_t*>(w_raw + (int64_t)qi * H);
      dma16_vaddr(reinterpret_cast<uint64_t>(wb + min(lane, H * 2 / 16 - 1) * 16),
                  (uint32_t)__builtin_amdgcn_readfirstlane(ring_w + (uint32_t)((K::SLOTS - 1) * K::TILE)));
    }
    if constexpr (F8) {
      // scale words of rows [r0, vis_end): bytes [(r0 >> ssh) * 4, ((vis_end - 1 >> ssh) + 1) * 4) of the
      // batch row, 16-byte aligned at the start (r0 is a multiple of 512); chunks past the end are
      // clamped onto the last one, which stays inside the 16-byte-multiple batch stride
      const uint8_t* sb = kscale + (int64_t)b * ks_bstride + (int64_t)(r0 >> ssh) * 4;
      const int nsc = (((vis_end - 1) >> ssh) - (r0 >> ssh) + 1) * 4;
      const int nch = (nsc + 15) / 16;
      for (int c = wave; c * 64 < nch; c += NW) {   // uniform per wave
        const int ch = min(c * 64 + lane, nch - 1);
        dma16_vaddr(reinterpret_cast<uint64_t>(sb + ch * 16),
                    (uint32_t)__builtin_amdgcn_readfirstlane(lds_offset(s_lds) + (uint32_t)(c * 1024)));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < K::SLOTS - 1; ++i) issue(i);
  wait_vmcnt<K::CPT * (K::SLOTS - 1)>();   // this wave's query / weight / scale copies landed
  __syncthreads();                         // ... and every other wave's
  bf16x8 qa[HT][KS];
  float wv[HT][4];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qa[ht][ks] = ld_bf16x8(q_lds + (ht * 16 + l16) * QROW + (((ks * 4 + g) ^ l16) * 16));
  {
    const bf16_t* wl = reinterpret_cast<const bf16_t*>(w_lds);
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[ht][i] = round_bf16(bf2f(wl[ht * 16 + 4 * g + i]) * w_scale);
  }
  __syncthreads();                         // every wave holds its query operands and weights: q_lds takes
                                           // scores, the last ring slot its first tile
  for (int i = 0; i < nt; ++i) {
    issue(i + K::SLOTS - 1);               // past the last tile: a clamped re-read, so counts stay exact
    wait_vmcnt<K::CPT * (K::SLOTS - 1)>(); // tile i landed
    const uint8_t* rowp = ring + (wave * K::SLOTS + i % K::SLOTS) * K::TILE + l16 * K::ROW;
    f32x4 acc[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) acc[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint32_t sw = 0u;
    if constexpr (F8) {                    // the scale word of this lane's (clamped) row
      const int row = min(r0 + 16 * (NW * i + wave) + l16, vis_end - 1);
      sw = *reinterpret_cast<const uint32_t*>(s_lds + ((row >> ssh) - (r0 >> ssh)) * 4);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 kop;
      if constexpr (F8) {                  // channels 32 ks + 8 g .. +8: half (g & 1) of chunk 2 ks + g / 2
        const uint2 c8 = *reinterpret_cast<const uint2*>(rowp + (((2 * ks + (g >> 1)) ^ K::swz(l16)) * 16) +
                                                         8 * (g & 1));
        kop = dequant_e4m3x8(c8.x, c8.y, e8m0_to_float((sw >> (8 * ks)) & 255u));
      } else {
        kop = ld_bf16x8(rowp + (((ks * 4 + g) ^ l16) * 16));
      }
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma16x16x32(qa[ht][ks], kop, acc[ht]);
    }
    float part = 0.0f;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) part += relu_bits(acc[ht][i2]) * wv[ht][i2];
    part = sum_rows4(part);
    if (g == 0) sc_lds[16 * (NW * i + wave) + l16] = part;
  }
  wait_vmcnt<0>();                         // no copy may land in LDS after the workgroup ends
  __syncthreads();                         // every score of the range is in LDS
  const uint8_t* cb = cand ? cand + (int64_t)qi * nb : nullptr;
  auto value = [&](int t) {                // the score of row r0 + t as the unfused form writes it
    return (t < vis_end - r0 && (!cb || cb[r0 + t])) ? sc_lds[t] : -INFINITY;
  };
  if constexpr (TJ > 0) {
    static_assert(TJ % 4 == 0 || TJ < 4, "keys per thread");
    RegSelShared& sh = *reinterpret_cast<RegSelShared*>(ring);   // the ring is free past the loop
    const int count = r1 - r0;
    const int i0 = tid * TJ;
    const int nvalid = min(max(count - i0, 0), TJ);
    uint32_t key[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) key[j] = j < nvalid ? order_key(value(i0 + j)) : 0u;
    select_top<TJ, NW * 64>(key, nvalid, min(topk, count), sh, [&](uint32_t rank, int j) {
      ckey[cbase + rank] = order_key(value(i0 + j));             // re-read: j is a run-time index
      cpos[cbase + rank] = r0 + i0 + j;
    });
  } else {
    for (int t = tid; t < r1 - r0; t += NW * 64) out[r0 + t] = value(t);
  }
}

// MXFP4 keys: the index cache holds each 128-channel key as fp4 e2m1 codes (64 bytes; byte p
// carries channels 2p and 2p+1, the even one in the low nibble) plus one ue8m0 scale byte per
// 32 channels (4 bytes) -- the lossless packed form of the fake_quant_fp4_ue8m0 keys that
// indexer.py:100-104 stores. The query comes in the same form (its prologue, indexer.py:119-121,
// quantizes it), so each lane loads its A operand -- 16 code bytes and a scale of one
// (head, 32-channel block) -- straight into registers: no staging, no barrier. Each 16-head x
// 16-row tile is one block-scaled fp4 MFMA over all 128 channels (16x16x128, e8m0 scales per
// 32-channel block on both operands, fp32 accumulate). The products are exact and the sums are
// fp32, as in the bf16 kernel; the epilogue (ReLU * w, head sum, masks) is the same.
typedef __attribute__((ext_vector_type(8))) int i32x8;

__device__ __forceinline__ f32x4 mfma_mxfp4(uint4 a, int sa, uint4 b, int sb) {
  const i32x8 av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  const i32x8 bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
  // cbsz = blgp = 4: both operands fp4 e2m1; scale bytes in byte 0 (opsel 0)
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, f32x4{0.f, 0.f, 0.f, 0.f}, 4, 4, 0, sa, 0, sb);
}

// fp8 keys: an fp4 e2m1 query (A, cbsz = 4) against e4m3 keys (B, blgp = 0). With 8-bit
// operands the 16x16x128 instruction takes a lane group's 32 bytes as two 16-channel halves:
// lane group g supplies channels [16g, 16g+16) in bytes 0-15 and [64+16g, 64+16g+16) in bytes
// 16-31 (a one-wave probe on the box pinned this against a float64 reference), while its scale
// byte is that of channel block g, like the fp4 operand's contiguous 32 channels. Products are
// exact; the probe measured the instruction's sums within 3e-5 of max|D| of the exact sum (a
// float32 channel-order sum of the same products was exact), so these scores are close to, not
// bit-equal with, the dequantizing kernel's.
__device__ __forceinline__ f32x4 mfma_q4_k8(uint4 a, int sa, uint4 b0, uint4 b1, int sb) {
  const i32x8 av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  const i32x8 bv = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, f32x4{0.f, 0.f, 0.f, 0.f}, 4, 0, 0, sa, 0, sb);
}

// 16 code bytes as a vector value: loads through it stay in registers (a struct copy of uint4
// from memory can leave the batch in private memory)
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
__device__ __forceinline__ u32x4 ld_u32x4(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ uint4 as_uint4(u32x4 v) { return make_uint4(v[0], v[1], v[2], v[3]); }

template <int U, bool KF8> struct MxBatch {
  u32x4 k[U];
  u32x4 k2[KF8 ? U : 1];                   // fp8 keys: the lane's second 16 code bytes
  uint32_t sc[U];
  uint32_t cf[U];
};

constexpr int kMxThreads = 512;  // 8 waves

// KF8: the keys are fp8 e4m3 rows (128 code bytes) whose ue8m0 scale word (one byte per 32
// channels) covers 2^ks_shift rows (1 or 32); the query stays MXFP4.
template <int HT, int TJ, bool KF8>
__global__ __launch_bounds__(kMxThreads) void indexer_score_mx_kernel(
    const uint8_t* __restrict__ qcodes, const uint8_t* __restrict__ qscales, const bf16_t* __restrict__ w_raw,
    float w_scale,
    const uint8_t* __restrict__ kcodes, int64_t kc_bstride, const uint8_t* __restrict__ kscales, int64_t ks_bstride,
    int ks_shift, const uint8_t* __restrict__ cand, float* __restrict__ scores, int n, int nb, int start_pos,
    int ratio, int rows_per_wg, int topk, uint32_t* __restrict__ ckey, int32_t* __restrict__ cpos) {
  constexpr int H = HT * 16;
  constexpr int DIM = 128;
  constexpr int KROW = KF8 ? DIM : DIM / 2;         // code bytes per key row
  // TJ > 0 (the fused top-k form): the range's scores collect in LDS and the workgroup keeps the
  // best min(topk, rows) as (order key, position) in position order, as indexer_decode_kernel does
  __shared__ float sc_lds[TJ > 0 ? TJ * kMxThreads : 1];
  __shared__ __align__(16) uint8_t sel_raw[TJ > 0 ? sizeof(RegSelShared) : 16];

  const int qi = blockIdx.y;               // b * n + s
  const int b = qi / n, s = qi - (qi / n) * n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, l16 = lane & 15;
  const int lens = (start_pos + s + 1) / ratio;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(r0 + rows_per_wg, nb);
  const int vis_end = max(r0, min(r1, lens));
  float* out = TJ ? nullptr : scores + (int64_t)qi * nb;
  const int64_t cbase = ((int64_t)qi * gridDim.x + blockIdx.x) * topk;   // this range's list (TJ > 0)
  if constexpr (TJ == 0) {
    for (int t = vis_end + tid; t < r1; t += kMxThreads) out[t] = -INFINITY;
  }
  if (vis_end <= r0) {                     // uniform: nothing visible in this row range
    if constexpr (TJ > 0) {                // all -inf: the lowest positions are the best
      for (int t = tid; t < min(topk, r1 - r0); t += kMxThreads) {
        ckey[cbase + t] = order_key(-INFINITY);
        cpos[cbase + t] = r0 + t;
      }
    }
    return;
  }

  // lane (l16, g) of a tile loads row l16's code bytes of block g (fp4: channels [32g, 32g+32);
  // fp8: [16g, 16g+16) and [64+16g, 64+16g+16), the instruction's 8-bit layout) and the scale word
  const uint8_t* kcb = kcodes + (int64_t)b * kc_bstride + g * 16;
  const uint8_t* ksb = kscales + (int64_t)b * ks_bstride;
  const uint8_t* cb = cand ? cand + (int64_t)qi * nb : nullptr;
  constexpr int NW = kMxThreads / 64;
  constexpr int U = 4;
  constexpr int STRIDE = 16 * U * NW;
  using Batch = MxBatch<U, KF8>;
  auto load = [&](Batch& kk, int t0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = min(t0 + 16 * u + l16, vis_end - 1);   // clamp: loads stay inside the cache
      kk.k[u] = ld_u32x4(kcb + (int64_t)row * KROW);
      if constexpr (KF8) kk.k2[u] = ld_u32x4(kcb + (int64_t)row * KROW + 64);
      kk.sc[u] = *reinterpret_cast<const uint32_t*>(ksb + (int64_t)(row >> ks_shift) * (DIM / 32));
      kk.cf[u] = cb ? (uint32_t)cb[row] : 1u;
    }
  };
  uint4 qa[HT];
  int qsa[HT];
  float wv[HT][4];
  auto compute = [&](const Batch& kk, int t0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int sb = (int)((kk.sc[u] >> (8 * g)) & 0xFFu);
      float part = 0.0f;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        f32x4 acc;
        if constexpr (KF8) acc = mfma_q4_k8(qa[ht], qsa[ht], as_uint4(kk.k[u]), as_uint4(kk.k2[u]), sb);
        else acc = mfma_mxfp4(qa[ht], qsa[ht], as_uint4(kk.k[u]), sb);
#pragma unroll
        for (int i = 0; i < 4; ++i) part += relu_bits(acc[i]) * wv[ht][i];
      }
      part = sum_rows4(part);
      const int row = t0 + 16 * u + l16;
      if (g == 0 && row < vis_end) {
        const float v = kk.cf[u] ? part : -INFINITY;
        if constexpr (TJ > 0) sc_lds[row - r0] = v;
        else out[row] = v;
      }
    }
  };
  int t0 = r0 + 16 * U * wave;
  // two register batches, named (not an array, which the compiler may keep in scratch memory):
  // one is in flight while the other is computed; the first goes out before the query operands
  Batch ba, bb;
  load(ba, t0);
  // the query's A operands: lane (l16, g) of head tile ht holds head ht*16 + l16, block g
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    const int64_t hq = (int64_t)qi * H + ht * 16 + l16;
    qa[ht] = *reinterpret_cast<const uint4*>(qcodes + hq * (DIM / 2) + g * 16);
    qsa[ht] = (int)qscales[hq * (DIM / 32) + g];
  }
  {
    const bf16_t* wrow = w_raw + (int64_t)qi * H;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[ht][i] = round_bf16(bf2f(wrow[ht * 16 + 4 * g + i]) * w_scale);
  }
  while (t0 < vis_end) {                   // wave-uniform
    load(bb, t0 + STRIDE);
    compute(ba, t0);
    t0 += STRIDE;
    if (t0 >= vis_end) break;
    load(ba, t0 + STRIDE);
    compute(bb, t0);
    t0 += STRIDE;
  }
  if constexpr (TJ > 0) {
    __syncthreads();                       // every score of the range is in LDS
    RegSelShared& sh = *reinterpret_cast<RegSelShared*>(sel_raw);
    auto value = [&](int t) { return t < vis_end - r0 ? sc_lds[t] : -INFINITY; };
    const int count = r1 - r0;
    const int i0 = tid * TJ;
    const int nvalid = min(max(count - i0, 0), TJ);
    uint32_t key[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) key[j] = j < nvalid ? order_key(value(i0 + j)) : 0u;
    select_top<TJ, kMxThreads>(key, nvalid, min(topk, count), sh, [&](uint32_t rank, int j) {
      ckey[cbase + rank] = order_key(value(i0 + j));             // re-read: j is a run-time index
      cpos[cbase + rank] = r0 + i0 + j;
    });
  }
}

// Prefill (many queries per batch row, no candidate mask): a workgroup scores 8 consecutive
// queries of one batch row -- one per wave -- against a range of kPfRows keys. The keys stream
// through an LDS ring in 64-row chunks with global_load_lds, so each key row is read from HBM
// once per workgroup instead of once per query; a wave holds its query's [heads x 128] block
// as MFMA A operands in registers and reads every chunk's B operands from LDS. Rows are stored
// with their 16-byte column chunks XOR-swizzled by (row % 16), so the 16 rows one B-operand read
// touches fall in distinct banks. Per chunk a wave runs 4 tiles x 4 k-steps x HT head tiles of
// 16x16x32 MFMA and the same epilogue as the decode kernel; queries mask rows past their own
// causal length, rows past the group's longest one are written as -inf without compute.
constexpr int kPfThreads = 512;        // 8 waves = 8 queries
constexpr int kPfChunk = 64;           // key rows per ring slot (16 KB at 128 channels)
constexpr int kPfSlots = 3;            // ring slots: 2 chunks in flight (48 KB: two workgroups per CU)
constexpr int kPfRows = 2048;          // key rows per workgroup

// (__launch_bounds__'s second argument, 4 waves per SIMD, caps VGPRs at 128 so that two
// workgroups share a CU)
template <int HT>
__global__ __launch_bounds__(kPfThreads, 4) void indexer_prefill_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ w_raw, float w_scale, const bf16_t* __restrict__ kcache,
    int64_t k_bstride, float* __restrict__ scores, int n, int nb, int start_pos, int ratio) {
  constexpr int H = HT * 16, DIM = 128, KS = 4;
  constexpr int ROWB = DIM * 2;                          // 256 bytes per key row
  constexpr int CHUNKB = kPfChunk * ROWB;
  constexpr int NL = CHUNKB / 1024 / (kPfThreads / 64);  // copies per wave per chunk
  static_assert(NL * 1024 * (kPfThreads / 64) == CHUNKB, "a chunk splits evenly into 1 KB copies per wave");
  __shared__ __align__(16) uint8_t ring[kPfSlots * CHUNKB];

  const int groups = (n + 7) / 8;
  const int b = blockIdx.y / groups, sg = blockIdx.y - (blockIdx.y / groups) * groups;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s = sg * 8 + wave;
  const bool qok = s < n;
  const int s_last = min(sg * 8 + 7, n - 1);
  const int lens_max = (start_pos + s_last + 1) / ratio;
  const int lens = (start_pos + min(s, n - 1) + 1) / ratio;
  const int r0 = blockIdx.x * kPfRows, r1 = min(r0 + kPfRows, nb);
  const int vis_end = max(r0, min(r1, lens_max));
  float* out = scores + ((int64_t)b * n + min(s, n - 1)) * nb;
  // rows past the group's visibility: -inf for each of its queries
  {
    const int span = r1 - vis_end;
    for (int e = tid; e < 8 * span; e += kPfThreads) {
      const int qq = e / span, row = vis_end + (e - qq * span);
      if (sg * 8 + qq < n) scores[((int64_t)b * n + sg * 8 + qq) * nb + row] = -INFINITY;
    }
  }
  if (vis_end <= r0) return;               // uniform: nothing visible in this row range
  const int nchunks = (vis_end - r0 + kPfChunk - 1) / kPfChunk;
  const uint8_t* kb = reinterpret_cast<const uint8_t*>(kcache + (int64_t)b * k_bstride);
  const uint32_t ring_base = lds_offset(ring);
  // chunk c -> slot c % kPfSlots; copy i (1 KB = 4 rows) goes to wave i / NL. Lane l of a copy
  // lands at row 4i + l/16, position l%16, and so loads column chunk (l%16) ^ (row % 16).
  auto issue = [&](int c) {
    const int slot = c % kPfSlots;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int ins = wave * NL + j;
      const int rloc = ins * 4 + (lane >> 4);
      const int row = min(r0 + c * kPfChunk + rloc, vis_end - 1);    // clamp: stays in the cache
      const int col = (lane & 15) ^ (rloc & 15);
      const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(ring_base + (uint32_t)(slot * CHUNKB + ins * 1024));
      dma16_vaddr(reinterpret_cast<uint64_t>(kb + (int64_t)row * ROWB + col * 16), dst);
    }
  };
  issue(0);
  // the query's A operands and head weights (an idle wave takes the last query and stores nothing)
  const int64_t qi = (int64_t)b * n + min(s, n - 1);
  bf16x8 qa[HT][KS];
  float wv[HT][4];
  {
    const bf16_t* qrow = q + qi * H * DIM;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qa[ht][ks] = ld_bf16x8(qrow + (ht * 16 + l16) * DIM + ks * 32 + g * 8);
    const bf16_t* wrow = w_raw + qi * H;
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[ht][i] = round_bf16(bf2f(wrow[ht * 16 + 4 * g + i]) * w_scale);
  }
  // query, weights and chunk 0 complete (a wait the compiler sees: no drain inside the loop)
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  for (int c = 1; c < nchunks && c < kPfSlots - 1; ++c) issue(c);

  for (int c = 0; c < nchunks; ++c) {
    const int after = min(nchunks - 1 - c, kPfSlots - 2);   // younger chunks allowed in flight
    static_assert(kPfSlots <= 4, "waits below cover at most 2 younger chunks");
    if (after >= 2) wait_vmcnt<2 * NL>();
    else if (after == 1) wait_vmcnt<NL>();
    else wait_vmcnt<0>();
    __syncthreads();                       // chunk c landed for every wave; chunk c-1 consumed
    if (c + kPfSlots - 1 < nchunks) issue(c + kPfSlots - 1);
    const uint8_t* buf = ring + (c % kPfSlots) * CHUNKB;
#pragma unroll
    for (int kt = 0; kt < kPfChunk / 16; ++kt) {
      f32x4 acc[HT];
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) acc[ht] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint8_t* rowp = buf + (kt * 16 + l16) * ROWB;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kop = ld_bf16x8(rowp + (((ks * 4 + g) ^ l16) * 16));
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) acc[ht] = mfma16x16x32(qa[ht][ks], kop, acc[ht]);
      }
      float part = 0.0f;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int i = 0; i < 4; ++i) part += relu_bits(acc[ht][i]) * wv[ht][i];
      part = sum_rows4(part);
      const int row = r0 + c * kPfChunk + kt * 16 + l16;
      if (qok && g == 0 && row < vis_end) out[row] = row < lens ? part : -INFINITY;
    }
  }
}

// fp32 path (parity configs): one thread per cache row, the query's q and w in LDS.
__global__ __launch_bounds__(256) void indexer_score_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ w_raw, float w_scale, const float* __restrict__ kcache,
    int64_t k_bstride, const uint8_t* __restrict__ cand, float* __restrict__ scores, int n, int heads, int dim,
    int nb, int start_pos, int ratio) {
  extern __shared__ float sm[];
  float* qs = sm;                          // [heads, dim]
  float* ws = sm + heads * dim;            // [heads]
  const int qi = blockIdx.y;
  const int b = qi / n, s = qi - (qi / n) * n;
  const float* qrow = q + (int64_t)qi * heads * dim;
  for (int i = threadIdx.x; i < heads * dim; i += 256) qs[i] = qrow[i];
  for (int i = threadIdx.x; i < heads; i += 256) ws[i] = w_raw[(int64_t)qi * heads + i] * w_scale;
  __syncthreads();
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= nb) return;
  const int lens = (start_pos + s + 1) / ratio;
  float v = -INFINITY;
  if (t < lens) {
    const float* kr = kcache + (int64_t)b * k_bstride + (int64_t)t * dim;
    v = 0.0f;
    for (int h = 0; h < heads; ++h) {
      float dot = 0.0f;
      for (int d = 0; d < dim; ++d) dot += qs[h * dim + d] * kr[d];
      v += fmaxf(dot, 0.0f) * ws[h];
    }
    if (cand && !cand[(int64_t)qi * nb + t]) v = -INFINITY;
  }
  scores[(int64_t)qi * nb + t] = v;
}

// Head tiles of the register-kernel instance for `heads` (1, 2, 4 or 8 tiles of 16; 0 if none
// serves: more than 128 heads).
static int head_tiles_instance(int heads) {
  const int t = (heads + 15) / 16;
  return t <= 1 ? 1 : t <= 2 ? 2 : t <= 4 ? 4 : t <= 8 ? 8 : 0;
}

template <int HT, int KS, bool F8>
static void launch_idx_bf16(dim3 grid, hipStream_t stream, const void* q, const void* w_raw, float w_scale,
                            const void* index_k, int64_t k_bstride, const uint8_t* kscale, int64_t ks_bstride,
                            int ks_rb, const uint8_t* cand, float* scores, int n, int nb, int start_pos, int ratio,
                            int rows_per_wg, int heads) {
  hipLaunchKernelGGL((indexer_score_bf16_kernel<HT, KS, F8>), grid, dim3(kIdxThreads), 0, stream,
                     (const bf16_t*)q, (const bf16_t*)w_raw, w_scale, index_k, k_bstride, kscale, ks_bstride, ks_rb,
                     cand, scores, n, nb, start_pos, ratio, rows_per_wg, heads);
}

// ~256 workgroups over all rows (one per CU), in multiples of one 8-wave sweep of four tiles
// (512 rows): long-lived workgroups amortize staging the query block
static dim3 idx_grid(int64_t rows_total, int nb, int bn, int* rows_per_wg) {
  const int64_t want = (rows_total + 255) / 256;
  int r = (int)((want + 511) / 512 * 512);
  if (r < 512) r = 512;
  if (r > 4096) r = 4096;
  *rows_per_wg = r;
  return dim3((unsigned)((nb + r - 1) / r), (unsigned)bn);
}

}  // namespace dsv41

using namespace dsv41;

extern "C" int dsv41_indexer_score(const void* q, const void* w_raw, float w_scale, const void* index_k,
                                   int64_t k_bstride, const uint8_t* candidates, float* scores, int32_t bsz,
                                   int32_t n, int32_t heads, int32_t dim, int32_t nb, int32_t start_pos,
                                   int32_t ratio, int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_indexer_score";
  DSV41_REQUIRE(q && w_raw && index_k && scores, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && dim > 0 && nb >= 0 && start_pos >= 0 && ratio > 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(k_bstride >= (int64_t)nb * dim, DSV41_E_ARG, "%s: k_bstride %lld < nb*dim", what,
                (long long)k_bstride);
  DSV41_REQUIRE((int64_t)bsz * n < 65536, DSV41_E_ARG, "%s: bsz*n must be < 65536", what);
  if ((int64_t)bsz * n == 0 || nb == 0) return 0;
  if (dtype == DSV41_F32) {
    const size_t smem = ((size_t)heads * dim + heads) * sizeof(float);
    DSV41_REQUIRE(smem <= 64 * 1024, DSV41_E_SHAPE, "%s: fp32 path needs heads*dim <= 16k", what);
    dim3 grid((unsigned)((nb + 255) / 256), (unsigned)(bsz * n));
    hipLaunchKernelGGL(indexer_score_f32_kernel, grid, dim3(256), smem, stream, (const float*)q,
                       (const float*)w_raw, w_scale, (const float*)index_k, k_bstride, candidates, scores, n,
                       heads, dim, nb, start_pos, ratio);
    return check_launch(what);
  }
  if (dtype != DSV41_BF16) return set_error(DSV41_E_DTYPE, "%s: dtype %d not supported", what, dtype);
  DSV41_REQUIRE(aligned16(q) && aligned16(index_k), DSV41_E_ARG, "%s: q and index_k must be 16-byte aligned", what);
  DSV41_REQUIRE(k_bstride % 8 == 0, DSV41_E_ARG, "%s: k_bstride must be a multiple of 8", what);
  if (n >= 8 && !candidates && dim == 128 && (heads == 64 || heads == 32 || heads == 16) &&
      (int64_t)bsz * ((n + 7) / 8) < 65536) {
    const dim3 pgrid((unsigned)((nb + kPfRows - 1) / kPfRows), (unsigned)(bsz * ((n + 7) / 8)));
#define DSV41_PF_CASE(HT_)                                                                                  \
    if (heads == HT_ * 16) {                                                                                 \
      hipLaunchKernelGGL((indexer_prefill_kernel<HT_>), pgrid, dim3(kPfThreads), 0, stream, (const bf16_t*)q, \
                         (const bf16_t*)w_raw, w_scale, (const bf16_t*)index_k, k_bstride, scores, n, nb,      \
                         start_pos, ratio);                                                                  \
      return check_launch(what);                                                                             \
    }
    DSV41_PF_CASE(4)
    DSV41_PF_CASE(2)
    DSV41_PF_CASE(1)
#undef DSV41_PF_CASE
  }
  int rows_per_wg = 0;
  const dim3 grid = idx_grid((int64_t)nb * bsz * n, nb, bsz * n, &rows_per_wg);
  if (dim == 128 && (heads == 64 || heads == 32 || heads == 16) && aligned16(w_raw) && rows_per_wg <= kIdxMaxRows) {
#define DSV41_DEC_CASE(HT_)                                                                                   \
    if (heads == HT_ * 16) {                                                                                  \
      hipLaunchKernelGGL((indexer_decode_kernel<HT_, kDecWaves, false, 0>), grid, dim3(kDecWaves * 64), 0,    \
                         stream, (const bf16_t*)q, (const bf16_t*)w_raw, w_scale, index_k, k_bstride, nullptr, \
                         0, 1, candidates, scores, n, nb, start_pos, ratio, rows_per_wg, 0, nullptr, nullptr); \
      return check_launch(what);                                                                              \
    }
    DSV41_DEC_CASE(4)
    DSV41_DEC_CASE(2)
    DSV41_DEC_CASE(1)
#undef DSV41_DEC_CASE
  }
  // the register kernel serves every head count up to 128 in whole 16-head tiles (the last one
  // padded with zero queries and weights), as the reference's kernel wrapper pads heads to 16
  const int ht_inst = head_tiles_instance(heads);
#define DSV41_IDX_CASE(HT_, KS_)                                                                          \
  if (ht_inst == HT_ && dim == KS_ * 32) {                                                                   \
    launch_idx_bf16<HT_, KS_, false>(grid, stream, q, w_raw, w_scale, index_k, k_bstride, nullptr, 0, 1,     \
                                     candidates, scores, n, nb, start_pos, ratio, rows_per_wg, heads);       \
    return check_launch(what);                                                                               \
  }
  DSV41_IDX_CASE(4, 4)   // 64 heads x 128
  DSV41_IDX_CASE(2, 4)   // 32 heads x 128 (the released model)
  DSV41_IDX_CASE(1, 4)
  DSV41_IDX_CASE(8, 4)
  DSV41_IDX_CASE(4, 2)
  DSV41_IDX_CASE(2, 2)
  DSV41_IDX_CASE(1, 2)
  DSV41_IDX_CASE(1, 1)
  DSV41_IDX_CASE(2, 1)
  DSV41_IDX_CASE(4, 1)
  DSV41_IDX_CASE(8, 2)
  DSV41_IDX_CASE(8, 1)
#undef DSV41_IDX_CASE
  return set_error(DSV41_E_SHAPE, "%s: bf16 path has no instance for heads=%d dim=%d", what, heads, dim);
}

// The fused decode form (indexer_decode_kernel with TJ > 0, then the top-k merge): shapes the
// staged-copy decode kernel serves (bf16 keys of 128 channels, 16/32/64 heads, fewer than 8
// queries per row or a candidate mask) with row ranges of 512, 1024, 2048 or 4096 rows, at least
// four times k.
static bool idx_topk_plan(int64_t bsz, int n, int heads, int dim, int nb, int k, bool cand, int* rows_per_wg,
                          dim3* grid, int* tj) {
  if (dim != 128 || !(heads == 64 || heads == 32 || heads == 16)) return false;
  if ((n >= 8 && !cand) || bsz * n >= 65536) return false;
  *grid = idx_grid((int64_t)nb * bsz * n, nb, (int)(bsz * n), rows_per_wg);
  *tj = *rows_per_wg / 512;                        // 512, 1024, 2048 or 4096 rows: 1, 2, 4 or 8 per thread
  if (*tj != 1 && *tj != 2 && *tj != 4 && *tj != 8) return false;
  // a range keeps at most a quarter of its rows: at k = rows / 2 (B = 16, 32,768 entries, top-1,024)
  // the per-range selection and a 16,384-entry merge cost what the unfused scores write saves
  return 4 * k <= *rows_per_wg && (int64_t)grid->x * k <= 32 * kSelThreads;
}

static size_t idx_topk_ws(int64_t rows, unsigned chunks, int k) {
  const size_t list = ((size_t)rows * chunks * k * sizeof(uint32_t) + 255) & ~(size_t)255;
  return 2 * list;                                 // order keys, then positions
}

extern "C" int dsv41_indexer_score_fp8(const void* q, const void* w_raw, float w_scale, const uint8_t* index_k,
                                       int64_t k_bstride, const uint8_t* k_scale, int64_t ks_bstride, int32_t ks_rb,
                                       const uint8_t* candidates, float* scores, int32_t bsz, int32_t n,
                                       int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                                       hipStream_t stream) {
  const char* what = "dsv41_indexer_score_fp8";
  DSV41_REQUIRE(q && w_raw && index_k && k_scale && scores, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && nb >= 0 && start_pos >= 0 && ratio > 0, DSV41_E_ARG,
                "%s: bad sizes", what);
  DSV41_REQUIRE(dim == 128, DSV41_E_SHAPE, "%s: fp8 index keys support dim 128, got %d", what, dim);
  DSV41_REQUIRE(ks_rb == 1 || ks_rb == 32, DSV41_E_ARG, "%s: scale row block must be 1 or 32", what);
  DSV41_REQUIRE(k_bstride >= (int64_t)nb * dim, DSV41_E_ARG, "%s: k_bstride too small", what);
  DSV41_REQUIRE(ks_bstride >= (int64_t)((nb + ks_rb - 1) / ks_rb) * (dim / 32), DSV41_E_ARG,
                "%s: ks_bstride too small", what);
  DSV41_REQUIRE((int64_t)bsz * n < 65536, DSV41_E_ARG, "%s: bsz*n must be < 65536", what);
  DSV41_REQUIRE(aligned16(q) && aligned16(index_k) && (reinterpret_cast<uintptr_t>(k_scale) & 3u) == 0,
                DSV41_E_ARG, "%s: q and index_k must be 16-byte aligned, k_scale 4-byte aligned", what);
  DSV41_REQUIRE(k_bstride % 16 == 0 && ks_bstride % 4 == 0, DSV41_E_ARG,
                "%s: k_bstride must be a multiple of 16 bytes, ks_bstride of 4", what);
  if ((int64_t)bsz * n == 0 || nb == 0) return 0;
  int rows_per_wg = 0;
  const dim3 grid = idx_grid((int64_t)nb * bsz * n, nb, bsz * n, &rows_per_wg);
  if ((heads == 64 || heads == 32 || heads == 16) && aligned16(w_raw) && aligned16(k_scale) &&
      ks_bstride % 16 == 0 && rows_per_wg <= kIdxMaxRows) {
#define DSV41_DEC8_CASE(HT_)                                                                                  \
    if (heads == HT_ * 16) {                                                                                  \
      hipLaunchKernelGGL((indexer_decode_kernel<HT_, kDecWaves, true, 0>), grid, dim3(kDecWaves * 64), 0,     \
                         stream, (const bf16_t*)q, (const bf16_t*)w_raw, w_scale, index_k, k_bstride, k_scale, \
                         ks_bstride, ks_rb, candidates, scores, n, nb, start_pos, ratio, rows_per_wg, 0,       \
                         nullptr, nullptr);                                                                   \
      return check_launch(what);                                                                              \
    }
    DSV41_DEC8_CASE(4)
    DSV41_DEC8_CASE(2)
    DSV41_DEC8_CASE(1)
#undef DSV41_DEC8_CASE
  }
  const int ht_inst = head_tiles_instance(heads);
#define DSV41_IDX8_CASE(HT_)                                                                                   \
  if (ht_inst == HT_) {                                                                                        \
    launch_idx_bf16<HT_, 4, true>(grid, stream, q, w_raw, w_scale, index_k, k_bstride, k_scale, ks_bstride,  \
                                  ks_rb, candidates, scores, n, nb, start_pos, ratio, rows_per_wg, heads);     \
    return check_launch(what);                                                                                 \
  }
  DSV41_IDX8_CASE(4)   // 64 heads
  DSV41_IDX8_CASE(2)   // 32 heads
  DSV41_IDX8_CASE(1)
#undef DSV41_IDX8_CASE
  return set_error(DSV41_E_SHAPE, "%s: no instance for heads=%d", what, heads);
}

// Scoring with an MXFP4 query against MXFP4 keys (kf8 false) or fp8 e4m3 keys whose scale word
// covers ks_rb rows (kf8 true). Strides in bytes.
static int mx_score_entry(const char* what, bool kf8, const uint8_t* q_codes, const uint8_t* q_scales,
                          const void* w_raw, float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                          const uint8_t* k_scales, int64_t ks_bstride, int ks_rb, const uint8_t* candidates,
                          float* scores, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                          int32_t start_pos, int32_t ratio, hipStream_t stream) {
  DSV41_REQUIRE(q_codes && q_scales && w_raw && k_codes && k_scales && scores, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && nb >= 0 && start_pos >= 0 && ratio > 0, DSV41_E_ARG,
                "%s: bad sizes", what);
  DSV41_REQUIRE(dim == 128, DSV41_E_SHAPE, "%s: MXFP4 queries and packed index keys support dim 128, got %d", what,
                dim);
  DSV41_REQUIRE(ks_rb == 1 || (kf8 && ks_rb == 32), DSV41_E_ARG, "%s: scale row block must be 1%s", what,
                kf8 ? " or 32" : "");
  const int64_t krow = kf8 ? dim : dim / 2;
  DSV41_REQUIRE(kc_bstride >= (int64_t)nb * krow && ks_bstride >= (int64_t)((nb + ks_rb - 1) / ks_rb) * (dim / 32),
                DSV41_E_ARG, "%s: batch strides too small", what);
  DSV41_REQUIRE((int64_t)bsz * n < 65536, DSV41_E_ARG, "%s: bsz*n must be < 65536", what);
  DSV41_REQUIRE(aligned16(q_codes) && aligned16(k_codes) && (reinterpret_cast<uintptr_t>(k_scales) & 3u) == 0,
                DSV41_E_ARG, "%s: q_codes and k_codes must be 16-byte aligned, k_scales 4-byte aligned", what);
  DSV41_REQUIRE(kc_bstride % 16 == 0 && ks_bstride % 4 == 0, DSV41_E_ARG,
                "%s: kc_bstride must be a multiple of 16 bytes, ks_bstride of 4", what);
  if ((int64_t)bsz * n == 0 || nb == 0) return 0;
  int rows_per_wg = 0;
  const dim3 grid = idx_grid((int64_t)nb * bsz * n, nb, bsz * n, &rows_per_wg);
  const int shift = ks_rb == 32 ? 5 : 0;
#define DSV41_IDXMX_CASE(HT_, KF8_)                                                                           \
  if (heads == HT_ * 16 && kf8 == KF8_) {                                                                     \
    hipLaunchKernelGGL((indexer_score_mx_kernel<HT_, 0, KF8_>), grid, dim3(kMxThreads), 0, stream, q_codes,   \
                       q_scales, (const bf16_t*)w_raw, w_scale, k_codes, kc_bstride, k_scales, ks_bstride,     \
                       shift, candidates, scores, n, nb, start_pos, ratio, rows_per_wg, 0, nullptr, nullptr);  \
    return check_launch(what);                                                                                \
  }
  DSV41_IDXMX_CASE(4, false) DSV41_IDXMX_CASE(2, false) DSV41_IDXMX_CASE(1, false)
  DSV41_IDXMX_CASE(4, true) DSV41_IDXMX_CASE(2, true) DSV41_IDXMX_CASE(1, true)
#undef DSV41_IDXMX_CASE
  return set_error(DSV41_E_SHAPE, "%s: no instance for heads=%d", what, heads);
}

extern "C" int dsv41_indexer_score_mxfp4(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                                         float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                                         const uint8_t* k_scales, int64_t ks_bstride, const uint8_t* candidates,
                                         float* scores, int32_t bsz, int32_t n, int32_t heads, int32_t dim,
                                         int32_t nb, int32_t start_pos, int32_t ratio, hipStream_t stream) {
  return mx_score_entry("dsv41_indexer_score_mxfp4", false, q_codes, q_scales, w_raw, w_scale, k_codes, kc_bstride,
                        k_scales, ks_bstride, 1, candidates, scores, bsz, n, heads, dim, nb, start_pos, ratio,
                        stream);
}

extern "C" int dsv41_indexer_score_mxq_fp8(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                                           float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                                           const uint8_t* k_scales, int64_t ks_bstride, int32_t ks_rb,
                                           const uint8_t* candidates, float* scores, int32_t bsz, int32_t n,
                                           int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                                           hipStream_t stream) {
  return mx_score_entry("dsv41_indexer_score_mxq_fp8", true, q_codes, q_scales, w_raw, w_scale, k_codes, kc_bstride,
                        k_scales, ks_bstride, ks_rb, candidates, scores, bsz, n, heads, dim, nb, start_pos, ratio,
                        stream);
}

extern "C" size_t dsv41_indexer_topk_workspace_bytes(int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                                                     int32_t topk, int32_t has_candidates) {
  if (bsz <= 0 || n <= 0 || nb <= 0 || topk <= 0 || heads <= 0 || dim <= 0) return 0;
  const int k = topk < nb ? topk : nb;
  int rpw = 0, tj = 0;
  dim3 grid;
  if (!idx_topk_plan(bsz, n, heads, dim, nb, k, has_candidates != 0, &rpw, &grid, &tj)) return 0;
  return idx_topk_ws((int64_t)bsz * n, grid.x, k);
}

extern "C" int dsv41_indexer_topk(const void* q, const void* w_raw, float w_scale, const void* index_k,
                                  int64_t k_bstride, const uint8_t* candidates, int32_t* out, int32_t bsz, int32_t n,
                                  int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                                  int32_t topk, int32_t offset, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  const char* what = "dsv41_indexer_topk";
  DSV41_REQUIRE(q && w_raw && index_k && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n > 0 && heads > 0 && dim > 0 && nb >= 0 && start_pos >= 0 && ratio > 0 && topk >= 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(k_bstride >= (int64_t)nb * dim, DSV41_E_ARG, "%s: k_bstride %lld < nb*dim", what,
                (long long)k_bstride);
  DSV41_REQUIRE(aligned16(q) && aligned16(index_k) && aligned16(w_raw) && k_bstride % 8 == 0, DSV41_E_ARG,
                "%s: q, w_raw and index_k must be 16-byte aligned, k_bstride a multiple of 8", what);
  const int k = topk < nb ? topk : nb;
  if ((int64_t)bsz * n == 0 || nb == 0 || k == 0) return 0;
  int rows_per_wg = 0, tj = 0;
  dim3 grid;
  DSV41_REQUIRE(idx_topk_plan(bsz, n, heads, dim, nb, k, candidates != nullptr, &rows_per_wg, &grid, &tj),
                DSV41_E_SHAPE, "%s: shape not served by the fused form (dsv41_indexer_topk_workspace_bytes is 0)",
                what);
  const size_t need = idx_topk_ws((int64_t)bsz * n, grid.x, k);
  DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed", what,
                need);
  DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
  uint32_t* ckey = reinterpret_cast<uint32_t*>(workspace);
  int32_t* cpos = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(workspace) + need / 2);
#define DSV41_FUSED_CASE(HT_, TJ_)                                                                             \
  if (heads == HT_ * 16 && tj == TJ_) {                                                                        \
    hipLaunchKernelGGL((indexer_decode_kernel<HT_, kDecWaves, false, TJ_>), grid, dim3(kDecWaves * 64), 0,     \
                       stream, (const bf16_t*)q, (const bf16_t*)w_raw, w_scale, index_k, k_bstride, nullptr, 0, 1, \
                       candidates, nullptr, n, nb, start_pos, ratio, rows_per_wg, k, ckey, cpos);             \
  } else
  DSV41_FUSED_CASE(4, 1) DSV41_FUSED_CASE(4, 2) DSV41_FUSED_CASE(4, 4) DSV41_FUSED_CASE(4, 8)
  DSV41_FUSED_CASE(2, 1) DSV41_FUSED_CASE(2, 2) DSV41_FUSED_CASE(2, 4) DSV41_FUSED_CASE(2, 8)
  DSV41_FUSED_CASE(1, 1) DSV41_FUSED_CASE(1, 2) DSV41_FUSED_CASE(1, 4) DSV41_FUSED_CASE(1, 8)
  return set_error(DSV41_E_SHAPE, "%s: no instance for heads=%d", what, heads);
#undef DSV41_FUSED_CASE
  const int rc = check_launch(what);
  if (rc) return rc;
  return topk_merge_launch(what, ckey, cpos, out, (int64_t)bsz * n, n, nb, k, (int)grid.x, rows_per_wg, start_pos,
                           ratio, offset, stream);
}

extern "C" int dsv41_indexer_topk_fp8(const void* q, const void* w_raw, float w_scale, const uint8_t* index_k,
                                      int64_t k_bstride, const uint8_t* k_scale, int64_t ks_bstride, int32_t ks_rb,
                                      const uint8_t* candidates, int32_t* out, int32_t bsz, int32_t n, int32_t heads,
                                      int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio, int32_t topk,
                                      int32_t offset, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* what = "dsv41_indexer_topk_fp8";
  DSV41_REQUIRE(q && w_raw && index_k && k_scale && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n > 0 && heads > 0 && dim > 0 && nb >= 0 && start_pos >= 0 && ratio > 0 && topk >= 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(ks_rb == 1 || ks_rb == 32, DSV41_E_ARG, "%s: scale row block must be 1 or 32", what);
  DSV41_REQUIRE(k_bstride >= (int64_t)nb * dim, DSV41_E_ARG, "%s: k_bstride too small", what);
  DSV41_REQUIRE(ks_bstride >= (int64_t)((nb + ks_rb - 1) / ks_rb) * (dim / 32), DSV41_E_ARG,
                "%s: ks_bstride too small", what);
  DSV41_REQUIRE(aligned16(q) && aligned16(w_raw) && aligned16(index_k) && aligned16(k_scale) &&
                    k_bstride % 16 == 0 && ks_bstride % 16 == 0,
                DSV41_E_ARG, "%s: q, w_raw, index_k and k_scale must be 16-byte aligned, both strides multiples of 16",
                what);
  const int k = topk < nb ? topk : nb;
  if ((int64_t)bsz * n == 0 || nb == 0 || k == 0) return 0;
  int rows_per_wg = 0, tj = 0;
  dim3 grid;
  DSV41_REQUIRE(idx_topk_plan(bsz, n, heads, dim, nb, k, candidates != nullptr, &rows_per_wg, &grid, &tj),
                DSV41_E_SHAPE, "%s: shape not served by the fused form (dsv41_indexer_topk_workspace_bytes is 0)",
                what);
  const size_t need = idx_topk_ws((int64_t)bsz * n, grid.x, k);
  DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed", what,
                need);
  DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
  uint32_t* ckey = reinterpret_cast<uint32_t*>(workspace);
  int32_t* cpos = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(workspace) + need / 2);
#define DSV41_FUSED8_CASE(HT_, TJ_)                                                                            \
  if (heads == HT_ * 16 && tj == TJ_) {                                                                        \
    hipLaunchKernelGGL((indexer_decode_kernel<HT_, kDecWaves, true, TJ_>), grid, dim3(kDecWaves * 64), 0,      \
                       stream, (const bf16_t*)q, (const bf16_t*)w_raw, w_scale, index_k, k_bstride, k_scale,   \
                       ks_bstride, ks_rb, candidates, nullptr, n, nb, start_pos, ratio, rows_per_wg, k, ckey, cpos); \
  } else
  DSV41_FUSED8_CASE(4, 1) DSV41_FUSED8_CASE(4, 2) DSV41_FUSED8_CASE(4, 4) DSV41_FUSED8_CASE(4, 8)
  DSV41_FUSED8_CASE(2, 1) DSV41_FUSED8_CASE(2, 2) DSV41_FUSED8_CASE(2, 4) DSV41_FUSED8_CASE(2, 8)
  DSV41_FUSED8_CASE(1, 1) DSV41_FUSED8_CASE(1, 2) DSV41_FUSED8_CASE(1, 4) DSV41_FUSED8_CASE(1, 8)
  return set_error(DSV41_E_SHAPE, "%s: no instance for heads=%d", what, heads);
#undef DSV41_FUSED8_CASE
  const int rc = check_launch(what);
  if (rc) return rc;
  return topk_merge_launch(what, ckey, cpos, out, (int64_t)bsz * n, n, nb, k, (int)grid.x, rows_per_wg, start_pos,
                           ratio, offset, stream);
}

static int mx_topk_entry(const char* what, bool kf8, const uint8_t* q_codes, const uint8_t* q_scales,
                         const void* w_raw, float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                         const uint8_t* k_scales, int64_t ks_bstride, int ks_rb, const uint8_t* candidates,
                         int32_t* out, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                         int32_t start_pos, int32_t ratio, int32_t topk, int32_t offset, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  DSV41_REQUIRE(q_codes && q_scales && w_raw && k_codes && k_scales && out, DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n > 0 && heads > 0 && nb >= 0 && start_pos >= 0 && ratio > 0 && topk >= 0, DSV41_E_ARG,
                "%s: bad sizes", what);
  DSV41_REQUIRE(dim == 128, DSV41_E_SHAPE, "%s: MXFP4 queries and packed index keys support dim 128, got %d", what,
                dim);
  DSV41_REQUIRE(ks_rb == 1 || (kf8 && ks_rb == 32), DSV41_E_ARG, "%s: scale row block must be 1%s", what,
                kf8 ? " or 32" : "");
  const int64_t krow = kf8 ? dim : dim / 2;
  DSV41_REQUIRE(kc_bstride >= (int64_t)nb * krow && ks_bstride >= (int64_t)((nb + ks_rb - 1) / ks_rb) * (dim / 32),
                DSV41_E_ARG, "%s: batch strides too small", what);
  DSV41_REQUIRE(aligned16(q_codes) && aligned16(k_codes) && (reinterpret_cast<uintptr_t>(k_scales) & 3u) == 0,
                DSV41_E_ARG, "%s: q_codes and k_codes must be 16-byte aligned, k_scales 4-byte aligned", what);
  DSV41_REQUIRE(kc_bstride % 16 == 0 && ks_bstride % 4 == 0, DSV41_E_ARG,
                "%s: kc_bstride must be a multiple of 16 bytes, ks_bstride of 4", what);
  const int k = topk < nb ? topk : nb;
  if ((int64_t)bsz * n == 0 || nb == 0 || k == 0) return 0;
  int rows_per_wg = 0, tj = 0;
  dim3 grid;
  DSV41_REQUIRE(idx_topk_plan(bsz, n, heads, dim, nb, k, candidates != nullptr, &rows_per_wg, &grid, &tj),
                DSV41_E_SHAPE, "%s: shape not served by the fused form (dsv41_indexer_topk_workspace_bytes is 0)",
                what);
  const size_t need = idx_topk_ws((int64_t)bsz * n, grid.x, k);
  DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed", what,
                need);
  DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
  uint32_t* ckey = reinterpret_cast<uint32_t*>(workspace);
  int32_t* cpos = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(workspace) + need / 2);
  const int shift = ks_rb == 32 ? 5 : 0;
#define DSV41_FUSEDMX_CASE(HT_, TJ_, KF8_)                                                                     \
  if (heads == HT_ * 16 && tj == TJ_ && kf8 == KF8_) {                                                         \
    hipLaunchKernelGGL((indexer_score_mx_kernel<HT_, TJ_, KF8_>), grid, dim3(kMxThreads), 0, stream, q_codes,  \
                       q_scales, (const bf16_t*)w_raw, w_scale, k_codes, kc_bstride, k_scales, ks_bstride,      \
                       shift, candidates, nullptr, n, nb, start_pos, ratio, rows_per_wg, k, ckey, cpos);      \
  } else
#define DSV41_FUSEDMX_HT(HT_, KF8_)                                                                            \
  DSV41_FUSEDMX_CASE(HT_, 1, KF8_) DSV41_FUSEDMX_CASE(HT_, 2, KF8_) DSV41_FUSEDMX_CASE(HT_, 4, KF8_)           \
  DSV41_FUSEDMX_CASE(HT_, 8, KF8_)
  DSV41_FUSEDMX_HT(4, false) DSV41_FUSEDMX_HT(2, false) DSV41_FUSEDMX_HT(1, false)
  DSV41_FUSEDMX_HT(4, true) DSV41_FUSEDMX_HT(2, true) DSV41_FUSEDMX_HT(1, true)
  return set_error(DSV41_E_SHAPE, "%s: no instance for heads=%d", what, heads);
#undef DSV41_FUSEDMX_HT
#undef DSV41_FUSEDMX_CASE
  const int rc = check_launch(what);
  if (rc) return rc;
  return topk_merge_launch(what, ckey, cpos, out, (int64_t)bsz * n, n, nb, k, (int)grid.x, rows_per_wg, start_pos,
                           ratio, offset, stream);
}

extern "C" int dsv41_indexer_topk_mxfp4(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                                        float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                                        const uint8_t* k_scales, int64_t ks_bstride, const uint8_t* candidates,
                                        int32_t* out, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                                        int32_t start_pos, int32_t ratio, int32_t topk, int32_t offset,
                                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return mx_topk_entry("dsv41_indexer_topk_mxfp4", false, q_codes, q_scales, w_raw, w_scale, k_codes, kc_bstride,
                       k_scales, ks_bstride, 1, candidates, out, bsz, n, heads, dim, nb, start_pos, ratio, topk,
                       offset, workspace, workspace_bytes, stream);
}

extern "C" int dsv41_indexer_topk_mxq_fp8(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                                          float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                                          const uint8_t* k_scales, int64_t ks_bstride, int32_t ks_rb,
                                          const uint8_t* candidates, int32_t* out, int32_t bsz, int32_t n,
                                          int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                                          int32_t topk, int32_t offset, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
  return mx_topk_entry("dsv41_indexer_topk_mxq_fp8", true, q_codes, q_scales, w_raw, w_scale, k_codes, kc_bstride,
                       k_scales, ks_bstride, ks_rb, candidates, out, bsz, n, heads, dim, nb, start_pos, ratio, topk,
                       offset, workspace, workspace_bytes, stream);
}
