// Sparse MLA, deepseek_v41_mlx/sparse_attention.py:34-60 (TileLang sparse_attn_kernel,
// docs/reference/kernel.py:310-403) and the attention core of attention.py:124-175.
//
// K = V: one shared [dim] row per selected position serves all heads of a query, so a query is
// a small GEMM of its [heads x dim] q block against the gathered [rows x dim] block.
//
// bf16 kernels (MFMA, fp32 accumulate). A wave owns 16 heads of one query:
//   S^T[rows x heads] = K[rows x d] Q^T[d x heads]   (16x16x32, K rows from LDS, Q^T in registers)
//   online softmax in log2 units with lazy rescaling; the sink seeds the running max and the
//     denominator once per head (sink in the denominator only, no value row); masked rows give 0;
//   O^T[d x heads] += V^T P^T   (P^T straight from the S^T accumulators -- same lane layout --
//     V^T through the LDS transpose read ds_read_b64_tr_b16).
// Selected rows are gathered with global_load_lds_dwordx4 (one 1 KB row per wave instruction at
// d = 512) into LDS ring buffers, so several tiles are in flight without staging registers.
// Decode (few queries) splits each query's index list across workgroups (two per CU in the
// half-LDS instance); a combine kernel merges the per-split partials (normalized bf16 numerator,
// fp32 max and denominator). The epilogue divides, rounds to bf16 as the reference does, then
// applies the inverse rope to the last rd channels (attention.py:174-175).
//
// fp32 kernel: a plain FMA implementation for the 1e-5 parity configs.
#include <mutex>

#include "mla.h"

namespace dsv41 {

// One-token decode: copy batch row b's KV row into ring slot start_pos % window. The slot holds
// position start_pos - window, which has just left the window, so no entry of the launch reads
// it; one wave per batch row does the copy, at its start.
template <typename T>
__device__ __forceinline__ void ring_store(const MlaArgs& a, int b, int lane, int lanes);

// The same store into an MXFP8 ring (rows of D e4m3fn codes, then D/32 ue8m0 scale bytes): one
// full wave, 8 channels per lane, a 32-channel block per 4 lanes, quantized by
// fake_quant_fp8_ue8m0's formula (fakequant.py:83-93). The window KV reaching the ring already
// holds that QAT's values, which this encodes exactly (the block scale it finds is the QAT's own
// or half of it, and either puts every value on the e4m3 grid).
template <int D>
__device__ __forceinline__ void ring_store_fp8(const MlaArgs& a, int b, int lane) {
  static_assert(D == 512, "MXFP8 ring rows: 512 channels");
  const KvSrc& S = a.src;
  const bf16_t* src = reinterpret_cast<const bf16_t*>(S.chunk) + (int64_t)b * S.chunk_bstride + lane * 8;
  uint8_t* row = reinterpret_cast<uint8_t*>(a.ring_w) + (int64_t)b * S.ring_bstride +
                 (int64_t)(a.start_pos % S.window) * (D + D / 32);
  float v[8];
  const uint4 x = *reinterpret_cast<const uint4*>(src);
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = bf2f((bf16_t)(xw[i / 2] >> (16 * (i % 2))));
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(group_max(amax, 4), 1e-4f);
  const float sc = pow2_ceil_log2(amax * (float)(1.0 / 448.0));
  const float inv = __fdiv_rn(1.0f, sc);        // exact: sc is a power of two
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i)
    w[i / 4] |= (uint32_t)e4m3_encode(e4m3_round(fminf(fmaxf(v[i] * inv, -448.0f), 448.0f))) << (8 * (i % 4));
  *reinterpret_cast<uint2*>(row + lane * 8) = make_uint2(w[0], w[1]);
  if ((lane & 3) == 0) row[D + (lane >> 2)] = (uint8_t)((__float_as_uint(sc) >> 23) & 0xFFu);
}

template <typename T>
__device__ __forceinline__ void ring_store(const MlaArgs& a, int b, int lane, int lanes) {
  const KvSrc& S = a.src;
  const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(S.chunk) + (int64_t)b * S.chunk_bstride);
  uint4* dst = reinterpret_cast<uint4*>(reinterpret_cast<T*>(a.ring_w) + (int64_t)b * S.ring_bstride +
                                        (int64_t)(a.start_pos % S.window) * a.dim);
  const int n16 = a.dim * (int)sizeof(T) / 16;
  for (int c = lane; c < n16; c += lanes) dst[c] = src[c];
}

// Masked list entries gather this zero row, so every step issues the same number of copies
// (their count is what s_waitcnt vmcnt waits on) and padded LDS rows hold finite zeros.
__device__ __align__(16) uint4 g_zero_row[128] = {};

// Copy one KV row (address `p`, wave-uniform; 0 = masked -> the zero row) of D bf16 into LDS at
// byte offset `dst`: one 1 KB wave instruction per 512 channels.
template <int D>
__device__ __forceinline__ void dma_row(uint64_t p, uint32_t dst, int lane) {
  constexpr int CPR = D / 8, IPR = (CPR + 63) / 64;
  const uint64_t src = p ? p : reinterpret_cast<uint64_t>(g_zero_row);
#pragma unroll
  for (int ii = 0; ii < IPR; ++ii) {
    const int ch = ii * 64 + lane;
    if (CPR % 64 == 0 || ch < CPR) dma16_sgpr(src, (uint32_t)ch * 16u, dst + ii * 1024);
  }
}

constexpr int kRopeRowPairs = 128;   // q rope pairs (rd / 2) staged in LDS by the decode kernel

template <int D, int NW, int ML, int BUDGET>
struct MlaLds {
  static constexpr int RS = D * 2 + 16;                   // padded row stride (bytes)
  static constexpr int SLOT = kStepRows * RS;
  static constexpr int XS = NW * 2 * 64 * 16;             // partial-score exchange
  static constexpr int FIXED = XS + ML * 8 + kMaxRing * kStepRows + 2 * kRopeRowPairs * 4 + 256;
  static constexpr int NS = (BUDGET - FIXED) / SLOT < kMaxRing ? (BUDGET - FIXED) / SLOT : kMaxRing;
  static_assert(NS >= 2, "ring needs two slots");
};

// Workgroup = (query, HT*16 heads, split of the index list), one wave per (head tile ht, dim
// slice dh) -- HT*DS waves. Per 32-row step:
//   every wave gathers 32/(HT*DS) rows into the step's ring slot (global_load_lds);
//   QK: wave (ht, dh) forms the partial S^T over its D/DS channels (Q^T slice in registers) and
//     the DS partials of a head tile are summed through LDS in a fixed order, so all DS waves of
//     the tile hold bit-identical scores and therefore identical softmax state;
//   PV: each wave accumulates O^T only for its own channel slice (D/DS x 16 heads).
// Register footprint per wave: Q^T slice D/DS/8 + accumulators D/DS/4 VGPRs.
// (__launch_bounds__'s second argument asks for 2 waves per SIMD: a 256-register budget, which
// keeps the accumulators in VGPRs instead of AGPR copies around every MFMA block.)
// CF: the compressed cache's format. kCompFp8: e4m3 rows + ue8m0 block scales; such a row and its
// scale bytes arrive in the second half of its bf16 slot row ([D, 2D) data, [2D, 2D + D/32)
// scales -- the row padding) with one copy instruction. kCompFp4: packed e2m1 rows with e4m3
// scales per 16 channels (D/2 + D/16 bytes, codes first), which arrive at the end of the bf16
// slot row, [2D - 9D/16, 2D). Either way copy counts and waits are unchanged; after its own
// copies land, the issuing wave dequantizes the row in place to bf16, before the step barrier.
// PAIR: the decode instance sized for two workgroups per CU (half the LDS: at most kPairList list
// entries, a two-slot ring), so that two independent step pipelines share each CU.
// CF | kWinFp8: the window ring is MXFP8 (rows of D e4m3 codes + D/32 ue8m0 scales, the layout
// of ring_store_fp8); such a row lands where an fp8 compressed row does.
constexpr int kCompBf16 = 0, kCompFp8 = 1, kCompFp4 = 2, kCompMask = 3, kWinFp8 = 4;

template <int CF>
struct CacheFmt {
  static constexpr bool F8 = (CF & kCompMask) == kCompFp8, F4 = (CF & kCompMask) == kCompFp4;
  static constexpr bool W8 = (CF & kWinFp8) != 0, PACKED = F8 || F4 || W8;
  static constexpr int F4ROW = 512 / 2 + 512 / 16;   // packed fp4 row bytes (D = 512)
  static constexpr int F4OFF = 2 * 512 - F4ROW;      // where it lands in the bf16 slot row
  static constexpr int W8ROW = 512 + 512 / 32;       // MXFP8 ring row bytes
};

// Unified position u of batch row b -> what a copy needs: a 16-byte aligned bf16 row address
// (tag 0), a packed compressed row (row << 2) | 1, an MXFP8 ring slot (slot << 2) | 2, or 0
// (masked; the zero row is gathered).
template <int D, int CF>
__device__ __forceinline__ uint64_t row_entry(const KvSrc& S, int b, int u) {
  using F = CacheFmt<CF>;
  const int ci = u - S.wp - S.n_chunk;
  if (F::W8 && u >= 0 && u < S.wp) return ((uint64_t)((S.ring_first + u) % S.window) << 2) | 2ull;
  return ((F::F8 || F::F4) && u >= 0 && ci >= 0 && ci < S.n_comp)
             ? (((uint64_t)ci << 2) | 1ull)
             : reinterpret_cast<uint64_t>(row_ptr<bf16_t>(S, b, u, D));
}

// Batch row b's bases of the packed sources (0 where the format has none).
struct PackedBase {
  uint64_t comp8, ring8, scal8;
  int rbs;   // scale row block (1 or 32) as a shift
};
template <int CF>
__device__ __forceinline__ PackedBase packed_base(const KvSrc& S, int b) {
  using F = CacheFmt<CF>;
  PackedBase p;
  p.comp8 = (F::F8 || F::F4) ? reinterpret_cast<uint64_t>(S.comp) + (uint64_t)b * (uint64_t)S.comp_bstride : 0ull;
  p.ring8 = F::W8 ? reinterpret_cast<uint64_t>(S.ring) + (uint64_t)b * (uint64_t)S.ring_bstride : 0ull;
  p.scal8 = F::F8 ? reinterpret_cast<uint64_t>(S.comp_scale) + (uint64_t)b * (uint64_t)S.comp_scale_bstride : 0ull;
  p.rbs = S.comp_scale_rb == 32 ? 5 : 0;
  return p;
}

// Layout of a staged row in LDS. Padded (mla_bf16_kernel): rows of 2D + 16 bytes, the bf16
// channels in order, packed bytes from D on (fp8 and MXFP8 scales in the padding). Swizzled
// (mla_roles_kernel): rows of 2D bytes, 16-byte chunk c of a bf16 row at chunk c ^ row_swz(r) (r:
// the row's index in its step), packed bytes ending at 2D.
template <int D, bool SWZ>
struct RowLayout {
  static constexpr int RS = SWZ ? 2 * D : 2 * D + 16;
  static constexpr int P8 = SWZ ? D - 16 : D;   // fp8 / MXFP8 codes, then their 16 scale bytes
};

// Chunk permutation of the swizzled layout, within each 256-byte group: row r's chunk c sits at
// c ^ row_swz(r). Bank-conflict counters over several layouts (measured on the two-role kernel):
// the transposed V reads (8 bytes per lane, rows r..r+3 and 64 bytes of each per 32 lanes) are
// conflict-free when row_swz / 4 takes 4 values over such rows, as here; the padded 1,040-byte rows
// and a plain XOR with r % 8 left them 2-way. The K fragment reads (16 bytes per lane, 16 rows at
// one chunk) counted 4 conflict cycles per instruction under every row-major layout tried, this
// one included; only lanes reading one contiguous 1 KB in lane order avoided that, which the
// transposed reads then pay for. Padding the P rows to 80 bytes removed their conflicts.
__device__ __forceinline__ int row_swz(int r) { return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }

// One wave copies RPW rows into LDS rows dst + rr * RS (lane rr < RPW holds row rr's entry; in
// the swizzled layout row rr is row r0 + rr of its step) and records each row's kind for the
// masking and the dequantization: 0 masked, 1 bf16, 2 packed compressed (tag 1), 3 MXFP8 ring
// (tag 2). Every row is whole copy instructions, the same count for every kind, so a step's copies
// are counted by vmcnt alone.
template <int D, int CF, int RPW, bool SWZ>
__device__ __forceinline__ void gather_rows(uint64_t mp, uint8_t* kind, uint32_t dst, int lane, const PackedBase& pb,
                                            int r0) {
  using F = CacheFmt<CF>;
  constexpr int RS = RowLayout<D, SWZ>::RS, P8 = RowLayout<D, SWZ>::P8;
  static_assert(!SWZ || D == 512, "swizzled rows: 512 channels");
  if (lane < RPW) kind[lane] = mp != 0ull ? (uint8_t)(1u + ((uint32_t)mp & 3u)) : 0;
  const uint32_t lo = (uint32_t)mp, hi = (uint32_t)(mp >> 32);
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const uint64_t ent = lane_u64(lo, hi, rr);
    const uint32_t tag = (uint32_t)ent & 3u;
    if (F::F8 && tag == 1u) {
      // lanes 0..31: the row's 512 fp8 bytes; lane 32: its 16 scale bytes
      const uint64_t ci = ent >> 2;
      const uint64_t src = lane < D / 16 ? pb.comp8 + ci * D + (uint64_t)lane * 16u
                                         : pb.scal8 + (ci >> pb.rbs) * (D / 32);
      if (lane <= D / 16) dma16_vaddr(src, dst + rr * RS + P8);
    } else if (F::F4 && tag == 1u) {
      // lanes 0..F4ROW/16-1: the row's codes and scales, one contiguous packed row
      const uint64_t src = pb.comp8 + (ent >> 2) * F::F4ROW + (uint64_t)lane * 16u;
      if (lane < F::F4ROW / 16) dma16_vaddr(src, dst + rr * RS + F::F4OFF);
    } else if (F::W8 && tag == 2u) {
      // lanes 0..32: the ring row's 512 codes and 16 scales, contiguous, to [P8, P8 + 528)
      const uint64_t src = pb.ring8 + (ent >> 2) * F::W8ROW + (uint64_t)lane * 16u;
      if (lane <= D / 16) dma16_vaddr(src, dst + rr * RS + P8);
    } else if constexpr (SWZ) {
      // lane l lands chunk l of the LDS row: it fetches chunk l ^ row_swz(r)
      dma16_sgpr(ent ? ent : reinterpret_cast<uint64_t>(g_zero_row), (uint32_t)(lane ^ row_swz(r0 + rr)) * 16u,
                 dst + rr * RS);
    } else {
      dma_row<D>(ent, dst + rr * RS, lane);
    }
  }
}

// A wave's own packed rows of a step have landed (sb: its first row, kind: their kinds):
// dequantize them in place. All of its rows are read before any is written (a single wave
// converts them), so the bf16 output may overlap the bytes it came from. Lane l converts channels
// 8l..8l+7 (its chunk, at chunk l ^ row_swz(r0 + rr) in the swizzled layout): fp8 rows (kind 3,
// or kind 2 of an fp8 compressed cache) hold their codes at [P8, P8 + D) and the ue8m0 scale of
// the lane's block at P8 + D + l/4; fp4 rows (kind 2) hold code bytes 4l..4l+3 at F4OFF and the
// e4m3 scale byte l/2 after the codes. The kinds come from one LDS read per 4 rows as
// wave-uniform values, so the loads of all rows go out together with no branch between them (a
// per-row conditional read serialized them: ~1 us per step).
template <int D, int CF, int RPW, bool SWZ>
__device__ __forceinline__ void dequant_rows(uint8_t* sb, const uint8_t* kind, int lane, int r0) {
  using F = CacheFmt<CF>;
  constexpr int RS = RowLayout<D, SWZ>::RS, P8 = RowLayout<D, SWZ>::P8;
  const uint32_t* kw = reinterpret_cast<const uint32_t*>(kind);
  uint32_t kinds[RPW / 4];
#pragma unroll
  for (int w4 = 0; w4 < RPW / 4; ++w4) kinds[w4] = (uint32_t)__builtin_amdgcn_readfirstlane((int)kw[w4]);
  uint2 raw[RPW];
  float sc[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const uint32_t k = (kinds[rr / 4] >> (8 * (rr % 4))) & 0xFFu;
    const bool f4row = F::F4 && k == 2u;
    const uint8_t* row = sb + rr * RS;
    raw[rr] = *reinterpret_cast<const uint2*>(row + (f4row ? F::F4OFF + lane * 4 : P8 + lane * 8));
    const uint32_t sbyte = row[f4row ? F::F4OFF + D / 2 + (lane >> 1) : P8 + D + (lane >> 2)];
    sc[rr] = f4row ? __builtin_amdgcn_cvt_f32_fp8((int)sbyte, 0) : e8m0_to_float(sbyte);
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const uint32_t k = (kinds[rr / 4] >> (8 * (rr % 4))) & 0xFFu;
    bf16x8* out = reinterpret_cast<bf16x8*>(sb + rr * RS + (SWZ ? lane ^ row_swz(r0 + rr) : lane) * 16);
    if (F::F4 && k == 2u) *out = dequant_e2m1x8(raw[rr].x, sc[rr]);
    else if (k >= 2u) *out = dequant_e4m3x8(raw[rr].x, raw[rr].y, sc[rr]);
  }
}

// Global address space: plain loads through such pointers are global_load (vmcnt only), where a
// generic pointer's flat_load would also hold lgkmcnt and so every LDS wait behind it.
#define GLOBAL __attribute__((address_space(1)))

// The register path of the two-slot decode ring (mla_bf16_kernel with NS = 2) for packed rows:
// instead of copying a packed row into LDS, reading it back and writing its bf16 form (~2x the
// LDS traffic of a bf16 row), lane l loads the row's bytes for channels 8l..8l+7 and their scale
// byte into registers when the step is issued; bf16 rows keep their LDS copies. raw/sb hold the
// wave's RPW rows of the next step, valid for the rows whose kind is 2 or 3.
//
// With an MXFP8 ring a list entry is resolved once, by the prologue's parallel pass (reg_row),
// into the row's code address with the entry's tag in its two low bits (every packed row starts
// 4-byte aligned) and its scale address; a bf16 or masked entry keeps its entry (tag 0) and gets
// the zero row as its scale address. A step then spends a few scalar instructions per row:
// resolving tags and row addresses at issue took ~590 scalar instructions per wave and step, and
// the CU's waves share one scalar unit (packed C4 1.572-1.580 -> 1.486-1.496 ms). With a bf16
// ring the per-kind branches below stay cheaper than the second LDS array (C5 1.180-1.182 against
// 1.193-1.196 ms), so there the entries stay as they are and ms is unused.
struct RegRow {
  uint64_t c, s;
};
template <int D, int CF>
__device__ __forceinline__ RegRow reg_row(uint64_t ent, const PackedBase& pb) {
  using F = CacheFmt<CF>;
  const uint32_t tag = (uint32_t)ent & 3u;
  const uint64_t idx = ent >> 2;
  RegRow r{ent, reinterpret_cast<uint64_t>(g_zero_row)};
  if ((F::F8 || F::F4) && tag == 1u) {
    constexpr uint64_t CROW = F::F4 ? (uint64_t)F::F4ROW : (uint64_t)D;
    const uint64_t row = pb.comp8 + idx * CROW;
    r.c = row | 1u;
    r.s = F::F8 ? pb.scal8 + (idx >> pb.rbs) * (D / 32) : row + D / 2;
  } else if (F::W8 && tag == 2u) {
    const uint64_t row = pb.ring8 + idx * F::W8ROW;
    r.c = row | 2u;
    r.s = row + D;
  }
  return r;
}

template <int D, int CF, int RPW>
__device__ __forceinline__ void gather_rows_reg(uint64_t mc, uint64_t ms, uint8_t* kind, uint32_t dst, int lane,
                                                const PackedBase& pb, uint2 (&raw)[RPW], uint32_t (&sb)[RPW]) {
  using F = CacheFmt<CF>;
  constexpr int RS = RowLayout<D, false>::RS;
  static_assert(D == 512, "packed rows: 512 channels, 8 per lane");
  static_assert(F::F4ROW % 4 == 0 && F::W8ROW % 4 == 0, "packed rows start 4-byte aligned: the tag fits below");
  if (lane < RPW) kind[lane] = mc != 0ull ? (uint8_t)(1u + ((uint32_t)mc & 3u)) : 0;
  const uint32_t clo = (uint32_t)mc, chi = (uint32_t)(mc >> 32), slo = (uint32_t)ms, shi = (uint32_t)(ms >> 32);
  const uint64_t zero = reinterpret_cast<uint64_t>(g_zero_row);
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const uint64_t ent = lane_u64(clo, chi, rr);
    const uint64_t sadr = lane_u64(slo, shi, rr);
    const uint32_t tag = (uint32_t)ent & 3u;
    if constexpr (F::W8) {
      // With an MXFP8 ring every row issues the same two loads into the same registers (a bf16
      // row reads the zero row and ignores it), from wave-uniform selects: with per-format
      // branches around the loads the compiler merged their registers after them and waited for
      // each load right where it was issued (3 us per 32-row step at B = 64). The scale comes as
      // the dword holding its byte (every scale base is 16-byte aligned): a byte load's
      // zero-extension consumed it at once.
      const bool packed = tag != 0u, c4 = F::F4 && tag == 1u;
      const uint64_t cbase = packed ? ent & ~3ull : zero;
      // codes: fp4 lanes read bytes 4l.. (8 bytes, the last 4 unused), fp8 lanes 8l..; scales:
      // fp4 block l/2 (16 channels), fp8 block l/4 (32 channels)
      const uint32_t coff = !packed ? 0u : (c4 ? (uint32_t)lane * 4u : (uint32_t)lane * 8u);
      const uint32_t soff = !packed ? 0u : (c4 ? (uint32_t)(lane >> 1) : (uint32_t)(lane >> 2));
      const uint64_t v = *reinterpret_cast<const GLOBAL uint64_t*>(cbase + coff);
      raw[rr] = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
      sb[rr] = *reinterpret_cast<const GLOBAL uint32_t*>((sadr + soff) & ~3ull);
      if (!packed) dma_row<D>(ent, dst + rr * RS, lane);
    } else {
      // compressed fp8 or fp4 rows, bf16 ring (entries as list_pos gives them): one branch per
      // kind (measured faster than the selects above here: the bf16 window rows issue no dummy
      // loads), the scale byte itself
      (void)sadr;
      const uint64_t idx = ent >> 2;
      if (tag == 1u) {
        if constexpr (F::F8) {
          const uint64_t v = *reinterpret_cast<const GLOBAL uint64_t*>(pb.comp8 + idx * D + (uint64_t)lane * 8u);
          raw[rr] = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
          sb[rr] = *reinterpret_cast<const GLOBAL uint8_t*>(pb.scal8 + (idx >> pb.rbs) * (D / 32) + (uint64_t)(lane >> 2));
        } else {
          const uint64_t row = pb.comp8 + idx * F::F4ROW;
          raw[rr].x = *reinterpret_cast<const GLOBAL uint32_t*>(row + (uint64_t)lane * 4u);
          sb[rr] = *reinterpret_cast<const GLOBAL uint8_t*>(row + D / 2 + (uint64_t)(lane >> 1));
        }
      } else {
        dma_row<D>(ent, dst + rr * RS, lane);
      }
    }
  }
}

// The step's loads have landed: this wave writes its packed rows to LDS as bf16 (lane l: its
// 16-byte chunk of each row). The kinds come back as wave-uniform words, as in dequant_rows.
template <int D, int CF, int RPW>
__device__ __forceinline__ void store_rows_reg(uint8_t* sbase, const uint8_t* kind, int lane, const uint2 (&raw)[RPW],
                                               const uint32_t (&sb)[RPW]) {
  using F = CacheFmt<CF>;
  constexpr int RS = RowLayout<D, false>::RS;
  const uint32_t* kw = reinterpret_cast<const uint32_t*>(kind);
  uint32_t kinds[RPW / 4];
#pragma unroll
  for (int w4 = 0; w4 < RPW / 4; ++w4) kinds[w4] = (uint32_t)__builtin_amdgcn_readfirstlane((int)kw[w4]);
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const uint32_t k = (kinds[rr / 4] >> (8 * (rr % 4))) & 0xFFu;
    bf16x8* out = reinterpret_cast<bf16x8*>(sbase + rr * RS + lane * 16);
    // with an MXFP8 ring sb holds the dword around the scale byte, otherwise the byte itself
    const int fsh = F::W8 ? 8 * ((lane >> 1) & 3) : 0, esh = F::W8 ? 8 * ((lane >> 2) & 3) : 0;
    if (F::F4 && k == 2u)
      *out = dequant_e2m1x8(raw[rr].x, __builtin_amdgcn_cvt_f32_fp8((int)((sb[rr] >> fsh) & 0xFFu), 0));
    else if (k >= 2u)
      *out = dequant_e4m3x8(raw[rr].x, raw[rr].y, e8m0_to_float((sb[rr] >> esh) & 0xFFu));
  }
}

template <int D, int HT, int DS, int CF, bool PAIR>
__global__ __launch_bounds__(64 * HT * DS, 2) void mla_bf16_kernel(MlaArgs a) {
  constexpr bool W8 = CacheFmt<CF>::W8, PACKED = CacheFmt<CF>::PACKED;
  constexpr int NW = HT * DS, NT = 64 * NW;
  constexpr int ML = PAIR ? kPairList : kMaxList;
  constexpr int DSL = D / DS, KSS = DSL / 32, DTS = DSL / 16;
  static_assert(DSL % 32 == 0, "dim slice must be a multiple of 32 channels");
  constexpr int R = kStepRows;
  static_assert(R % NW == 0, "rows per step must split evenly over the waves");
  constexpr int RPW = R / NW;
  constexpr int IPR = (D / 8 + 63) / 64;
  constexpr int NL = RPW * IPR;                 // copies each wave issues per step
  using Lds = MlaLds<D, NW, ML, PAIR ? kLdsBudget / 2 : kLdsBudget>;
  constexpr int RS = Lds::RS, SLOT = Lds::SLOT, NS = Lds::NS;
  static_assert(RS == RowLayout<D, false>::RS, "padded row layout");
  __shared__ __align__(16) uint8_t ring[NS * SLOT];
  __shared__ __align__(16) f32x4 xs[NW][2][64];
  // packed rows through registers: with two slots every step waits for all its loads (vmcnt 0),
  // so plain loads and the bf16 rows' LDS copies need no separate counts
  constexpr bool REG = PACKED && NS == 2;
  constexpr bool PRE = REG && W8;               // entries resolved to row addresses (reg_row)
  __shared__ uint64_t rows[ML];                 // resolved row addresses, 0 = masked (PRE: reg_row's .c)
  __shared__ uint64_t rows_s[PRE ? ML : 1];     // PRE: each entry's scale address (reg_row's .s)
  __shared__ __align__(4) uint8_t vrow[NS][R];
  __shared__ float rope_cs[2][kRopeRowPairs];   // the query position's (cos, sin) row of the q rope
  static_assert(sizeof(ring) + sizeof(xs) + sizeof(rows) + sizeof(rows_s) + sizeof(vrow) + sizeof(rope_cs) <=
                    (PAIR ? kLdsBudget / 2 : kLdsBudget),
                "LDS budget (PAIR: two workgroups per CU)");

  const KvSrc& S = a.src;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);   // (unit, split, head group), head group fastest
  const int hg = tile % a.hgroups;
  const int sp = (tile / a.hgroups) % a.splits;
  const int unit = tile / (a.hgroups * a.splits);
  const int b = unit / a.m, qs = unit - (unit / a.m) * a.m;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar address math
  const int ht = wave % HT, dh = wave / HT;
  if (a.ring_w && hg == 0 && sp == 0 && wave == 0) {
    if constexpr (W8) ring_store_fp8<D>(a, b, lane);
    else ring_store<bf16_t>(a, b, lane, 64);
  }
  const int wc = window_count(S, qs);
  // The split's entries: its share of the window rows, then its share of the index list (one
  // split takes the whole list). Window rows need no index read, so a split whose first step is
  // all window rows issues that step before its index entries arrive.
  const int ws = (wc + a.splits - 1) / a.splits, ks = (S.k + a.splits - 1) / a.splits;
  const int w0 = min(sp * ws, wc), nw = min(w0 + ws, wc) - w0;
  const int k0 = min(sp * ks, S.k), nk = min(k0 + ks, S.k) - k0;
  const int cnt = min(nw + nk, ML);             // planner: nw + nk <= ML
  auto entry_row = [&](int e) {                  // split entry -> copy entry (0 = masked)
    return row_entry<D, CF>(S, b, list_pos(S, b, a.m, qs, e < nw ? w0 + e : wc + k0 + (e - nw), wc));
  };
  static_assert(!PACKED || D == 512, "packed cache rows: 512 channels (one copy instruction per row)");

  const int nsteps = (cnt + R - 1) / R;
  const uint32_t ring_base = lds_offset(ring);
  const PackedBase pbase = packed_base<CF>(S, b);
  uint2 praw[RPW];
  uint32_t psb[RPW];
  auto list_entry = [&](int t) {                 // this wave's lane entry of step t (0 past the list)
    const int mine = t * R + wave * RPW + (lane % RPW);
    return mine < cnt ? rows[mine] : 0ull;
  };
  auto issue = [&](int t, bool direct) {
    const int slot = t % NS;
    const int mine = t * R + wave * RPW + (lane % RPW);
    const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(ring_base + (uint32_t)(slot * SLOT + wave * RPW * RS));
    if constexpr (PRE) {
      RegRow rr{0ull, reinterpret_cast<uint64_t>(g_zero_row)};
      if (mine < cnt) rr = direct ? reg_row<D, CF>(entry_row(mine), pbase) : RegRow{rows[mine], rows_s[mine]};
      gather_rows_reg<D, CF, RPW>(rr.c, rr.s, &vrow[slot][wave * RPW], dst, lane, pbase, praw, psb);
    } else if constexpr (REG) {
      const uint64_t mp = mine < cnt ? (direct ? entry_row(mine) : rows[mine]) : 0ull;
      gather_rows_reg<D, CF, RPW>(mp, 0ull, &vrow[slot][wave * RPW], dst, lane, pbase, praw, psb);
    } else {
      const uint64_t mp = mine < cnt ? (direct ? entry_row(mine) : rows[mine]) : 0ull;
      gather_rows<D, CF, RPW, false>(mp, &vrow[slot][wave * RPW], dst, lane, pbase, 0);
    }
  };
  const int h = hg * (HT * 16) + ht * 16 + l16;
  const bool hok = h < a.heads;
  bf16x8 qb[KSS];
  {
    const bf16_t* qrow =
        reinterpret_cast<const bf16_t*>(a.q) + ((int64_t)unit * a.heads + (hok ? h : 0)) * D + dh * DSL;
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks) qb[ks] = hok ? ld_bf16x8(qrow + ks * 32 + 8 * g) : zero_bf16x8();
  }
  // the q rope's table row goes out with the other prologue loads, one pair per thread, into LDS;
  // the rotation waits for the list barrier below (reading the table per pair inside the
  // rotation made one dependent round trip per pair, several us with the table out of cache)
  const bool rope_lds = a.q_rd > 0 && (a.q_rd >> 1) <= kRopeRowPairs;
  if (rope_lds && tid < (a.q_rd >> 1)) {
    const int64_t row = ((int64_t)a.start_pos + qs) * (a.q_rd >> 1);
    rope_cs[0][tid] = a.cos_tab[row + tid];
    rope_cs[1][tid] = a.sin_tab[row + tid];
  }
  if (a.q_rd > 0 && !rope_lds && hok) {
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks) {
      const int c0 = dh * DSL + ks * 32 + 8 * g;
      if (c0 + 8 > D - a.q_rd) qb[ks] = rope_q8(a, D, qs, c0, qb[ks]);
    }
  }
  const float sl2 = a.scale * kLog2e;
  // m_run: the exponent reference of acc and l_run, shared by the 4 lane groups of a head.
  // l_run: this lane's share of the denominator (its own rows); the lane groups are summed once
  // after the loop, so the sink term is seeded in lane group 0 only.
  float m_run = kNegFloor, l_run = 0.0f;
  if (sp == 0 && hok) {
    const float s2 = a.sink[h] * kLog2e;
    m_run = fmaxf(s2, kNegFloor);
    l_run = g == 0 ? exp2f(s2 - m_run) : 0.0f;
  }
  const bool early = nw >= R;                   // step 0: window rows only
  if (early) issue(0, true);
  // resolve the split's list once (segment, ring slot, batch row): no global reads are left
  // inside the copy pipeline and a step spends a few instructions per row
  for (int e = tid; e < cnt; e += NT) {
    if constexpr (PRE) {
      const RegRow rr = reg_row<D, CF>(entry_row(e), pbase);
      rows[e] = rr.c;
      rows_s[e] = rr.s;
    } else {
      rows[e] = entry_row(e);
    }
  }

  f32x4 acc[DTS];
#pragma unroll
  for (int dt = 0; dt < DTS; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The query, sink and list loads are complete on every path before the step loop. Without a
  // wait the compiler can see, it waits for the query registers at their first use inside the
  // loop -- vmcnt(0) at every step, which also drains the copies in flight.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();                         // rows[] and the rope row complete
  if (rope_lds && hok) {
    const int t0 = D - a.q_rd;             // first channel of the rope tail
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks) {
      const int c0 = dh * DSL + ks * 32 + 8 * g;
      if (dh * DSL + ks * 32 + 32 > t0) {  // wave-uniform: the chunk reaches into the tail
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)qb[ks][i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = c0 + 2 * j;
          const int pr = max(d - t0, 0) >> 1;
          const float cs = rope_cs[0][pr], sn = rope_cs[1][pr];
          float x0 = v[2 * j], x1 = v[2 * j + 1];
          rotate_pair(x0, x1, cs, sn);
          if (d >= t0) {
            v[2 * j] = x0;
            v[2 * j + 1] = x1;
          }
        }
        qb[ks] = cvt_bf16x8(v);
      }
    }
  }

  for (int t = early ? 1 : 0; t < nsteps && t < NS - 1; ++t) issue(t, false);
  // bf16 rows: a wave reads its list entries one step ahead of their copies, which then go out
  // right after the step barrier with no dependent LDS read in front of them (bs32 sparse MLA
  // 18.0-18.2 -> 17.7-17.8 us). Packed rows keep their issue after the QK MFMAs, measured faster
  // for them.
  uint64_t mp_next = 0ull;
  if constexpr (!PACKED)
    if (NS - 1 < nsteps) mp_next = list_entry(NS - 1);

  for (int t = 0; t < nsteps; ++t) {
    // REG: the same wait (two slots: vmcnt 0) as the builtin, so that the wait-count pass knows
    // the row registers have landed and adds no waits of its own where the next step reloads them
    if constexpr (REG) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    else wait_steps<NL>(min(nsteps - 1 - t, NS - 2));
    if constexpr (REG)   // this wave's packed rows of step t are in registers
      store_rows_reg<D, CF, RPW>(ring + (t % NS) * SLOT + wave * RPW * RS, &vrow[t % NS][wave * RPW], lane, praw, psb);
    else if constexpr (PACKED)   // this wave's own packed rows of step t have landed
      dequant_rows<D, CF, RPW, false>(ring + (t % NS) * SLOT + wave * RPW * RS, &vrow[t % NS][wave * RPW], lane, 0);
    __syncthreads();                       // step t landed; every wave is done with step t-1
    if constexpr (!PACKED) {               // slot (t-1) % NS is free past the barrier
      if (t + NS - 1 < nsteps) {
        const int ns = (t + NS - 1) % NS;
        const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(ring_base + (uint32_t)(ns * SLOT + wave * RPW * RS));
        gather_rows<D, CF, RPW, false>(mp_next, &vrow[ns][wave * RPW], dst, lane, pbase, 0);
        if (t + NS < nsteps) mp_next = list_entry(t + NS);
      }
    }
    const int slot = t % NS;
    const uint8_t* buf = ring + slot * SLOT;
    // four independent MFMA chains (row tile x k parity)
    f32x4 sq[2][2];
    sq[0][0] = sq[0][1] = sq[1][0] = sq[1][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        sq[rt][ks & 1] = mfma16x16x32(ld_bf16x8(buf + (rt * 16 + l16) * RS + (dh * DSL + ks * 32 + 8 * g) * 2),
                                      qb[ks], sq[rt][ks & 1]);
    // packed rows: the next copies go out while the MFMAs drain
    if constexpr (PACKED)
      if (t + NS - 1 < nsteps) issue(t + NS - 1, false);
    f32x4 sacc[2];
    sacc[0] = sq[0][0] + sq[0][1];
    sacc[1] = sq[1][0] + sq[1][1];
    if constexpr (DS > 1) {
      xs[wave][0][lane] = sacc[0];
      xs[wave][1][lane] = sacc[1];
      __syncthreads();
      sacc[0] = xs[ht][0][lane];
      sacc[1] = xs[ht][1][lane];
#pragma unroll
      for (int d2 = 1; d2 < DS; ++d2) {
        sacc[0] += xs[ht + HT * d2][0][lane];
        sacc[1] += xs[ht + HT * d2][1][lane];
      }
    }
    const uint32_t v0 = *reinterpret_cast<const uint32_t*>(&vrow[slot][4 * g]);
    const uint32_t v1 = *reinterpret_cast<const uint32_t*>(&vrow[slot][16 + 4 * g]);
    float p[8];
    float tmax = kNegFloor;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = (((rt ? v1 : v0) >> (8 * i)) & 0xFFu) != 0u;
        const float l2 = sacc[rt][i] * sl2;
        p[rt * 4 + i] = ok ? l2 : -INFINITY;
        if (ok) tmax = fmaxf(tmax, l2);
      }
    // lazy rescale: only when some lane's rows exceed the shared reference by kRescale is the
    // head's exact maximum over its 4 lane groups formed (two shuffles) and the reference moved
    if (__any(tmax > m_run + kRescale)) {
      float gmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      gmax = fmaxf(gmax, __shfl_xor(gmax, 32, 64));
      const bool grow = gmax > m_run + kRescale;
      const float alpha = grow ? fast_exp2(m_run - gmax) : 1.0f;
#pragma unroll
      for (int dt = 0; dt < DTS; ++dt) acc[dt] *= alpha;
      l_run *= alpha;
      m_run = grow ? gmax : m_run;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = fast_exp2(p[e] - m_run);
    const bf16x8 pb = cvt_bf16x8(p);
    // the denominator sums the weights as the PV product takes them (rounded to bf16), so every
    // output is a normalized average of its rows: the rounding moves weight between rows but
    // never scales a head's output
    {
      const uint4 pu = __builtin_bit_cast(uint4, pb);
      l_run += (sum_bf16x2(pu.x) + sum_bf16x2(pu.y)) + (sum_bf16x2(pu.z) + sum_bf16x2(pu.w));
    }
#pragma unroll
    for (int dt = 0; dt < DTS; ++dt) {
      const uint8_t* col = buf + (dh * DSL + dt * 16 + 4 * (l16 & 3)) * 2;
      const i16x4 lo = lds_read_tr16(col + (4 * g + (l16 >> 2)) * RS);
      const i16x4 hi = lds_read_tr16(col + (16 + 4 * g + (l16 >> 2)) * RS);
      acc[dt] = mfma16x16x32(join_bf16x8(lo, hi), pb, acc[dt]);
    }
  }

  l_run += __shfl_xor(l_run, 16, 64);      // denominator: sum of the 4 lane groups
  l_run += __shfl_xor(l_run, 32, 64);
  if (!hok) return;                        // no barrier follows
  // The two endings are separate straight-line blocks: this code runs once per workgroup with a
  // cold instruction cache, and one interleaved per-tile branch made it ~3,000 instructions.
  if (a.splits > 1) {
    // a split's partial is stored normalized (numerator / its own denominator) in bf16; a split
    // whose rows are all masked (denominator 0) stores zeros, which the combine weighs by 0
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    bf16_t* tile0 = a.part_o + part_tile(a, unit, sp, h, dh * DSL + 4 * g);
#pragma unroll
    for (int dt = 0; dt < DTS; ++dt) {
      uint2 st;
      st.x = pack2_bf16(acc[dt][0] * inv, acc[dt][1] * inv);
      st.y = pack2_bf16(acc[dt][2] * inv, acc[dt][3] * inv);
      *reinterpret_cast<uint2*>(tile0 + dt * 256) = st;   // next 16-channel tile: 256 elements on
    }
    if (dh == 0 && g == 0) {
      const int64_t slot_id = ((int64_t)unit * a.splits + sp) * a.heads + h;
      *reinterpret_cast<float2*>(a.part_ml + slot_id * 2) = make_float2(m_run, l_run);
    }
    return;
  }
  bf16_t* orow = reinterpret_cast<bf16_t*>(a.o) + ((int64_t)unit * a.heads + h) * D;
#pragma unroll
  for (int dt = 0; dt < DTS; ++dt) store_out4(a, D, qs, orow, dh * DSL + dt * 16 + 4 * g, acc[dt], l_run);
}

typedef __attribute__((ext_vector_type(16))) float f32x16;

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Sparse MLA for many queries with two wave roles (chunked prefill: rows of 512 channels, 64
// heads per workgroup, the whole list in one workgroup). In mla_bf16_kernel every wave runs
// the same serial step (QK, score exchange, softmax, PV) in lockstep with the other wave on its
// SIMD, so the MFMA pipe idles through the exchange and the softmax. Here each SIMD holds one
// wave of each role:
//   score waves 0-3, 16 heads each over all 512 channels: S^T = K Q^T of step t (Q^T in VGPRs),
//     masking, the running max and denominator with lazy rescaling, P rounded to bf16 into LDS
//     as P^T [head][row], and the step's rescale factor per head (1 when the max did not move);
//   value waves 4-7, all 64 heads x 128 channels each (v_mfma_f32_32x32x16_bf16, two 32-head
//     blocks per V^T fragment): O^T = alpha O^T + V^T P^T for step t - 1, with V^T through the
//     LDS transpose read.
// One barrier per step: past it, step t's rows are in LDS for the score waves and step t-1's P
// for the value waves, and the ring slot of step t-2 takes the copies of step t+2. A gathered row
// is read from LDS four times for QK and once for PV (mla_bf16_kernel: four and four, plus
// the partial-score exchange).
// Lane layouts of the 32x32x16 MFMA: lane l supplies A[l % 32][k] and B[k][l % 32] for
// k = 8 (l / 32) .. + 7, and receives D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] in accumulator
// register i.
// Copies, the in-place dequantization of packed rows (CF), masking, sink, lazy rescaling,
// rounding and the inverse rope are mla_bf16_kernel's; only the order of the fp32 additions in S
// and O differs.
constexpr int kRolesSlots = 4;          // ring: the score step, the value step, two in flight

template <int CF>
__global__ __launch_bounds__(512, 1) void mla_roles_kernel(MlaArgs a) {
  constexpr int D = 512, R = kStepRows, NT = 512, NS = kRolesSlots;
  constexpr int RS = RowLayout<D, true>::RS, SLOT = R * RS;
  constexpr int VR = R / 4;                       // rows each value wave copies per step
  constexpr int KSS = D / 32;
  __shared__ __align__(16) uint8_t ring[NS * SLOT];
  __shared__ uint64_t rows[kMaxList];             // resolved row entries, 0 = masked
  __shared__ __align__(16) uint8_t pbuf[2][64][R * 2 + 16];   // P^T: [head][row] bf16, rows padded
                                                  // to 80 bytes against bank conflicts
  __shared__ float abuf[2][64];                   // the step's rescale factor per head
  __shared__ float lbuf[64];                      // denominators
  __shared__ __align__(4) uint8_t vrow[NS][R];
  static_assert(sizeof(ring) + sizeof(rows) + sizeof(pbuf) + sizeof(abuf) + sizeof(lbuf) + sizeof(vrow) <=
                    kLdsBudget,
                "LDS budget");

  const KvSrc& S = a.src;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);   // (unit, head group), head group fastest
  const int hg = tile % a.hgroups, unit = tile / a.hgroups;
  const int b = unit / a.m, qs = unit - (unit / a.m) * a.m;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (a.ring_w && hg == 0 && wave == 0) {
    if constexpr (CacheFmt<CF>::W8) ring_store_fp8<D>(a, b, lane);
    else ring_store<bf16_t>(a, b, lane, 64);
  }
  const int wc = window_count(S, qs);
  const int cnt = min(wc + S.k, kMaxList);      // planner: the list fits
  const int nsteps = (cnt + R - 1) / R;
  for (int e = tid; e < cnt; e += NT) rows[e] = row_entry<D, CF>(S, b, list_pos(S, b, a.m, qs, e, wc));

  if (wave < 4) {
    // ---- score wave: heads ht * 16 + l16 of the group, all 512 channels
    const int ht = wave;
    const int hl = ht * 16 + l16;
    const int h = hg * 64 + hl;
    bf16x8 qb[KSS];
    const bf16_t* qrow = reinterpret_cast<const bf16_t*>(a.q) + ((int64_t)unit * a.heads + h) * D;
#pragma unroll
    for (int ks = 0; ks < KSS; ++ks) qb[ks] = ld_bf16x8(qrow + ks * 32 + 8 * g);
    if (a.q_rd > 0) {
#pragma unroll
      for (int ks = 0; ks < KSS; ++ks) {
        const int c0 = ks * 32 + 8 * g;
        if (c0 + 8 > D - a.q_rd) qb[ks] = rope_q8(a, D, qs, c0, qb[ks]);
      }
    }
    const float sl2 = a.scale * kLog2e;
    // m_run: the exponent reference shared by the head's 4 lane groups; l_run: this lane's share
    // of the denominator (its own rows), the sink seeded in lane group 0
    const float s2 = a.sink[h] * kLog2e;
    float m_run = fmaxf(s2, kNegFloor);
    float l_run = g == 0 ? exp2f(s2 - m_run) : 0.0f;
    // K fragment of k-step ks, row tile rt: row rt * 16 + l16, logical chunk 4 ks + g, stored at
    // chunk 4 ks ^ (g ^ row_swz(l16)): 256 (ks / 4) bytes on from the row plus a per-lane offset
    // for each ks % 4
    const int xk = g ^ row_swz(l16);
    const int ko[4] = {16 * xk, 16 * (4 ^ xk), 16 * (8 ^ xk), 16 * (12 ^ xk)};
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);    // q, sink and list loads done
    __syncthreads();                              // rows[] complete
    for (int t = 0; t <= nsteps; ++t) {
      __syncthreads();                            // step t landed; step t-1's P was taken
      if (t == nsteps) break;
      const int slot = t % NS;
      const uint8_t* buf = ring + slot * SLOT;
      f32x4 sq[2][2];
      sq[0][0] = sq[0][1] = sq[1][0] = sq[1][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSS; ++ks)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          sq[rt][ks & 1] = mfma16x16x32(ld_bf16x8(buf + (rt * 16 + l16) * RS + 256 * (ks >> 2) + ko[ks & 3]),
                                        qb[ks], sq[rt][ks & 1]);
      const f32x4 sacc[2] = {sq[0][0] + sq[0][1], sq[1][0] + sq[1][1]};
      const uint32_t v0 = *reinterpret_cast<const uint32_t*>(&vrow[slot][4 * g]);
      const uint32_t v1 = *reinterpret_cast<const uint32_t*>(&vrow[slot][16 + 4 * g]);
      float p[8];
      float tmax = kNegFloor;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = (((rt ? v1 : v0) >> (8 * i)) & 0xFFu) != 0u;
          const float l2 = sacc[rt][i] * sl2;
          p[rt * 4 + i] = ok ? l2 : -INFINITY;
          if (ok) tmax = fmaxf(tmax, l2);
        }
      float alpha = 1.0f;
      if (__any(tmax > m_run + kRescale)) {
        float gmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        gmax = fmaxf(gmax, __shfl_xor(gmax, 32, 64));
        const bool grow = gmax > m_run + kRescale;
        alpha = grow ? fast_exp2(m_run - gmax) : 1.0f;
        l_run *= alpha;
        m_run = grow ? gmax : m_run;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = fast_exp2(p[e] - m_run);
      // rows 16 rt + 4 g .. + 3 of head hl; the denominator sums the weights as the value waves
      // take them (rounded to bf16), so every output is a normalized average of its rows
      uint8_t* pt = &pbuf[t & 1][hl][0];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const uint32_t w0 = pack2_bf16(p[4 * rt], p[4 * rt + 1]), w1 = pack2_bf16(p[4 * rt + 2], p[4 * rt + 3]);
        *reinterpret_cast<uint2*>(pt + (16 * rt + 4 * g) * 2) = make_uint2(w0, w1);
        l_run += sum_bf16x2(w0) + sum_bf16x2(w1);
      }
      if (g == 0) abuf[t & 1][hl] = alpha;
    }
    l_run += __shfl_xor(l_run, 16, 64);           // denominator: sum of the 4 lane groups
    l_run += __shfl_xor(l_run, 32, 64);
    if (g == 0) lbuf[hl] = l_run;
    __syncthreads();                              // denominators to the value waves
    return;
  }

  // ---- value wave: all 64 heads of the group (two 32-head blocks hb, head hb * 32 + l32),
  // channels cb0 .. cb0 + 127; it also copies rows 8 vw .. 8 vw + 7 of every step (the score
  // waves' path is the longer one). Each V^T fragment feeds both head blocks, so a staged row is
  // read once for PV (four waves of 32 heads x 256 channels read it twice: 64 KB of LDS reads per
  // 32-row step instead of 32 KB, against 16 KB of P^T reads instead of 8).
  constexpr int DQ = D / 4;                       // channels per value wave
  const int vw = wave - 4, cb0 = vw * DQ;
  const int l32 = lane & 31, hi = lane >> 5, q4 = lane >> 4, r16 = lane & 15;
  const uint32_t ring_base = lds_offset(ring);
  const PackedBase pbase = packed_base<CF>(S, b);
  auto entry_of = [&](int t) -> uint64_t {
    const int mine = t * R + vw * VR + (lane % VR);
    return mine < cnt ? rows[mine] : 0ull;
  };
  auto issue = [&](int t, uint64_t mp) {
    const int slot = t % NS;
    const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(ring_base + (uint32_t)(slot * SLOT + vw * VR * RS));
    gather_rows<D, CF, VR, true>(mp, &vrow[slot][vw * VR], dst, lane, pbase, vw * VR);
  };
  // V^T fragments: the 16-lane group q4 reads channels 16 (q4 & 1) + (0..15) of a 32-channel tile
  // ct, rows 16 kk + vrb (lo) and 16 kk + vrb + 4 (hi), 8 bytes each. Logical chunk 4 ct + j of
  // such a row (j = 2 (q4 & 1) + (r16 & 3) / 2, counted from channel cb0) sits at chunk
  // 4 ct ^ (j ^ row_swz(row)): 256 (ct / 4) bytes on plus a per-lane offset for each ct % 4.
  const int vrb = 8 * (q4 >> 1) + (r16 >> 2);
  const int jv = 2 * (q4 & 1) + ((r16 & 3) >> 1);
  const int xl = jv ^ row_swz(vrb), xh = jv ^ row_swz(vrb + 4), e8 = 8 * (r16 & 1);
  const int vlo[4] = {16 * xl + e8, 16 * (4 ^ xl) + e8, 16 * (8 ^ xl) + e8, 16 * (12 ^ xl) + e8};
  const int vhi[4] = {16 * xh + e8, 16 * (4 ^ xh) + e8, 16 * (8 ^ xh) + e8, 16 * (12 ^ xh) + e8};
  f32x16 acc[DQ / 32][2];
#pragma unroll
  for (int ct = 0; ct < DQ / 32; ++ct)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[ct][hb][i] = 0.0f;
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();                                // rows[] complete
  for (int t = 0; t < NS - 2 && t < nsteps; ++t) issue(t, entry_of(t));
  for (int t = 0; t <= nsteps; ++t) {
    const uint64_t mp = t + NS - 2 < nsteps ? entry_of(t + NS - 2) : 0ull;
    if (t < nsteps) {
      wait_steps<VR>(min(NS - 3, nsteps - 1 - t));   // this wave's rows of step t landed
      if constexpr (CacheFmt<CF>::PACKED)
        dequant_rows<D, CF, VR, true>(ring + (t % NS) * SLOT + vw * VR * RS, &vrow[t % NS][vw * VR], lane, vw * VR);
    }
    __syncthreads();                              // step t-1's P and rescale factors are in LDS
    if (t + NS - 2 < nsteps) issue(t + NS - 2, mp);   // into step t-2's slot
    if (t == 0) continue;
    const int s = t - 1;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const float alpha = abuf[s & 1][hb * 32 + l32];
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int ct = 0; ct < DQ / 32; ++ct) acc[ct][hb] *= alpha;
      }
    }
    // P^T as the B operand of two 16-row k-steps per head block: rows 16 kk + 8 hi .. + 7 of head
    // hb * 32 + l32
    bf16x8 pbk[2][2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const uint8_t* pt = &pbuf[s & 1][hb * 32 + l32][0];
      pbk[hb][0] = ld_bf16x8(pt + (8 * hi) * 2);
      pbk[hb][1] = ld_bf16x8(pt + (16 + 8 * hi) * 2);
    }
    const uint8_t* buf = ring + (s % NS) * SLOT + 2 * cb0;
#pragma unroll
    for (int ct = 0; ct < DQ / 32; ++ct) {
      const uint8_t* col = buf + 256 * (ct >> 2);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const i16x4 lo4 = lds_read_tr16(col + (16 * kk + vrb) * RS + vlo[ct & 3]);
        const i16x4 hi4 = lds_read_tr16(col + (16 * kk + vrb + 4) * RS + vhi[ct & 3]);
        const bf16x8 vt = join_bf16x8(lo4, hi4);
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) acc[ct][hb] = mfma32x32x16(vt, pbk[hb][kk], acc[ct][hb]);
      }
    }
  }
  __syncthreads();                                // denominators written
  // accumulator register i of tile (ct, hb): channel cb0 + 32 ct + 8 (i / 4) + 4 hi + i % 4 of
  // head hb * 32 + l32
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    const int hl = hb * 32 + l32;
    const float den = lbuf[hl];
    bf16_t* orow = reinterpret_cast<bf16_t*>(a.o) + ((int64_t)unit * a.heads + hg * 64 + hl) * D;
#pragma unroll
    for (int ct = 0; ct < DQ / 32; ++ct)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        store_out4(a, D, qs, orow, cb0 + 32 * ct + 8 * j + 4 * hi,
                   f32x4{acc[ct][hb][4 * j], acc[ct][hb][4 * j + 1], acc[ct][hb][4 * j + 2], acc[ct][hb][4 * j + 3]},
                   den);
  }
}

// Merges split partials of one query. The partials lie in 16-head x 16-channel tiles of 512
// contiguous bytes (part_tile), and the merge reads them in that order: a wave takes two
// neighbouring channel tiles of one 16-head tile, lane l the 8 channels (l & 1) * 8 .. + 7 of head
// (l & 31) / 2 in tile l / 32, so each split's read is 1 KB contiguous per wave. (One head per
// wave read 32-byte pieces 512 bytes apart.) The workgroups of a query are numbered as the
// attention launch numbers its tiles (xcd_tile), so they read the partials on the XCD whose L2 the
// attention workgroups wrote them to. Split s holds (m_s, l_s, o_s) = (log2-domain max,
// denominator, numerator / l_s in bf16); the merged row is sum_s w_s o_s / sum_s w_s with
// w_s = l_s 2^(m_s - M). NB numerator chunks and (m, l) pairs (splits clamped to the last one,
// whose weight past ns is 0) are loaded together before any weight is formed; splits beyond NB
// are streamed.
template <typename T, int NB>
__global__ __launch_bounds__(256) void mla_combine_kernel(MlaArgs a) {
  const int D = a.dim, ns = a.splits;
  const int htiles = (a.heads + 15) >> 4, dpairs = D >> 5;
  const int wpu = (htiles * dpairs + 3) >> 2;                  // workgroups per query
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int unit = tile / wpu;
  const int lane = threadIdx.x & 63;
  const int idx = (tile - unit * wpu) * 4 + (threadIdx.x >> 6);   // (head tile, channel-tile pair)
  if (idx >= htiles * dpairs) return;
  const int ht = idx / dpairs, dp = idx - ht * dpairs;
  const int h = ht * 16 + ((lane & 31) >> 1);
  const int d = (2 * dp + (lane >> 5)) * 16 + (lane & 1) * 8;
  if (h >= a.heads) return;
  const int qs = unit % a.m;
  const int64_t slot0 = (int64_t)unit * ns * a.heads + h;     // split s: slot0 + s * heads
  T* orow = reinterpret_cast<T*>(a.o) + ((int64_t)unit * a.heads + h) * D;
  auto part = [&](int s) { return *reinterpret_cast<const uint4*>(a.part_o + part_tile(a, unit, s, h, d)); };
  // the inverse-rope factors of this lane's pairs are fetched with the partials (unpredicated:
  // a pair outside the tail reads the table's first pair of its row and ignores it)
  float cs[4] = {0.f, 0.f, 0.f, 0.f}, sn[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.rd > 0) {
    const int64_t row = ((int64_t)a.start_pos + qs) * (a.rd >> 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = max(d + 2 * j - (D - a.rd), 0) >> 1;
      cs[j] = a.cos_tab[row + p];
      sn[j] = a.sin_tab[row + p];
    }
  }
  uint4 pv[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) pv[s] = part(s < ns ? s : ns - 1);
  auto ml = [&](int s) { return *reinterpret_cast<const float2*>(a.part_ml + (slot0 + (int64_t)s * a.heads) * 2); };
  float2 mlv[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) mlv[s] = ml(s < ns ? s : ns - 1);
  float M = kNegFloor;
#pragma unroll
  for (int s = 0; s < NB; ++s) M = s < ns ? fmaxf(M, mlv[s].x) : M;
  for (int s = NB; s < ns; ++s) M = fmaxf(M, ml(s).x);
  float wv[NB], den = 0.0f;
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    wv[s] = s < ns ? mlv[s].y * exp2f(mlv[s].x - M) : 0.0f;
    den += wv[s];
  }
  for (int s = NB; s < ns; ++s) {
    const float2 v = ml(s);
    den += v.y * exp2f(v.x - M);
  }
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add = [&](int s, const uint4& v) {
    float w;
    if (s < NB) {
      w = 0.0f;
#pragma unroll
      for (int t = 0; t < NB; ++t) w = t == s ? wv[t] : w;
    } else {
      const float2 m2 = ml(s);
      w = m2.y * exp2f(m2.x - M);
    }
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] += w * __uint_as_float(wd[i] << 16);
      x[2 * i + 1] += w * __uint_as_float(wd[i] & 0xFFFF0000u);
    }
  };
#pragma unroll
  for (int s = 0; s < NB; ++s) add(s, pv[s]);
  for (int s = NB; s < ns; ++s) add(s, part(s));
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = io<T>::rnd(x[i] / den);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (in_rope_tail(a, D, d + 2 * j)) rope_inv_apply(cs[j], -sn[j], v[2 * j], v[2 * j + 1]);
  if constexpr (sizeof(T) == 2) {
    uint4 st;
    st.x = pack2_bf16(v[0], v[1]);
    st.y = pack2_bf16(v[2], v[3]);
    st.z = pack2_bf16(v[4], v[5]);
    st.w = pack2_bf16(v[6], v[7]);
    *reinterpret_cast<uint4*>(orow + d) = st;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) io<T>::st(orow + d + i, v[i]);
  }
}

template <int NB>
static void launch_combine(const MlaArgs& a, int64_t units, hipStream_t stream) {
  const int wpu = (((a.heads + 15) >> 4) * (a.dim >> 5) + 3) >> 2;   // workgroups per query
  hipLaunchKernelGGL((mla_combine_kernel<bf16_t, NB>), dim3((unsigned)(units * wpu)), dim3(256), 0, stream, a);
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
  if (a.ring_w && blockIdx.y == 0) ring_store<float>(a, b, tid, 256);
  const int wc = window_count(S, qs);
  const int L = wc + S.k;
  const float* qrow = reinterpret_cast<const float*>(a.q) + (int64_t)unit * a.heads * D;
  for (int i = 2 * tid; i < kF32Heads * D; i += 512) {   // adjacent pairs: D is even
    const int h = hbase + i / D, d = i % D;
    float x0 = 0.0f, x1 = 0.0f;
    if (h < a.heads) {
      x0 = qrow[(int64_t)h * D + d];
      x1 = qrow[(int64_t)h * D + d + 1];
      rope_q_pair(a, D, qs, d, x0, x1);
    }
    q_l[i] = x0;
    q_l[i + 1] = x1;
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
  bool wide;                     // 64-head workgroups of 8 waves (else 32-head, 4 waves)
  bool pair;                     // decode instance with half the LDS, two workgroups per CU
  int hgroups, splits, per_split;
};

// Many queries (prefill): one workgroup per (query, head group) over the whole list, 64 heads
// per workgroup when there are more than 32. Few queries (decode): (query, 32-head, split)
// workgroups, the list split in whole 32-row steps until about 256 workgroups exist -- or 512,
// two per CU, when there are already >= 128 (query, head group) units or the list is >= 1024
// entries long (measured: bs32 / 640 rows is fastest at 4 splits, B=16 / 1152 rows and B=64 at
// ~2 workgroups per CU). Splits of at most kPairList entries with head_dim <= 512 run the PAIR
// instance (~77 KB of LDS, a two-slot ring), the rest one ~160 KB workgroup per CU. A workgroup
// stages at most kMaxList list entries.
static MlaPlan plan_bf16(int64_t units, int heads, int list_max, int dim) {
  MlaPlan p{};
  const int lm = list_max > 0 ? list_max : 1;
  const int hg32 = (heads + 31) / 32;
  if (units * hg32 >= 512 && lm <= kMaxList) {
    p.wide = heads > 32;
    p.hgroups = p.wide ? (heads + 63) / 64 : hg32;
    p.splits = 1;
    p.per_split = lm;
    return p;
  }
  p.wide = false;
  p.hgroups = hg32;
  const int64_t wgs = units * p.hgroups;
  const int64_t target = dim <= 512 && wgs >= 128 ? 512 : 256;
  int want = wgs < target ? (int)((target + wgs - 1) / wgs) : 1;
  const int cap = (lm + kStepRows - 1) / kStepRows;
  if (want > cap) want = cap;
  if (want > 16) want = 16;
  if (want < 1) want = 1;
  auto per = [&](int w) { return ((lm + w - 1) / w + kStepRows - 1) / kStepRows * kStepRows; };
  p.per_split = per(want);
  // a split holds ceil(window / splits) + ceil(k / splits) <= per_split + 1 entries
  p.pair = dim <= 512 && p.per_split + 1 <= kPairList;
  while (p.per_split + 1 > (p.pair ? kPairList : kMaxList)) p.per_split = per(++want);
  p.splits = (lm + p.per_split - 1) / p.per_split;
  return p;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Split partials: numerators in 16-head tiles (heads rounded up to 16), then (max, denominator).
static size_t part_o_bytes(const MlaPlan& p, int64_t units, int heads, int dim) {
  return align256((size_t)units * p.splits * ((heads + 15) / 16 * 16) * dim * sizeof(bf16_t));
}

static size_t workspace_for(const MlaPlan& p, int64_t units, int heads, int dim) {
  if (p.splits <= 1) return 0;
  const size_t slots = (size_t)units * p.splits * heads;
  return part_o_bytes(p, units, heads, dim) + align256(slots * 2 * sizeof(float));
}

static bool bf16_dim_supported(int d) { return d == 64 || d == 128 || d == 256 || d == 512 || d == 576; }

template <int D, int CF>
static void launch_bf16_d(const MlaArgs& a, const MlaPlan& p, int64_t units, hipStream_t stream) {
  const unsigned wgs = (unsigned)(units * p.hgroups * p.splits);
  if constexpr (D <= 512) {                    // the planner pairs only rows of up to 512 channels
    if (p.pair && !p.wide) {
      hipLaunchKernelGGL((mla_bf16_kernel<D, 2, 2, CF, true>), dim3(wgs), dim3(256), 0, stream, a);
      return;
    }
  }
  if (D == 512 && p.wide && a.heads % 64 == 0)
    hipLaunchKernelGGL(mla_roles_kernel<CF>, dim3(wgs), dim3(512), 0, stream, a);
  else if (p.wide)
    hipLaunchKernelGGL((mla_bf16_kernel<D, 4, 2, CF, false>), dim3(wgs), dim3(512), 0, stream, a);
  else
    hipLaunchKernelGGL((mla_bf16_kernel<D, 2, 2, CF, false>), dim3(wgs), dim3(256), 0, stream, a);
}

// comp_format: kCompFp8, the compressed source is an e4m3 cache with ue8m0 block scales; kCompFp4,
// packed e2m1 rows with e4m3 scales per 16 channels (q, o and the other sources are bf16; head_dim
// 512).
static int run_mla(const char* what, MlaArgs a, int64_t units, int list_max, int dtype, void* workspace,
                   size_t workspace_bytes, hipStream_t stream, int comp_format = kCompBf16) {
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
  const MlaPlan p = plan_bf16(units, a.heads, list_max, a.dim);
  DSV41_REQUIRE(units * p.hgroups * p.splits < (1ll << 31), DSV41_E_ARG, "%s: too many workgroups", what);
  DSV41_REQUIRE(p.splits <= 64, DSV41_E_SHAPE, "%s: index list of %d entries is too long for the decode path", what,
                list_max);
  a.hgroups = p.hgroups;
  a.splits = p.splits;
  a.per_split = p.per_split;
  const size_t need = workspace_for(p, units, a.heads, a.dim);
  if (need) {
    DSV41_REQUIRE(workspace && workspace_bytes >= need, DSV41_E_WORKSPACE, "%s: workspace of %zu bytes needed",
                  what, need);
    DSV41_REQUIRE(aligned16(workspace), DSV41_E_ARG, "%s: workspace must be 16-byte aligned", what);
    a.part_o = reinterpret_cast<bf16_t*>(workspace);
    a.part_ml = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + part_o_bytes(p, units, a.heads, a.dim));
  }
  if (comp_format != kCompBf16) {
    DSV41_REQUIRE(a.dim == 512, DSV41_E_SHAPE, "%s: the packed cache paths support dim 512, got %d", what, a.dim);
    if (comp_format == kCompFp8) launch_bf16_d<512, kCompFp8>(a, p, units, stream);
    else if (comp_format == kCompFp4) launch_bf16_d<512, kCompFp4>(a, p, units, stream);
    else if (comp_format == (kCompFp4 | kWinFp8)) launch_bf16_d<512, kCompFp4 | kWinFp8>(a, p, units, stream);
    else return set_error(DSV41_E_ARG, "%s: no kernel for cache format %d", what, comp_format);
  } else {
    switch (a.dim) {
      case 64: launch_bf16_d<64, kCompBf16>(a, p, units, stream); break;
      case 128: launch_bf16_d<128, kCompBf16>(a, p, units, stream); break;
      case 256: launch_bf16_d<256, kCompBf16>(a, p, units, stream); break;
      case 512: launch_bf16_d<512, kCompBf16>(a, p, units, stream); break;
      default: launch_bf16_d<576, kCompBf16>(a, p, units, stream); break;
    }
  }
  int rc = check_launch(what);
  if (rc || p.splits == 1) return rc;
  if (p.splits <= 2) launch_combine<2>(a, units, stream);
  else if (p.splits <= 4) launch_combine<4>(a, units, stream);
  else if (p.splits <= 8) launch_combine<8>(a, units, stream);
  else launch_combine<16>(a, units, stream);
  return check_launch(what);
}

}  // namespace dsv41

using namespace dsv41;

extern "C" size_t dsv41_sparse_mla_workspace_bytes(int32_t bsz, int32_t m, int32_t heads, int32_t dim,
                                                   int32_t rows_per_query, int32_t dtype) {
  if (dtype != DSV41_BF16 || bsz <= 0 || m <= 0 || heads <= 0 || dim <= 0) return 0;
  const int64_t units = (int64_t)bsz * m;
  return workspace_for(plan_bf16(units, heads, rows_per_query, dim), units, heads, dim);
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

static int sparse_mla_layer(const char* what, const void* q, const void* win_kv, const void* chunk_kv,
                            const void* comp_kv, int64_t comp_bstride, int32_t n_comp, const float* sink,
                            const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads, int32_t dim,
                            int32_t window, int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab,
                            int32_t rd, int32_t q_rd, int32_t dtype, void* workspace, size_t workspace_bytes,
                            bool write_ring, hipStream_t stream) {
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
  DSV41_REQUIRE(q_rd == 0 || (q_rd > 0 && cos_tab && sin_tab && q_rd % 2 == 0 && q_rd <= dim &&
                              (rd == 0 || rd == q_rd)),
                DSV41_E_ARG, "%s: bad query rope tail (q_rd %d, rd %d)", what, q_rd, rd);
  MlaArgs a{};
  a.q = q; a.o = o; a.sink = sink;
  a.src.ring = win_kv; a.src.ring_bstride = (int64_t)window * dim; a.src.window = window; a.src.wp = wp;
  a.src.ring_first = (start_pos - wp) % window;
  a.src.chunk = chunk_kv; a.src.chunk_bstride = (int64_t)n * dim; a.src.n_chunk = n;
  a.src.comp = comp_kv; a.src.comp_bstride = comp_bstride; a.src.n_comp = n_comp;
  a.src.idx = idx; a.src.k = k; a.src.win_implicit = 1;
  a.m = n; a.heads = heads; a.dim = dim; a.scale = scale;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.q_rd = q_rd; a.start_pos = start_pos;
  if (write_ring) {
    DSV41_REQUIRE(n == 1 && win_kv, DSV41_E_ARG, "%s: the ring store needs one token per row and a ring", what);
    a.ring_w = const_cast<void*>(win_kv);
  }
  const int weff = window < wp + n ? window : wp + n;
  return run_mla(what, a, (int64_t)bsz * n, weff + k, dtype, workspace, workspace_bytes, stream);
}

extern "C" int dsv41_sparse_mla(const void* q, const void* win_kv, const void* chunk_kv, const void* comp_kv,
                                int64_t comp_bstride, int32_t n_comp, const float* sink, const int32_t* idx, int32_t k,
                                void* o, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t window,
                                int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab, int32_t rd,
                                int32_t q_rd, int32_t dtype, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
  return sparse_mla_layer("dsv41_sparse_mla", q, win_kv, chunk_kv, comp_kv, comp_bstride, n_comp, sink, idx, k, o, bsz,
                          n, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd, dtype, workspace,
                          workspace_bytes, false, stream);
}

extern "C" int dsv41_sparse_mla_decode(const void* q, void* win_kv, const void* chunk_kv, const void* comp_kv,
                                       int64_t comp_bstride, int32_t n_comp, const float* sink, const int32_t* idx,
                                       int32_t k, void* o, int32_t bsz, int32_t heads, int32_t dim, int32_t window,
                                       int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab,
                                       int32_t rd, int32_t q_rd, int32_t dtype, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
  return sparse_mla_layer("dsv41_sparse_mla_decode", q, win_kv, chunk_kv, comp_kv, comp_bstride, n_comp, sink, idx, k,
                          o, bsz, 1, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd, dtype, workspace,
                          workspace_bytes, true, stream);
}

// ------------------------------------------------------------------ allocation-free decode
//
// dsv41_sparse_mla_decode_noalloc keeps the split partials in `scratch`, a file-scope device array
// (one copy per GPU, held for the life of the process), instead of a caller workspace. Host code
// never passes the array's name to a kernel: on the host that name is a stand-in, not a device
// address. The device address is looked up once per device, with that device current, and kept.

constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;   // 32 MiB per GPU
constexpr int kMaxScratchDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's address of `scratch`, looked up on its first use on that device.
static int scratch_of_current_device(const char* what, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error((int)e, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  DSV41_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, DSV41_E_ARG, "%s: device %d beyond the %d the scratch table holds",
                what, dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return set_error((int)e, "%s: hipGetSymbolAddress(scratch) failed: %s", what,
                                          hipGetErrorString(e));
    DSV41_REQUIRE(p != nullptr, DSV41_E_ARG, "%s: scratch has no address on device %d", what, dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

extern "C" int dsv41_sparse_mla_decode_noalloc(const void* q, void* win_kv, const void* chunk_kv, const void* comp_kv,
                                               int64_t comp_bstride, int32_t n_comp, const float* sink,
                                               const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t heads,
                                               int32_t dim, int32_t window, int32_t start_pos, float scale,
                                               const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                                               int32_t dtype, hipStream_t stream) {
  const char* what = "dsv41_sparse_mla_decode_noalloc";
  const int wp = start_pos < window ? start_pos : window;
  const int weff = window < wp + 1 ? window : wp + 1;
  size_t need = 0;
  if (dtype == DSV41_BF16 && bsz > 0 && heads > 0 && dim > 0 && k >= 0)
    need = workspace_for(plan_bf16(bsz, heads, weff + k, dim), bsz, heads, dim);
  DSV41_REQUIRE(need <= kNoAllocScratchBytes, DSV41_E_WORKSPACE,
                "%s: this shape needs %zu bytes of split scratch, beyond the %zu-byte static buffer (use "
                "dsv41_sparse_mla_decode with a workspace)", what, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need) {
    int rc = scratch_of_current_device(what, &ws);
    if (rc) return rc;
  }
  return sparse_mla_layer(what, q, win_kv, chunk_kv, comp_kv, comp_bstride, n_comp, sink, idx, k, o, bsz, 1, heads, dim,
                          window, start_pos, scale, cos_tab, sin_tab, rd, q_rd, dtype, ws, need, true, stream);
}

static int sparse_mla_fp8_layer(const char* what, const void* q, const void* win_kv, const void* chunk_kv,
                                const uint8_t* comp_kv, int64_t comp_bstride, int32_t n_comp, const uint8_t* comp_scale,
                                int64_t comp_scale_bstride, int32_t comp_scale_rb, const float* sink,
                                const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads,
                                int32_t dim, int32_t window, int32_t start_pos, float scale, const float* cos_tab,
                                const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes,
                                bool write_ring, hipStream_t stream) {
  const int wp = start_pos < window ? start_pos : window;
  DSV41_REQUIRE(q && chunk_kv && sink && o && (idx || k == 0) && (win_kv || wp == 0) &&
                    ((comp_kv && comp_scale) || n_comp == 0),
                DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && window > 0 && start_pos >= 0 && k >= 0 && n_comp >= 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dim == 512, DSV41_E_SHAPE, "%s: the fp8 cache path supports dim 512, got %d", what, dim);
  DSV41_REQUIRE(comp_scale_rb == 1 || comp_scale_rb == 32, DSV41_E_ARG, "%s: scale row block must be 1 or 32", what);
  DSV41_REQUIRE(n_comp == 0 || comp_bstride >= (int64_t)n_comp * dim, DSV41_E_ARG, "%s: comp_bstride too small", what);
  DSV41_REQUIRE(n_comp == 0 || comp_scale_bstride >= (int64_t)((n_comp + comp_scale_rb - 1) / comp_scale_rb) * (dim / 32),
                DSV41_E_ARG, "%s: comp_scale_bstride too small", what);
  DSV41_REQUIRE(aligned16(q) && aligned16(chunk_kv) && aligned16(o) && (!win_kv || aligned16(win_kv)) &&
                    (!comp_kv || (aligned16(comp_kv) && aligned16(comp_scale))),
                DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  DSV41_REQUIRE(comp_bstride % 16 == 0 && comp_scale_bstride % 16 == 0, DSV41_E_ARG,
                "%s: comp_bstride and comp_scale_bstride must be multiples of 16 bytes", what);
  DSV41_REQUIRE(rd == 0 || (cos_tab && sin_tab && rd % 2 == 0 && rd <= dim), DSV41_E_ARG, "%s: bad rope tail", what);
  DSV41_REQUIRE(q_rd == 0 || (q_rd > 0 && cos_tab && sin_tab && q_rd % 2 == 0 && q_rd <= dim &&
                              (rd == 0 || rd == q_rd)),
                DSV41_E_ARG, "%s: bad query rope tail (q_rd %d, rd %d)", what, q_rd, rd);
  MlaArgs a{};
  a.q = q; a.o = o; a.sink = sink;
  a.src.ring = win_kv; a.src.ring_bstride = (int64_t)window * dim; a.src.window = window; a.src.wp = wp;
  a.src.ring_first = (start_pos - wp) % window;
  a.src.chunk = chunk_kv; a.src.chunk_bstride = (int64_t)n * dim; a.src.n_chunk = n;
  a.src.comp = comp_kv; a.src.comp_bstride = comp_bstride; a.src.n_comp = n_comp;
  a.src.comp_scale = comp_scale; a.src.comp_scale_bstride = comp_scale_bstride; a.src.comp_scale_rb = comp_scale_rb;
  a.src.idx = idx; a.src.k = k; a.src.win_implicit = 1;
  a.m = n; a.heads = heads; a.dim = dim; a.scale = scale;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.q_rd = q_rd; a.start_pos = start_pos;
  if (write_ring) {
    DSV41_REQUIRE(n == 1 && win_kv, DSV41_E_ARG, "%s: the ring store needs one token per row and a ring", what);
    a.ring_w = const_cast<void*>(win_kv);
  }
  const int weff = window < wp + n ? window : wp + n;
  return run_mla(what, a, (int64_t)bsz * n, weff + k, DSV41_BF16, workspace, workspace_bytes, stream, kCompFp8);
}

// The compressed source as packed fp4 rows: e2m1 codes then e4m3 scales per 16 channels, 288 bytes
// per 512-channel row, comp_bstride bytes per batch row. ring8_bstride > 0: the window ring is
// MXFP8 rows (512 e4m3 codes + 16 ue8m0 scales, 528 bytes), ring8_bstride bytes per batch row;
// else it is bf16.
static int sparse_mla_fp4_layer(const char* what, const void* q, const void* win_kv, const void* chunk_kv,
                                const uint8_t* comp_kv4, int64_t comp_bstride, int32_t n_comp, const float* sink,
                                const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads,
                                int32_t dim, int32_t window, int32_t start_pos, float scale, const float* cos_tab,
                                const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes,
                                bool write_ring, hipStream_t stream, int64_t ring8_bstride = 0) {
  const int wp = start_pos < window ? start_pos : window;
  DSV41_REQUIRE(q && chunk_kv && sink && o && (idx || k == 0) && (win_kv || wp == 0) && (comp_kv4 || n_comp == 0),
                DSV41_E_ARG, "%s: null tensor", what);
  DSV41_REQUIRE(bsz >= 0 && n >= 0 && heads > 0 && window > 0 && start_pos >= 0 && k >= 0 && n_comp >= 0,
                DSV41_E_ARG, "%s: bad sizes", what);
  DSV41_REQUIRE(dim == 512, DSV41_E_SHAPE, "%s: the packed fp4 cache path supports dim 512, got %d", what, dim);
  const int64_t row = dim / 2 + dim / 16;
  DSV41_REQUIRE(n_comp == 0 || comp_bstride >= (int64_t)n_comp * row, DSV41_E_ARG, "%s: comp_bstride too small", what);
  DSV41_REQUIRE(aligned16(q) && aligned16(chunk_kv) && aligned16(o) && (!win_kv || aligned16(win_kv)) &&
                    (!comp_kv4 || aligned16(comp_kv4)),
                DSV41_E_ARG, "%s: tensors must be 16-byte aligned", what);
  DSV41_REQUIRE(comp_bstride % 16 == 0, DSV41_E_ARG, "%s: comp_bstride must be a multiple of 16 bytes", what);
  DSV41_REQUIRE(rd == 0 || (cos_tab && sin_tab && rd % 2 == 0 && rd <= dim), DSV41_E_ARG, "%s: bad rope tail", what);
  DSV41_REQUIRE(q_rd == 0 || (q_rd > 0 && cos_tab && sin_tab && q_rd % 2 == 0 && q_rd <= dim &&
                              (rd == 0 || rd == q_rd)),
                DSV41_E_ARG, "%s: bad query rope tail (q_rd %d, rd %d)", what, q_rd, rd);
  const bool w8 = ring8_bstride > 0;
  if (w8)
    DSV41_REQUIRE(ring8_bstride >= (int64_t)window * (dim + dim / 32) && ring8_bstride % 16 == 0, DSV41_E_ARG,
                  "%s: the ring's batch stride must hold %d rows of %d bytes and be a multiple of 16", what, window,
                  dim + dim / 32);
  MlaArgs a{};
  a.q = q; a.o = o; a.sink = sink;
  a.src.ring = win_kv; a.src.ring_bstride = w8 ? ring8_bstride : (int64_t)window * dim; a.src.window = window;
  a.src.wp = wp;
  a.src.ring_first = (start_pos - wp) % window;
  a.src.chunk = chunk_kv; a.src.chunk_bstride = (int64_t)n * dim; a.src.n_chunk = n;
  a.src.comp = comp_kv4; a.src.comp_bstride = comp_bstride; a.src.n_comp = n_comp;
  a.src.idx = idx; a.src.k = k; a.src.win_implicit = 1;
  a.m = n; a.heads = heads; a.dim = dim; a.scale = scale;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rd = rd; a.q_rd = q_rd; a.start_pos = start_pos;
  if (write_ring) {
    DSV41_REQUIRE(n == 1 && win_kv, DSV41_E_ARG, "%s: the ring store needs one token per row and a ring", what);
    a.ring_w = const_cast<void*>(win_kv);
  }
  const int weff = window < wp + n ? window : wp + n;
  return run_mla(what, a, (int64_t)bsz * n, weff + k, DSV41_BF16, workspace, workspace_bytes, stream,
                 w8 ? (kCompFp4 | kWinFp8) : kCompFp4);
}

extern "C" int dsv41_sparse_mla_packed(const void* q, const uint8_t* win_kv8, int64_t ring_bstride,
                                       const void* chunk_kv, const uint8_t* comp_kv4, int64_t comp_bstride,
                                       int32_t n_comp, const float* sink, const int32_t* idx, int32_t k, void* o,
                                       int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t window,
                                       int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab,
                                       int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
  DSV41_REQUIRE(ring_bstride > 0, DSV41_E_ARG, "dsv41_sparse_mla_packed: ring_bstride must be positive");
  return sparse_mla_fp4_layer("dsv41_sparse_mla_packed", q, win_kv8, chunk_kv, comp_kv4, comp_bstride, n_comp, sink,
                              idx, k, o, bsz, n, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd,
                              workspace, workspace_bytes, false, stream, ring_bstride);
}

extern "C" int dsv41_sparse_mla_packed_decode(const void* q, uint8_t* win_kv8, int64_t ring_bstride,
                                              const void* chunk_kv, const uint8_t* comp_kv4, int64_t comp_bstride,
                                              int32_t n_comp, const float* sink, const int32_t* idx, int32_t k, void* o,
                                              int32_t bsz, int32_t heads, int32_t dim, int32_t window,
                                              int32_t start_pos, float scale, const float* cos_tab,
                                              const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace,
                                              size_t workspace_bytes, hipStream_t stream) {
  DSV41_REQUIRE(ring_bstride > 0, DSV41_E_ARG, "dsv41_sparse_mla_packed_decode: ring_bstride must be positive");
  return sparse_mla_fp4_layer("dsv41_sparse_mla_packed_decode", q, win_kv8, chunk_kv, comp_kv4, comp_bstride, n_comp,
                              sink, idx, k, o, bsz, 1, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd,
                              workspace, workspace_bytes, true, stream, ring_bstride);
}

extern "C" int dsv41_sparse_mla_fp4(const void* q, const void* win_kv, const void* chunk_kv, const uint8_t* comp_kv4,
                                    int64_t comp_bstride, int32_t n_comp, const float* sink, const int32_t* idx,
                                    int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads, int32_t dim,
                                    int32_t window, int32_t start_pos, float scale, const float* cos_tab,
                                    const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  return sparse_mla_fp4_layer("dsv41_sparse_mla_fp4", q, win_kv, chunk_kv, comp_kv4, comp_bstride, n_comp, sink, idx, k,
                              o, bsz, n, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd, workspace,
                              workspace_bytes, false, stream);
}

extern "C" int dsv41_sparse_mla_fp4_decode(const void* q, void* win_kv, const void* chunk_kv, const uint8_t* comp_kv4,
                                           int64_t comp_bstride, int32_t n_comp, const float* sink, const int32_t* idx,
                                           int32_t k, void* o, int32_t bsz, int32_t heads, int32_t dim, int32_t window,
                                           int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab,
                                           int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
  return sparse_mla_fp4_layer("dsv41_sparse_mla_fp4_decode", q, win_kv, chunk_kv, comp_kv4, comp_bstride, n_comp, sink,
                              idx, k, o, bsz, 1, heads, dim, window, start_pos, scale, cos_tab, sin_tab, rd, q_rd,
                              workspace, workspace_bytes, true, stream);
}

extern "C" int dsv41_sparse_mla_fp8(const void* q, const void* win_kv, const void* chunk_kv, const uint8_t* comp_kv,
                                    int64_t comp_bstride, int32_t n_comp, const uint8_t* comp_scale,
                                    int64_t comp_scale_bstride, int32_t comp_scale_rb, const float* sink,
                                    const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads,
                                    int32_t dim, int32_t window, int32_t start_pos, float scale, const float* cos_tab,
                                    const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  return sparse_mla_fp8_layer("dsv41_sparse_mla_fp8", q, win_kv, chunk_kv, comp_kv, comp_bstride, n_comp, comp_scale,
                              comp_scale_bstride, comp_scale_rb, sink, idx, k, o, bsz, n, heads, dim, window, start_pos,
                              scale, cos_tab, sin_tab, rd, q_rd, workspace, workspace_bytes, false, stream);
}

extern "C" int dsv41_sparse_mla_fp8_decode(const void* q, void* win_kv, const void* chunk_kv, const uint8_t* comp_kv,
                                           int64_t comp_bstride, int32_t n_comp, const uint8_t* comp_scale,
                                           int64_t comp_scale_bstride, int32_t comp_scale_rb, const float* sink,
                                           const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t heads,
                                           int32_t dim, int32_t window, int32_t start_pos, float scale,
                                           const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return sparse_mla_fp8_layer("dsv41_sparse_mla_fp8_decode", q, win_kv, chunk_kv, comp_kv, comp_bstride, n_comp,
                              comp_scale, comp_scale_bstride, comp_scale_rb, sink, idx, k, o, bsz, 1, heads, dim,
                              window, start_pos, scale, cos_tab, sin_tab, rd, q_rd, workspace, workspace_bytes, true,
                              stream);
}
