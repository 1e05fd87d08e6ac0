/*
 * dsv41.h -- C ABI of the MI355X (gfx950) DeepSeek-V4.1 sparse-attention hot path.
 *
 * One extern "C" entry point per kernel. Conventions shared by every entry point:
 *   - all tensor arguments are raw device pointers to contiguous row-major memory,
 *     described by explicit sizes (and, for caches, a batch stride in elements);
 *   - `dtype` arguments take a dsv41_dtype value; bf16 is stored as raw 16-bit words;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the default stream) and
 *     nothing synchronises with the host; no entry point allocates device memory:
 *     scratch space is passed in by the caller, sized by the *_workspace_bytes query;
 *   - the return value is 0 on success, a negative dsv41_status for a contract
 *     violation (bad size, dtype, null pointer, unsupported shape), or a positive
 *     hipError_t from the launch; dsv41_last_error_string() then describes it
 *     (thread-local, valid until the next call on the same thread);
 *   - calls are stateless and reentrant, with one exception: dsv41_sparse_mla_decode_noalloc
 *     keeps its split partials in one process-wide static device array per GPU, so its calls
 *     on one GPU must be ordered on one stream (overlapping calls race on that array).
 *
 * Reference citations name files of the reference repository (thedracle/deepseek-v41-mlx):
 * the MLX modules under deepseek_v41_mlx/ and DeepSeek's TileLang kernels in
 * docs/reference/kernel.py, whose wrappers are the native seam the reference's tests
 * swap out (tests/test_parity.py:57-58).
 */
#ifndef DSV41_H
#define DSV41_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  DSV41_F32 = 0,      /* float32 */
  DSV41_BF16 = 1,     /* bfloat16 (raw uint16) */
  DSV41_FP8_E4M3 = 2  /* OCP e4m3fn bytes + ue8m0 (biased exponent) scale bytes */
} dsv41_dtype;

typedef enum {
  DSV41_OK = 0,
  DSV41_E_ARG = -1,         /* null pointer or a size out of range */
  DSV41_E_DTYPE = -2,       /* dtype not supported by this entry point */
  DSV41_E_SHAPE = -3,       /* shape not supported (e.g. head_dim not a multiple of 32) */
  DSV41_E_WORKSPACE = -4    /* workspace missing or too small */
} dsv41_status;

/* Library identification and the last error of the calling thread. */
const char* dsv41_version(void);
const char* dsv41_last_error_string(void);

/* ---------------------------------------------------------------- fake-quant --
 * In-place-capable (x == y allowed) QAT round trips over the last dimension,
 * `rows` rows of `cols` elements, `cols % block == 0`. dtype is F32 or BF16 (in == out).
 */

/* fake_quant_fp8_ue8m0, deepseek_v41_mlx/fakequant.py:83-93;
 * act_quant(x, block, scale_fmt="ue8m0", inplace=True), docs/reference/kernel.py:98-124. */
int dsv41_fq_fp8_ue8m0(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                       int32_t dtype, hipStream_t stream);

/* fake_quant_fp4_ue8m0, deepseek_v41_mlx/fakequant.py:96-106;
 * fp4_act_quant(x, block, inplace=True), docs/reference/kernel.py:184-204. */
int dsv41_fq_fp4_ue8m0(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                       int32_t dtype, hipStream_t stream);

/* fake_quant_fp4_e4m3, deepseek_v41_mlx/fakequant.py:109-119;
 * fp4_act_quant(x, block, inplace=True, scale_dtype=float8_e4m3fn), kernel.py:160-163. */
int dsv41_fq_fp4_e4m3(const void* x, void* y, int64_t rows, int32_t cols, int32_t block,
                      int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------- rope / norm --
 */

/* cos/sin tables [seqlen, half] of the fp32 angles t*freqs[i] (the trigonometric half of
 * precompute_freqs_cis, deepseek_v41_mlx/layers.py:36-56; freqs[half] comes from the host). */
int dsv41_rope_table(float* cos_out, float* sin_out, const float* freqs, int32_t seqlen,
                     int32_t half, hipStream_t stream);

/* rope_tail, deepseek_v41_mlx/layers.py:59-84: rotate adjacent pairs of the last `rd`
 * channels of x [bsz, seqlen, heads, dim] (heads = 1 for 3-D tensors) by the angle of
 * position pos_base + s * pos_step (s = token index); inverse != 0 conjugates.
 * The first dim - rd channels are copied unchanged. x == y allowed. dim % 32 == 0 and
 * dim / 32 a power of two <= 64. */
int dsv41_rope_tail(const void* x, void* y, int32_t bsz, int32_t seqlen, int32_t heads,
                    int32_t dim, int32_t rd, const float* cos_tab, const float* sin_tab,
                    int32_t pos_base, int32_t pos_step, int32_t inverse, int32_t dtype,
                    hipStream_t stream);

/* RMSNorm, deepseek_v41_mlx/layers.py:20-33: y = cast(w * x * rsqrt(mean(x^2) + eps)),
 * computed in fp32, over `rows` rows of `dim` elements. x == y allowed. */
int dsv41_rmsnorm(const void* x, void* y, const float* weight, int64_t rows, int32_t dim,
                  float eps, int32_t dtype, hipStream_t stream);

/* The residual add of one block and the next block's attn_norm, deepseek_v41_mlx/model.py:141-154
 * (h = h + attn(attn_norm(h)), MoE and hyper-connections as identity) with the RMSNorm of
 * layers.py:20-33: h <- cast(h + delta) in place, then y = rmsnorm(h, weight) as dsv41_rmsnorm
 * computes it. Rows of `dim` elements, dim a multiple of 8 (bf16) or 4 (fp32), at most 8,192 bf16
 * or 4,096 fp32 channels, 16-byte aligned; y must not alias h or delta. */
int dsv41_add_rmsnorm(void* h, const void* delta, void* y, const float* weight, int64_t rows,
                      int32_t dim, float eps, int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------- window KV --
 */

/* The window-KV prologue of Attention.__call__, deepseek_v41_mlx/attention.py:119-122:
 * kv [bsz, n, dim] <- fake_quant_fp8_ue8m0(rope_tail(kv_norm(kv), positions start_pos+s), 32),
 * in place, with the dtype rounding between the three steps that the reference performs. */
int dsv41_kv_window_prep(void* kv, const float* norm_w, const float* cos_tab,
                         const float* sin_tab, int32_t bsz, int32_t n, int32_t dim, int32_t rd,
                         int32_t start_pos, float eps, int32_t dtype, hipStream_t stream);

/* LayerCache.write_window, deepseek_v41_mlx/cache.py:61-67: the last min(n, window) rows
 * of kv [bsz, n, dim] go to ring slots (pos) % window of win_kv [bsz, window, dim]. */
int dsv41_window_write(void* win_kv, const void* kv, int32_t bsz, int32_t n, int32_t dim,
                       int32_t window, int32_t start_pos, int32_t dtype, hipStream_t stream);

/* dsv41_window_write into an MXFP8 ring, the lossless packed form of the window KV's fp8 QAT
 * (attention.py:120-122, fakequant.py:83-93): per row dim e4m3fn codes, then one ue8m0 scale
 * byte per 32 channels (dim + dim/32 bytes; 528 at dim 512), win_kv8 [bsz, window, row] with
 * ring_bstride bytes per batch row (a multiple of 8). Each row is stored as
 * fake_quant_fp8_ue8m0's codes and scales, so decoding gives exactly the QAT values the window KV
 * already holds (values that do not carry the QAT are quantized by it). */
int dsv41_window_write_mxfp8(uint8_t* win_kv8, int64_t ring_bstride, const void* kv, int32_t bsz,
                             int32_t n, int32_t dim, int32_t window, int32_t start_pos, int32_t dtype,
                             hipStream_t stream);

/* window_idx_matrix, deepseek_v41_mlx/attention.py:40-50: out [n, min(window, wp+n)] int32. */
int dsv41_window_idx(int32_t* out, int32_t wp, int32_t n, int32_t window, hipStream_t stream);

/* ---------------------------------------------------------------- compressor --
 */

/* Compressor.__call__ after its two fp32 projections, deepseek_v41_mlx/compressor.py:58-79
 * (ratio > 1): prepend the m = start_pos % ratio carried rows of kv_state/score_state
 * [bsz, ratio, dim] (fp32, updated in place with the new remainder), pool every complete
 * group with a per-channel softmax over the ratio axis, RMSNorm the pooled vector (after the
 * reference's cast to dtype) and write latents [bsz, g, dim], g = (m + n) / ratio (latents
 * may be NULL when g == 0). kv, score: [bsz, n, dim] fp32. dim <= 1024. */
int dsv41_compress_pool(const float* kv, const float* score, float* kv_state, float* score_state,
                        void* latents, const float* norm_w, int32_t bsz, int32_t n, int32_t dim,
                        int32_t ratio, int32_t start_pos, float eps, int32_t dtype,
                        hipStream_t stream);

/* The compressed-cache write of Attention.__call__, deepseek_v41_mlx/attention.py:157-163:
 * comp_kv[b, g0 + j] <- fake_quant_fp4_e4m3(rope_tail(latents[b, j], position (g0+j)*ratio), 16)
 * for latents [bsz, g, dim]; comp_kv has `cache_bstride` elements per batch row. */
int dsv41_comp_write(const void* latents, void* comp_kv, int64_t cache_bstride,
                     const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                     int32_t dim, int32_t rd, int32_t g0, int32_t ratio, int32_t dtype,
                     hipStream_t stream);

/* dsv41_comp_write into a packed fp4 cache, the lossless packed form of the same
 * fake_quant_fp4_e4m3 values (attention.py:157-163, fakequant.py:109-118): per row dim/2 bytes
 * of e2m1 codes (byte p holds channels 2p, 2p+1, the even one in the low nibble), then one e4m3fn
 * scale byte per 16 channels (the block's fake-quant scale) -- dim/2 + dim/16 bytes per row
 * (288 at dim 512), comp_kv4 [bsz, >=g0+g, row] with cache_bstride bytes per batch row (both
 * multiples of 16). Decoding e2m1(code) * scale gives exactly dsv41_comp_write's values. */
int dsv41_comp_write_fp4(const void* latents, uint8_t* comp_kv4, int64_t cache_bstride,
                         const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                         int32_t dim, int32_t rd, int32_t g0, int32_t ratio, int32_t dtype,
                         hipStream_t stream);

/* Indexer.publish_keys after the wk projection, deepseek_v41_mlx/indexer.py:89-104:
 * index_k[b, g0 + j] <- fake_quant_fp4_ue8m0(rope_tail(k_norm(k_raw[b, j]), (g0+j)*ratio), 32)
 * for k_raw [bsz, g, dim]; index_k has `cache_bstride` elements per batch row. */
int dsv41_index_key_publish(const void* k_raw, void* index_k, int64_t cache_bstride,
                            const float* norm_w, const float* cos_tab, const float* sin_tab,
                            int32_t bsz, int32_t g, int32_t dim, int32_t rd, int32_t g0,
                            int32_t ratio, float eps, int32_t dtype, hipStream_t stream);

/* The writers of the fp8 cache variant: the compressed-cache write (attention.py:157-163) and
 * the index-key publish (indexer.py:89-104) with the row's values -- rope(latent), resp.
 * rope(k_norm(k_raw)), in dtype -- quantized by fake_quant_fp8_ue8m0's formula
 * (fakequant.py:83-93) and stored packed: e4m3fn codes [bsz, >=g0+g, dim] and one ue8m0 scale
 * byte per 32 channels of every scale_rb rows [bsz, >=ceil((g0+g)/scale_rb), dim/32] (the
 * layout of dsv41_sparse_mla_fp8 / dsv41_indexer_score_fp8), batch strides in bytes. This
 * replaces the reference's fp4 QAT at these two stores. scale_rb = 1: decoding gives
 * fake_quant_fp8_ue8m0(value). scale_rb = 32 (32 x 32 blocks): a row that opens a block
 * (row % 32 == 0) sets the block's scale by that formula and the block's later rows, in this
 * call or later ones, are rounded with it: e4m3(clip(value / scale, +-448)) * scale. */
int dsv41_comp_write_fp8(const void* latents, uint8_t* codes, int64_t c_bstride, uint8_t* scales,
                         int64_t s_bstride, int32_t scale_rb, const float* cos_tab, const float* sin_tab,
                         int32_t bsz, int32_t g, int32_t dim, int32_t rd, int32_t g0, int32_t ratio,
                         int32_t dtype, hipStream_t stream);
int dsv41_index_key_publish_fp8(const void* k_raw, uint8_t* codes, int64_t c_bstride, uint8_t* scales,
                                int64_t s_bstride, int32_t scale_rb, const float* norm_w,
                                const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                                int32_t dim, int32_t rd, int32_t g0, int32_t ratio, float eps,
                                int32_t dtype, hipStream_t stream);

/* dsv41_index_key_publish into an MXFP4 index cache, the lossless packed form of the same
 * fake_quant_fp4_ue8m0 keys (indexer.py:100-104): per 32-channel block one ue8m0 scale byte
 * (scale 2^(e-127), the block's fake-quant scale) and 16 bytes of e2m1 codes (byte p holds
 * channels 2p, 2p+1 of the block, the even one in the low nibble). k_codes [bsz, >=g0+g, dim/2]
 * and k_scales [bsz, >=g0+g, dim/32] bytes with kc_bstride / ks_bstride bytes per batch row.
 * Decoding e2m1(code) * scale gives exactly dsv41_index_key_publish's values. */
int dsv41_index_key_publish_mxfp4(const void* k_raw, uint8_t* k_codes, int64_t kc_bstride,
                                  uint8_t* k_scales, int64_t ks_bstride, const float* norm_w,
                                  const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t g,
                                  int32_t dim, int32_t rd, int32_t g0, int32_t ratio, float eps,
                                  int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------- indexer --
 */

/* The index-query prologue, deepseek_v41_mlx/indexer.py:119-121: in place on
 * q [bsz, n, heads, dim], q <- fake_quant_fp4_ue8m0(rope_tail(q, positions start_pos+s), 32). */
int dsv41_index_q_prep(void* q, const float* cos_tab, const float* sin_tab, int32_t bsz,
                       int32_t n, int32_t heads, int32_t dim, int32_t rd, int32_t start_pos,
                       int32_t dtype, hipStream_t stream);

/* Indexer scoring, deepseek_v41_mlx/indexer.py:123-138:
 *   scores[b,s,t] = sum_h relu(q[b,s,h,:] . index_k[b,t,:]) * w[b,s,h]      (fp32)
 *   w = round_dtype(w_raw * w_scale); t >= (start_pos+s+1)/ratio -> -inf;
 *   candidates (optional, uint8 [bsz,n,nb], 0 = masked) -> -inf.
 * q [bsz,n,heads,dim], w_raw [bsz,n,heads] in `dtype`; index_k rows of `dim` elements with
 * `k_bstride` elements per batch row (the owner's cache read in place); scores [bsz,n,nb].
 * dtype F32 or BF16; bf16 runs on MFMA and needs heads % 16 == 0 and dim % 32 == 0. */
int dsv41_indexer_score(const void* q, const void* w_raw, float w_scale, const void* index_k,
                        int64_t k_bstride, const uint8_t* candidates, float* scores,
                        int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                        int32_t start_pos, int32_t ratio, int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------- top-k --
 */

/* dsv41_indexer_score with fp8 index keys: the packed, lossless form of the fp4/ue8m0-QAT keys
 * publish_keys stores (indexer.py:89-104) or of the fp8 cache variant. index_k holds e4m3fn
 * bytes [bsz, >=nb, 128] (k_bstride bytes per batch row); k_scale holds one ue8m0 byte per 32
 * channels for every ks_rb rows (1 or 32): [bsz, ceil(nb / ks_rb), 4], ks_bstride bytes per
 * batch row. Keys are dequantized to bf16 in-kernel (exact), so scores equal
 * dsv41_indexer_score's on the dequantized keys. q and w_raw are bf16; dim is 128. */
int dsv41_indexer_score_fp8(const void* q, const void* w_raw, float w_scale, const uint8_t* index_k,
                            int64_t k_bstride, const uint8_t* k_scale, int64_t ks_bstride,
                            int32_t ks_rb, const uint8_t* candidates, float* scores, int32_t bsz,
                            int32_t n, int32_t heads, int32_t dim, int32_t nb, int32_t start_pos,
                            int32_t ratio, hipStream_t stream);

/* dsv41_index_q_prep writing the query in MXFP4 form (the layout of
 * dsv41_index_key_publish_mxfp4): q [bsz, n, heads, dim] is read, not modified;
 * q_codes [bsz, n, heads, dim/2] and q_scales [bsz, n, heads, dim/32] bytes receive
 * fake_quant_fp4_ue8m0(rope_tail(q)) losslessly packed (indexer.py:119-121). */
int dsv41_index_q_prep_mxfp4(const void* q, uint8_t* q_codes, uint8_t* q_scales,
                             const float* cos_tab, const float* sin_tab, int32_t bsz, int32_t n,
                             int32_t heads, int32_t dim, int32_t rd, int32_t start_pos,
                             int32_t dtype, hipStream_t stream);

/* dsv41_indexer_score with query and keys in MXFP4 form (dsv41_index_q_prep_mxfp4 and
 * dsv41_index_key_publish_mxfp4 layouts; dim 128: 64 code bytes and 4 scale bytes per head
 * or key). Each 16-head x 16-key tile is one block-scaled fp4 MFMA over the 128 channels
 * (exact products, fp32 sums), so the scores equal dsv41_indexer_score's on the decoded
 * values up to fp32 summation order. w_raw bf16; heads 16, 32 or 64; k_codes / k_scales with
 * kc_bstride / ks_bstride bytes per batch row. */
int dsv41_indexer_score_mxfp4(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                              float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                              const uint8_t* k_scales, int64_t ks_bstride, const uint8_t* candidates,
                              float* scores, int32_t bsz, int32_t n, int32_t heads, int32_t dim,
                              int32_t nb, int32_t start_pos, int32_t ratio, hipStream_t stream);

/* dsv41_indexer_score with the query in MXFP4 form (dsv41_index_q_prep_mxfp4; the index query is
 * fp4 fake-quantized by construction, indexer.py:119-121, so the form is lossless) against fp8
 * e4m3 keys in the layout of dsv41_indexer_score_fp8 (ue8m0 scales per 32 channels of every
 * ks_rb = 1 or 32 rows). Each 16-head x 16-key tile is one block-scaled MFMA over the 128
 * channels with fp4 A and fp8 B operands (exact products, fp32 sums): the scores equal
 * dsv41_indexer_score_fp8's up to fp32 summation order, without dequantizing the keys.
 * Heads 16, 32 or 64; dim 128. */
int dsv41_indexer_score_mxq_fp8(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                                float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                                const uint8_t* k_scales, int64_t ks_bstride, int32_t ks_rb,
                                const uint8_t* candidates, float* scores, int32_t bsz, int32_t n,
                                int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                                hipStream_t stream);

/* Indexer scoring followed by top-k selection, fused for decode (deepseek_v41_mlx/indexer.py:
 * 115-144: the scores of dsv41_indexer_score, then the selection of dsv41_topk_select, with
 * identical results): the [bsz*n, nb] scores are never written -- each workgroup's row range
 * keeps its best k (key, position) pairs in the workspace and a merge selects each query's k.
 * Served shapes: bf16 keys of dim 128, 16/32/64 heads, n < 8 or a candidate mask, row ranges of
 * 512, 1024, 2048 or 4096 rows at least four times k, and at most 32768 listed pairs per query;
 * dsv41_indexer_topk_workspace_bytes returns 0 for the others (the entry point then returns
 * DSV41_E_SHAPE). out [bsz*n, k] int32, k = min(topk, nb). The workspace is 16-byte aligned;
 * calls that share one must not overlap (same stream, or ordered by events). */
size_t dsv41_indexer_topk_workspace_bytes(int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                                          int32_t topk, int32_t has_candidates);
int dsv41_indexer_topk(const void* q, const void* w_raw, float w_scale, const void* index_k,
                       int64_t k_bstride, const uint8_t* candidates, int32_t* out, int32_t bsz,
                       int32_t n, int32_t heads, int32_t dim, int32_t nb, int32_t start_pos,
                       int32_t ratio, int32_t topk, int32_t offset, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* dsv41_indexer_topk over fp8 index keys (the layout of dsv41_indexer_score_fp8: e4m3 codes with
 * k_bstride bytes per batch row, ue8m0 scales per 32 channels of every ks_rb = 1 or 32 rows with
 * ks_bstride bytes per batch row): bit-equal to dsv41_indexer_score_fp8 followed by
 * dsv41_topk_select. Served shapes and the workspace are dsv41_indexer_topk's (same size query);
 * q, w_raw, index_k and k_scale 16-byte aligned, both strides multiples of 16 bytes. */
int dsv41_indexer_topk_fp8(const void* q, const void* w_raw, float w_scale, const uint8_t* index_k,
                           int64_t k_bstride, const uint8_t* k_scale, int64_t ks_bstride, int32_t ks_rb,
                           const uint8_t* candidates, int32_t* out, int32_t bsz, int32_t n, int32_t heads,
                           int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio, int32_t topk,
                           int32_t offset, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* dsv41_indexer_topk over MXFP4 query and keys (the layouts of dsv41_indexer_score_mxfp4):
 * bit-equal to dsv41_indexer_score_mxfp4 followed by dsv41_topk_select. Served shapes and the
 * workspace are dsv41_indexer_topk's (same size query). */
int dsv41_indexer_topk_mxfp4(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                             float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                             const uint8_t* k_scales, int64_t ks_bstride, const uint8_t* candidates,
                             int32_t* out, int32_t bsz, int32_t n, int32_t heads, int32_t dim, int32_t nb,
                             int32_t start_pos, int32_t ratio, int32_t topk, int32_t offset,
                             void* workspace, size_t workspace_bytes, hipStream_t stream);

/* dsv41_indexer_topk with an MXFP4 query against fp8 keys (the layouts of
 * dsv41_indexer_score_mxq_fp8): bit-equal to dsv41_indexer_score_mxq_fp8 followed by
 * dsv41_topk_select. Served shapes and the workspace are dsv41_indexer_topk's. */
int dsv41_indexer_topk_mxq_fp8(const uint8_t* q_codes, const uint8_t* q_scales, const void* w_raw,
                               float w_scale, const uint8_t* k_codes, int64_t kc_bstride,
                               const uint8_t* k_scales, int64_t ks_bstride, int32_t ks_rb,
                               const uint8_t* candidates, int32_t* out, int32_t bsz, int32_t n,
                               int32_t heads, int32_t dim, int32_t nb, int32_t start_pos, int32_t ratio,
                               int32_t topk, int32_t offset, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);

/* Top-k selection, deepseek_v41_mlx/indexer.py:140-144: per row of scores [bsz*n, nb],
 * the k = min(topk, nb) best positions (ties -> lowest position; -0.0 == +0.0), sorted
 * ascending, written as idx + offset when idx < lens else -1, lens = (start_pos+s+1)/ratio,
 * s = row % n. out [bsz*n, k] int32. nb <= 1<<22. */
int dsv41_topk_select(const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                      int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset,
                      hipStream_t stream);

/* The same selection with a caller-owned workspace (same reference function,
 * deepseek_v41_mlx/indexer.py:140-144; identical results): rows longer than 16384 scores with
 * k <= 2048 are then selected in two stages (each 4096-score chunk's best k, then the best k of
 * those lists), spreading a row over several workgroups. The workspace is
 * dsv41_topk_workspace_bytes(rows, nb, topk) bytes, 16-byte aligned (0: one stage, workspace
 * may be null). */
size_t dsv41_topk_workspace_bytes(int64_t rows, int32_t nb, int32_t topk);
int dsv41_topk_select_ws(const float* scores, int32_t* out, int64_t rows, int32_t n, int32_t nb,
                         int32_t topk, int32_t start_pos, int32_t ratio, int32_t offset,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* select_candidate_blocks, deepseek_v41_mlx/indexer.py:38-64: block maxima over blocks of
 * block_size (padded with -inf), the block holding position lens-1 pinned to +inf, the best
 * min(topk_blocks, n_blocks) blocks kept (ties -> lowest block) when their value is > -inf,
 * expanded back to positions. keep [bsz*n, nb] uint8 (1 = candidate). lens: optional device
 * int32 [n] of visible positions per query (NULL: (start_pos+s+1)/ratio). n_blocks <= 8192. */
int dsv41_candidate_blocks(const float* scores, uint8_t* keep, int64_t rows, int32_t n,
                           int32_t nb, int32_t topk_blocks, int32_t block_size,
                           const int32_t* lens, int32_t start_pos, int32_t ratio,
                           hipStream_t stream);

/* ---------------------------------------------------------------- sparse MLA --
 */

/* Scratch bytes the sparse-MLA entry points need for split partial results at this shape
 * (0 when no split is used). `rows_per_query` = window rows + index rows. */
size_t dsv41_sparse_mla_workspace_bytes(int32_t bsz, int32_t m, int32_t heads, int32_t dim,
                                        int32_t rows_per_query, int32_t dtype);

/* sparse_attn, deepseek_v41_mlx/sparse_attention.py:34-60 and the TileLang kernel wrapper
 * sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale), docs/reference/kernel.py:392-403:
 *   o[b,s,h] = sum_j e^{l_j - M} kv[b,idx_j] / (sum_j e^{l_j - M} + e^{sink_h - M}),
 *   l_j = scale * q[b,s,h].kv[b,idx_j] for idx_j >= 0 (others contribute nothing),
 *   M = max(max_j l_j, sink_h, -1e30); K = V; an all-masked row gives 0.
 * q, o [bsz,m,heads,dim]; kv [bsz,nkv,dim]; sink [heads] fp32; idx [bsz,m,k] int32
 * (indices >= nkv are treated as masked). dtype F32 or BF16 (q, kv and o alike). */
int dsv41_sparse_attn(const void* q, const void* kv, const float* sink, const int32_t* idx,
                      void* o, int32_t bsz, int32_t m, int32_t heads, int32_t dim, int32_t nkv,
                      int32_t k, float scale, int32_t dtype, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* The attention core of Attention.__call__, deepseek_v41_mlx/attention.py:124-175, reading
 * every KV source in place instead of concatenating them (attention.py:127, 165-168):
 *   unified position u < wp            -> window ring slot (start_pos - wp + u) % window
 *                   wp <= u < wp + n   -> chunk row u - wp              (this call's KV)
 *                   u >= wp + n        -> comp row u - wp - n < n_comp  (the source owner's cache)
 * with wp = min(start_pos, window). Query s sees the window positions
 * [max(wp+s-window+1, 0), wp+s] (window_idx_matrix, attention.py:40-50) plus idx[b,s,:]
 * (the indexer's output, already offset by wp + n; -1 masked; may be NULL with k = 0).
 * Output o [bsz,n,heads,dim] gets the inverse rope on its last rd channels at position
 * start_pos + s when rd > 0 (attention.py:174-175). q_rd > 0: q is wq_b's output before
 * its rope, and the launch applies the forward rope of attention.py:117 (rope_tail, inverse
 * false) to q's last q_rd channels as it loads q, at position start_pos + s, rounding each
 * rotated value to q's dtype as dsv41_rope_tail does (q itself is not written); q_rd = 0: q
 * arrives roped. cos_tab/sin_tab are [positions, w/2] for w = the nonzero of rd and q_rd (equal
 * when both are). win_kv [bsz,window,dim], chunk [bsz,n,dim], comp with comp_bstride elements
 * per batch row. dtype F32 or BF16. Every dsv41_sparse_mla_* form below takes rd and q_rd so. */
int dsv41_sparse_mla(const void* q, const void* win_kv, const void* chunk_kv,
                     const void* comp_kv, int64_t comp_bstride, int32_t n_comp,
                     const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz,
                     int32_t n, int32_t heads, int32_t dim, int32_t window, int32_t start_pos,
                     float scale, const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                     int32_t dtype, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* One-token decode form of dsv41_sparse_mla (n = 1) that also performs the ring write of
 * LayerCache.write_window, deepseek_v41_mlx/cache.py:61-67 (attention.py:131): chunk_kv's row
 * is stored into win_kv slot start_pos % window within the same launch. That slot holds
 * position start_pos - window, which has left the token's window, so the attention reads are
 * unaffected; the output equals dsv41_sparse_mla's and the ring equals what the separate
 * write produces. */
int dsv41_sparse_mla_decode(const void* q, void* win_kv, const void* chunk_kv,
                            const void* comp_kv, int64_t comp_bstride, int32_t n_comp,
                            const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz,
                            int32_t heads, int32_t dim, int32_t window, int32_t start_pos,
                            float scale, const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                            int32_t dtype, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* dsv41_sparse_mla_decode without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference: its sparse_attn allocates its output and scratch per call.
 * Same arguments, result and ring write as dsv41_sparse_mla_decode. The split partials live in a
 * static 32 MiB device array inside the library, one per GPU, held until the process ends; a
 * shape whose split scratch (dsv41_sparse_mla_workspace_bytes) exceeds 32 MiB returns
 * DSV41_E_WORKSPACE before any launch. Nothing is allocated or freed. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, no ordering between them)
 * race; calls ordered on one stream are safe (each call writes every partial it reads). */
int dsv41_sparse_mla_decode_noalloc(const void* q, void* win_kv, const void* chunk_kv,
                                    const void* comp_kv, int64_t comp_bstride, int32_t n_comp,
                                    const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz,
                                    int32_t heads, int32_t dim, int32_t window, int32_t start_pos,
                                    float scale, const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                                    int32_t dtype, hipStream_t stream);

/* dsv41_sparse_mla with the compressed source stored as fp8: the packed, lossless form of the
 * QAT values that attention.py:157-163 writes into the cache (e4m3 code times a power-of-two
 * block scale, the ue8m0 convention of fakequant.py:83-93). comp_kv holds e4m3fn bytes
 * [bsz, >=n_comp, 512] (comp_bstride bytes per batch row); comp_scale holds one ue8m0 byte
 * (scale 2^(e-127)) per 32 channels for every comp_scale_rb rows (1 or 32):
 * [bsz, ceil(n_comp / rb), 16] with comp_scale_bstride bytes per batch row. Rows are
 * dequantized to bf16 in-kernel, exactly (e4m3 x 2^k is bf16-representable), so the result
 * equals dsv41_sparse_mla's on the dequantized cache. q, win_kv, chunk_kv and o are bf16;
 * dim is 512; the workspace is sized by dsv41_sparse_mla_workspace_bytes(..., DSV41_BF16). */
int dsv41_sparse_mla_fp8(const void* q, const void* win_kv, const void* chunk_kv,
                         const uint8_t* comp_kv, int64_t comp_bstride, int32_t n_comp,
                         const uint8_t* comp_scale, int64_t comp_scale_bstride, int32_t comp_scale_rb,
                         const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz,
                         int32_t n, int32_t heads, int32_t dim, int32_t window, int32_t start_pos,
                         float scale, const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* dsv41_sparse_mla_fp8 for one token per row (n = 1) that also performs the ring write of
 * LayerCache.write_window, deepseek_v41_mlx/cache.py:61-67, as dsv41_sparse_mla_decode does. */
int dsv41_sparse_mla_fp8_decode(const void* q, void* win_kv, const void* chunk_kv,
                                const uint8_t* comp_kv, int64_t comp_bstride, int32_t n_comp,
                                const uint8_t* comp_scale, int64_t comp_scale_bstride,
                                int32_t comp_scale_rb, const float* sink, const int32_t* idx, int32_t k,
                                void* o, int32_t bsz, int32_t heads, int32_t dim, int32_t window,
                                int32_t start_pos, float scale, const float* cos_tab, const float* sin_tab,
                                int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* dsv41_sparse_mla with the compressed source in dsv41_comp_write_fp4's packed layout: 288-byte
 * rows (512 e2m1 codes, then 32 e4m3fn scales, one per 16 channels), comp_bstride bytes per
 * batch row (a multiple of 16). Rows are decoded to bf16 in-kernel, exactly (an e2m1 value times
 * an e4m3 value is bf16-representable), so the result equals dsv41_sparse_mla's on the decoded
 * cache -- the values the reference's bf16 cache holds after its fp4 QAT (attention.py:157-163).
 * q, win_kv, chunk_kv and o are bf16; dim is 512; the workspace is sized by
 * dsv41_sparse_mla_workspace_bytes(..., DSV41_BF16). */
int dsv41_sparse_mla_fp4(const void* q, const void* win_kv, const void* chunk_kv,
                         const uint8_t* comp_kv4, int64_t comp_bstride, int32_t n_comp, const float* sink,
                         const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n, int32_t heads,
                         int32_t dim, int32_t window, int32_t start_pos, float scale, const float* cos_tab,
                         const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* dsv41_sparse_mla_fp4 for one token per row (n = 1) that also performs the ring write of
 * LayerCache.write_window, deepseek_v41_mlx/cache.py:61-67, as dsv41_sparse_mla_decode does. */
int dsv41_sparse_mla_fp4_decode(const void* q, void* win_kv, const void* chunk_kv,
                                const uint8_t* comp_kv4, int64_t comp_bstride, int32_t n_comp,
                                const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz,
                                int32_t heads, int32_t dim, int32_t window, int32_t start_pos, float scale,
                                const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* dsv41_sparse_mla_fp4 with the window ring also packed: win_kv8 holds MXFP8 rows in
 * dsv41_window_write_mxfp8's layout (528 bytes at dim 512), ring_bstride bytes per batch row (> 0,
 * a multiple of 16). Both packed sources are decoded to bf16 in-kernel, exactly, so the result
 * equals dsv41_sparse_mla's on the decoded caches. comp_kv4 may be NULL with n_comp = 0 (a
 * window-only layer). */
int dsv41_sparse_mla_packed(const void* q, const uint8_t* win_kv8, int64_t ring_bstride,
                            const void* chunk_kv, const uint8_t* comp_kv4, int64_t comp_bstride, int32_t n_comp,
                            const float* sink, const int32_t* idx, int32_t k, void* o, int32_t bsz, int32_t n,
                            int32_t heads, int32_t dim, int32_t window, int32_t start_pos, float scale,
                            const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* dsv41_sparse_mla_packed for one token per row (n = 1) that also performs the ring write of
 * LayerCache.write_window (cache.py:61-67) into the MXFP8 ring, encoded as
 * dsv41_window_write_mxfp8 encodes it. */
int dsv41_sparse_mla_packed_decode(const void* q, uint8_t* win_kv8, int64_t ring_bstride,
                                   const void* chunk_kv, const uint8_t* comp_kv4, int64_t comp_bstride,
                                   int32_t n_comp, const float* sink, const int32_t* idx, int32_t k, void* o,
                                   int32_t bsz, int32_t heads, int32_t dim, int32_t window, int32_t start_pos,
                                   float scale, const float* cos_tab, const float* sin_tab, int32_t rd, int32_t q_rd,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The grouped block-diagonal output LoRA of Attention.__call__, deepseek_v41_mlx/attention.py:
 * 176-179 (DeepSeek's docs/reference/model.py:783-787): o viewed as [rows, groups, d], wo_a's
 * weight as [groups, r, d], einsum "bsgd,grd->bsgr" in fp32, cast to the activation dtype:
 *   out[m, g*r + j] = sum_k o[m, g*d + k] * wo_a[g*r + j, k].
 * o [rows, groups*d] (the attention output) and wo_a [groups*r, d] (nn.Linear's weight,
 * unquantized) in dtype (BF16 or F32); out [rows, groups*r] in out_dtype: BF16 (the fp32 sum
 * rounded to nearest even once, as astype does) or F32. Sums are fp32 in a fixed order:
 * deterministic, equal to the reference up to the order of fp32 additions (bf16 products are
 * exact). bf16 with d a multiple of 64 and r of 128 (the release's 4096 and 1024) runs on MFMA;
 * any other shape, and fp32, on a plain fp32 kernel. */
int dsv41_wo_a_grouped(const void* o, const void* wo_a, void* out, int32_t rows, int32_t groups,
                       int32_t d, int32_t r, int32_t dtype, int32_t out_dtype, hipStream_t stream);

/* The dense projections of Attention.__call__ at decode row counts, deepseek_v41_mlx/attention.py:
 * 114-116 and 179 (wq_a, wq_b, wkv and wo_b: nn.Linear, y = x @ w^T): x [rows, k] and the Linear
 * weight w [n, k] as they lie, bf16, y [rows, n] bf16 (fp32 sums rounded once). For rows <= 128
 * the weight is streamed once by the decode tile kernel of dsv41_wo_a_grouped, with the
 * contraction cut into `splits` ranges so that the workgroups fill the chip (n / 32 x splits; at
 * 33-64 rows n / 128 or n / 160 x splits when each range holds >= 1024 channels and that gives
 * 128-256); each
 * range's fp32 partial goes to `workspace` ([rows, splits * n] floats,
 * dsv41_linear_rows_workspace_bytes; none for splits == 1) and a second kernel sums them in
 * range order: deterministic, equal to the reference up to the order of fp32 additions.
 * k a multiple of 64 * splits, n of 32, splits <= 64. */
size_t dsv41_linear_rows_workspace_bytes(int32_t rows, int32_t n, int32_t splits);
int dsv41_linear_rows(const void* x, const void* w, void* y, void* workspace, size_t workspace_bytes,
                      int32_t rows, int32_t k, int32_t n, int32_t splits, int32_t dtype,
                      hipStream_t stream);

/* Two projections of the same rows in one launch, deepseek_v41_mlx/attention.py:114 and :116
 * (wq_a(x) and wkv(x)): y0 = x @ w0^T [rows, n0] and y1 = x @ w1^T [rows, n1], each weight as it
 * lies. The same arithmetic and order of additions as dsv41_linear_rows over the two weights
 * stacked, so each output equals that call's on its own weight when the split is the same.
 * splits >= 2; the workspace is dsv41_linear_rows_workspace_bytes(rows, n0 + n1, splits). */
int dsv41_linear_rows_pair(const void* x, const void* w0, const void* w1, void* y0, void* y1,
                           void* workspace, size_t workspace_bytes, int32_t rows, int32_t k, int32_t n0,
                           int32_t n1, int32_t splits, int32_t dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV41_H */
