"""CPU restatement of the deepseek_v41_mlx attention hot path -- TEST INFRASTRUCTURE ONLY.

This module is the oracle the HIP path is checked against. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the timed CPU baseline. The product path
(``dsv41``) never imports it and has no CPU fallback.

Everything is numpy float32 (int32 for indices). Tensors that the reference keeps
in bfloat16 are float32 arrays holding bf16-representable values; ``cast(x, dt)``
reproduces the reference's dtype conversions (round-to-nearest-even), so the
intermediate roundings happen at the same points as in the reference.

Each function cites the reference file:line it restates (paths relative to the
reference repository root).

Pinning status (what checks each function; see tests/test_oracle.py):
  * bf16/e4m3 rounding        -- torch's own casts over exhaustive grids (library routines)
  * e4m3 decode / fp8 cache   -- torch's float8_e4m3fn over all 256 codes; per-element loop
  * fp8_block_rows            -- rb = 1 equals fq_fp8_ue8m0 row by row; rb = 32: block openers
                                 equal fq_fp8_ue8m0, later rows torch's e4m3 cast at that scale
  * MXFP4 encode / decode     -- decode(encode(x)) == fq_fp4_ue8m0(x) bit for bit (signed zeros
                                 included) on the fake-quant known-answer inputs; every code's
                                 value against the e2m1 grid definition
  * fake-quants (a1-a3)       -- known-answer vectors (reference test inputs, rng 3 +
                                 midpoint vector) with answers from an independent
                                 brute-force nearest-grid search; closed-form scales
  * rope (a4)                 -- rotate then inverse-rotate = identity; complex multiply
  * RMSNorm (a5)              -- closed form, float64 recomputation
  * window index (a6)         -- brute-force position reconstruction
  * ring / caches (a7)        -- chronological read-back invariant
  * compressor (a8)           -- chunk-split invariance, ratio-1 reduction, float64 softmax pool
  * indexer scoring (a11)     -- float64 brute-force einsum, ReLU/sign special cases
  * candidate blocks (a12)    -- brute force over tiny inputs, pin and -inf-drop rules
  * top-k (a13)               -- brute-force python sort on (-score, index), adversarial ties
  * sparse attention (a14)    -- float64 brute force, closed forms (single index, sink -> -inf,
                                 all masked -> 0)
  * attention layer/stack     -- DeepSeek's torch Attention / Compressor / Indexer (the reference's
    (AttentionLayer,             docs/reference/model.py:429-789) run as an attention-only stack
     AttentionStack,             over the same weights: tests/golden/layer_golden.npz holds its
     publish_keys,               prefill and decode outputs, owner caches, the scores each index
     indexer_forward,            source ranks and its selection, for three topologies (ratio 4;
     index_weight_scale,         ratios 0/2/1 as released), fake-quant off and on; planted
     group_positions)            composition mistakes fail it. Plus decode == tail of prefill and
                                 chunked == single forward (the reference has no chunked path).
  * index_weight_scale in bf16 -- the rounding of the python scalar to the activation dtype follows
                                 MLX's weak scalar typing (an array's dtype wins); the fixtures run
                                 in float32, where the scale is exact, so the bf16 rounding of the
                                 scalar itself is "parity unpinned".
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32
NEG_INF = F32(-np.inf)
POS_INF = F32(np.inf)
FP8_MAX = F32(448.0)
FP4_MAX = F32(6.0)
FP8_MAX_INV = F32(1.0 / 448.0)
FP4_MAX_INV = F32(1.0 / 6.0)

# ---------------------------------------------------------------------------
# dtype emulation
# ---------------------------------------------------------------------------


def to_bf16(x) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even); returns float32 values."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    out = r.view(F32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out


def cast(x, dtype: str) -> np.ndarray:
    """The reference's ``.astype(dtype)`` for dtype in {"f32", "bf16"}."""
    x = np.asarray(x, dtype=F32)
    if dtype == "f32":
        return x
    if dtype == "bf16":
        return to_bf16(x)
    raise ValueError(f"unknown dtype {dtype}")


def e4m3_round(x) -> np.ndarray:
    """Round float32 to the nearest OCP e4m3fn value, ties to even (torch's
    ``float8_e4m3fn`` cast, which the reference's test pins against MLX's
    ``to_fp8`` -- tests/test_parity.py:333-337). Inputs are expected within
    +-448 (every caller clips first); returns float32."""
    x = np.ascontiguousarray(x, dtype=F32)
    a = np.abs(x)
    u = a.view(np.uint32).astype(np.uint64)
    # normal range: keep 3 mantissa bits, round to nearest even at bit 20
    r = ((u + 0x7FFFF + ((u >> 20) & 1)) & ~np.uint64(0xFFFFF)).astype(np.uint32).view(F32)
    # subnormal range (|x| < 2^-6): fixed quantum 2^-9
    sub = (np.rint(a * F32(512.0)) / F32(512.0)).astype(F32)
    res = np.where(a < F32(2.0 ** -6), sub, r).astype(F32)
    return np.copysign(res, x).astype(F32)


# ---------------------------------------------------------------------------
# fake-quantization (QAT simulation) -- deepseek_v41_mlx/fakequant.py
# ---------------------------------------------------------------------------

DISABLE_FAKE_QUANT = False

_E2M1_LUT = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=F32)


def e4m3_decode(codes) -> np.ndarray:
    """float32 values of e4m3fn codes (uint8): sign, 4-bit exponent (bias 7), 3-bit mantissa;
    exponent 0 is subnormal (m * 2^-9); 0x7F / 0xFF are NaN. The byte form of the values
    e4m3_round produces (the fp8 QAT of fakequant.py:83-93 stores exactly these)."""
    c = np.asarray(codes, np.uint8).astype(np.int32)
    s, e, m = (c >> 7) & 1, (c >> 3) & 15, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(s == 1, -v, v).astype(F32)


def e4m3_encode(q) -> np.ndarray:
    """e4m3fn codes (uint8) of float32 values already on the e4m3 grid (|q| <= 448): the inverse
    of e4m3_decode on finite values."""
    q = np.ascontiguousarray(q, dtype=F32)
    a = np.abs(q)
    u = a.view(np.uint32)
    e = ((u >> 23) & 0xFF).astype(np.int32) - 127 + 7
    normal = (e << 3) | ((u >> 20) & 7).astype(np.int32)
    sub = np.rint(a * F32(512.0)).astype(np.int32)
    c = np.where(a < F32(2.0 ** -6), sub, normal) | (np.signbit(q).astype(np.int32) << 7)
    return c.astype(np.uint8)


def dequant_fp8_cache(codes, scales, rb: int) -> np.ndarray:
    """An fp8 cache [b, rows, D] of e4m3 codes with ue8m0 block scales [b, ceil(rows/rb), D/32]
    (scale 2^(e-127) for every rb rows x 32 channels) -> float32 values."""
    v = e4m3_decode(codes)
    b, rows, d = v.shape
    sc = np.ldexp(np.ones(np.shape(scales), F32), np.asarray(scales, np.int32) - 127).astype(F32)
    sc_rows = np.repeat(sc, rb, axis=1)[:, :rows]
    return (v * np.repeat(sc_rows, 32, axis=2)).astype(F32)


def pow2_ceil_log2(r) -> np.ndarray:
    """2**ceil(log2(r)) from IEEE bits (fakequant.py:47-62; kernel.py:22-37)."""
    r = np.ascontiguousarray(r, dtype=F32)
    bits = r.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFF) != 0)
    return ((e + 127) << 23).astype(np.uint32).view(F32)


def e2m1_round(v) -> np.ndarray:
    """Nearest e2m1 magnitude with the reference's tie table (fakequant.py:65-73):
    ties at .25/1.25/2.5/5 round down, at .75/1.75/3.5 round up; sign kept."""
    v = np.asarray(v, dtype=F32)
    mag = np.abs(v)
    idx = np.zeros(mag.shape, dtype=np.int32)
    for t in (0.25, 1.25, 2.5, 5.0):
        idx += (mag > F32(t))
    for t in (0.75, 1.75, 3.5):
        idx += (mag >= F32(t))
    return np.copysign(_E2M1_LUT[idx], v).astype(F32)


def _blockify(x, block):
    n = x.shape[-1]
    if n % block:
        raise ValueError(f"last dim {n} not divisible by block {block}")
    return np.asarray(x, dtype=F32).reshape(*x.shape[:-1], n // block, block)


def fq_fp8_ue8m0(x, block: int = 32, dtype: str = "f32") -> np.ndarray:
    """fake_quant_fp8_ue8m0 (fakequant.py:83-93; act_quant inplace, kernel.py:40-124)."""
    if DISABLE_FAKE_QUANT:
        return cast(x, dtype)
    shape = x.shape
    xb = _blockify(x, block)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(1e-4))
    s = pow2_ceil_log2(amax * FP8_MAX_INV)
    q = e4m3_round(np.clip(xb / s, -FP8_MAX, FP8_MAX)) * s
    return cast(q.reshape(shape), dtype)


def fp8_block_rows(x, row0: int, rb: int, scales_in=None):
    """The fp8 cache variant's stored values when one ue8m0 scale covers 32 channels of every rb
    rows (rb = 1: fq_fp8_ue8m0 per row; rb = 32: 32 x 32 blocks). x [b, g, d] are the values
    written at cache rows row0 .. row0+g-1. A row that opens a block (row % rb == 0) sets the
    block's scale by fake_quant_fp8_ue8m0's formula (fakequant.py:83-93); the block's later rows
    are rounded with it: e4m3(clip(v / s, +-448)) * s. scales_in [b, blocks, d/32] holds the
    scales of blocks opened before row0 (as powers of two). Returns (values, block scales)."""
    x = np.asarray(x, F32)
    b, g, d = x.shape
    nblk = -(-(row0 + g) // rb)
    sc = np.zeros((b, nblk, d // 32), F32)
    if scales_in is not None:
        prev = np.asarray(scales_in, F32)[:, :nblk]
        sc[:, :prev.shape[1]] = prev
    out = np.empty_like(x)
    for j in range(g):
        r = row0 + j
        xb = _blockify(x[:, j], 32)                                   # [b, d/32, 32]
        if r % rb == 0:
            amax = np.maximum(np.abs(xb).max(axis=-1), F32(1e-4))
            sc[:, r // rb] = pow2_ceil_log2(amax * FP8_MAX_INV)
        s = sc[:, r // rb][..., None]
        out[:, j] = (e4m3_round(np.clip(xb / s, -FP8_MAX, FP8_MAX)) * s).reshape(b, d)
    return out, sc


def fq_fp4_ue8m0(x, block: int = 32, dtype: str = "f32") -> np.ndarray:
    """fake_quant_fp4_ue8m0 (fakequant.py:96-106; fp4_act_quant e8m0, kernel.py:127-204)."""
    if DISABLE_FAKE_QUANT:
        return cast(x, dtype)
    shape = x.shape
    xb = _blockify(x, block)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(6.0 * 2.0 ** -126))
    s = pow2_ceil_log2(amax * FP4_MAX_INV)
    q = e2m1_round(np.clip(xb / s, -FP4_MAX, FP4_MAX)) * s
    return cast(q.reshape(shape), dtype)


def mxfp4_encode(x):
    """MXFP4 form of fake_quant_fp4_ue8m0(x, 32) over the last dim (d % 32 == 0): the block
    scale s of fakequant.py:96-106 as a ue8m0 byte (log2(s) + 127) and each x/s rounded by
    e2m1_round as a 4-bit code (sign in bit 3, magnitude index into 0, .5, 1, 1.5, 2, 3, 4, 6),
    two per byte, the even channel in the low nibble. Returns (codes [..., d/2], scales
    [..., d/32]) uint8."""
    xb = _blockify(x, 32)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(6.0 * 2.0 ** -126))
    s = pow2_ceil_log2(amax * FP4_MAX_INV)
    r = e2m1_round(np.clip(xb / s, -FP4_MAX, FP4_MAX))
    mag = np.searchsorted(_E2M1_LUT, np.abs(r)).astype(np.uint8)          # exact grid values
    code = mag | (np.signbit(r).astype(np.uint8) << 3)
    code = code.reshape(*np.shape(x)[:-1], -1)
    codes = (code[..., 0::2] | (code[..., 1::2] << 4)).astype(np.uint8)
    scales = ((s.view(np.uint32) >> 23) & 0xFF).astype(np.uint8)[..., 0]
    return codes, scales


def mxfp4_decode(codes, scales) -> np.ndarray:
    """float32 values of an MXFP4 encoding (mxfp4_encode's layout): e2m1(code) * 2^(scale-127)."""
    c = np.asarray(codes, np.uint8)
    nib = np.stack([c & 15, c >> 4], axis=-1).reshape(*c.shape[:-1], -1)
    v = _E2M1_LUT[nib & 7] * np.where(nib & 8, F32(-1.0), F32(1.0))
    sc = np.ldexp(np.ones(np.shape(scales), F32), np.asarray(scales, np.int32) - 127).astype(F32)
    return (v * np.repeat(sc, 32, axis=-1)).astype(F32)


def fq_fp4_e4m3(x, block: int = 16, dtype: str = "f32") -> np.ndarray:
    """fake_quant_fp4_e4m3 (fakequant.py:109-119; fp4_act_quant e4m3 scale, kernel.py:160-163)."""
    if DISABLE_FAKE_QUANT:
        return cast(x, dtype)
    shape = x.shape
    xb = _blockify(x, block)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(6.0 * 2.0 ** -9))
    s = e4m3_round((amax / FP4_MAX).astype(F32))
    q = e2m1_round(np.clip(xb / s, -FP4_MAX, FP4_MAX)) * s
    return cast(q.reshape(shape), dtype)


def mxfp8_encode(x):
    """MXFP8 rows of fake_quant_fp8_ue8m0(x, 32) over the last dim (fakequant.py:83-93): d
    e4m3fn codes of x / s, then the d/32 block scales s as ue8m0 bytes (log2(s) + 127).
    Returns uint8 [..., d + d/32]."""
    xb = _blockify(x, 32)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(1e-4))
    s = pow2_ceil_log2(amax * FP8_MAX_INV)
    q = e4m3_round(np.clip(xb / s, -FP8_MAX, FP8_MAX))
    codes = e4m3_encode(q).reshape(*np.shape(x)[:-1], -1)
    scales = ((s.view(np.uint32) >> 23) & 0xFF).astype(np.uint8)[..., 0]
    return np.concatenate([codes, scales], axis=-1)


def mxfp8_decode(rows) -> np.ndarray:
    """float32 values of mxfp8_encode's rows: e4m3(code) * 2^(scale - 127) per 32 channels."""
    rows = np.asarray(rows, np.uint8)
    d = rows.shape[-1] * 32 // 33
    sc = np.ldexp(np.ones(rows[..., d:].shape, F32), rows[..., d:].astype(np.int32) - 127).astype(F32)
    return (e4m3_decode(rows[..., :d]) * np.repeat(sc, 32, axis=-1)).astype(F32)


def fp4_e4m3_encode(x, block: int = 16):
    """Packed form of fake_quant_fp4_e4m3(x, block) over the last dim (fakequant.py:109-119):
    per row d/2 bytes of e2m1 codes (the rounding of fq_fp4_e4m3 as a 4-bit code, sign in bit 3,
    two per byte, the even channel in the low nibble), then one e4m3fn byte per block holding
    the block scale s = e4m3_round(max(amax, 6 * 2^-9) / 6). Returns uint8 [..., d/2 + d/block]."""
    xb = _blockify(x, block)
    amax = np.maximum(np.abs(xb).max(axis=-1, keepdims=True), F32(6.0 * 2.0 ** -9))
    s = e4m3_round((amax / FP4_MAX).astype(F32))
    r = e2m1_round(np.clip(xb / s, -FP4_MAX, FP4_MAX))
    mag = np.searchsorted(_E2M1_LUT, np.abs(r)).astype(np.uint8)
    code = (mag | (np.signbit(r).astype(np.uint8) << 3)).reshape(*np.shape(x)[:-1], -1)
    codes = (code[..., 0::2] | (code[..., 1::2] << 4)).astype(np.uint8)
    return np.concatenate([codes, e4m3_encode(s[..., 0])], axis=-1)


def fp4_e4m3_decode(rows, block: int = 16) -> np.ndarray:
    """float32 values of fp4_e4m3_encode's rows: e2m1(code) * e4m3(scale byte of the block)."""
    rows = np.asarray(rows, np.uint8)
    d = (rows.shape[-1] * 2 * block) // (block + 2)
    c = rows[..., :d // 2]
    nib = np.stack([c & 15, c >> 4], axis=-1).reshape(*c.shape[:-1], -1)
    v = _E2M1_LUT[nib & 7] * np.where(nib & 8, F32(-1.0), F32(1.0))
    sc = e4m3_decode(rows[..., d // 2:])
    return (v * np.repeat(sc, block, axis=-1)).astype(F32)


# ---------------------------------------------------------------------------
# layers -- deepseek_v41_mlx/layers.py
# ---------------------------------------------------------------------------


def rmsnorm(x, weight, eps: float = 1e-20, dtype: str = "f32") -> np.ndarray:
    """RMSNorm in fp32, cast back (layers.py:20-33)."""
    xf = np.asarray(x, dtype=F32)
    var = np.mean(np.square(xf), axis=-1, keepdims=True, dtype=F32)
    xf = xf * (F32(1.0) / np.sqrt(var + F32(eps)))
    return cast(np.asarray(weight, F32) * xf, dtype)


def yarn_freqs(dim: int, original_seq_len: int, base: float, factor: float,
               beta_fast: int, beta_slow: int) -> np.ndarray:
    """The YaRN-ramped inverse frequencies of precompute_freqs_cis (layers.py:36-52)."""
    def corrected_dim(rotations):
        return dim * math.log(original_seq_len / (rotations * 2 * math.pi)) / (2 * math.log(base))

    freqs = (F32(1.0) / (F32(base) ** (np.arange(0, dim, 2, dtype=F32) / F32(dim)))).astype(F32)
    if original_seq_len > 0:
        low = max(math.floor(corrected_dim(beta_fast)), 0)
        high = min(math.ceil(corrected_dim(beta_slow)), dim - 1)
        ramp = np.clip((np.arange(dim // 2, dtype=F32) - F32(low)) / F32(max(high - low, 1e-3)),
                       F32(0), F32(1)).astype(F32)
        smooth = (F32(1) - ramp).astype(F32)
        freqs = (freqs / F32(factor) * (F32(1) - smooth) + freqs * smooth).astype(F32)
    return freqs


def precompute_freqs_cis(dim: int, seqlen: int, original_seq_len: int, base: float,
                         factor: float, beta_fast: int, beta_slow: int):
    """(cos, sin) tables [seqlen, dim//2] (layers.py:36-56)."""
    freqs = yarn_freqs(dim, original_seq_len, base, factor, beta_fast, beta_slow)
    ang = (np.arange(seqlen, dtype=F32)[:, None] * freqs[None, :]).astype(F32)
    return np.cos(ang).astype(F32), np.sin(ang).astype(F32)


def apply_rotary_emb(x, cos, sin, inverse: bool = False, dtype: str = "f32") -> np.ndarray:
    """Adjacent-pair complex rotation (layers.py:59-79). cos/sin [s, d/2]; x [b,s,d] or [b,s,h,d]."""
    xf = np.asarray(x, dtype=F32)
    shape = xf.shape
    xp = xf.reshape(*shape[:-1], shape[-1] // 2, 2)
    xr, xi = xp[..., 0], xp[..., 1]
    if xr.ndim == 4:
        c, s = cos[None, :, None, :], sin[None, :, None, :]
    else:
        c, s = cos[None, :, :], sin[None, :, :]
    if inverse:
        s = -s
    out = np.stack([xr * c - xi * s, xr * s + xi * c], axis=-1).astype(F32)
    return cast(out.reshape(shape), dtype)


def rope_tail(x, rd: int, cos, sin, inverse: bool = False, dtype: str = "f32") -> np.ndarray:
    """Rope on the last rd channels only (layers.py:82-84)."""
    x = np.asarray(x, dtype=F32)
    return np.concatenate([x[..., :-rd], apply_rotary_emb(x[..., -rd:], cos, sin, inverse, dtype)],
                          axis=-1)


# ---------------------------------------------------------------------------
# sparse attention -- deepseek_v41_mlx/sparse_attention.py
# ---------------------------------------------------------------------------

ATTN_NEG = F32(-1e30)


def sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale: float, chunk: int = 256,
                dtype: str = "f32") -> np.ndarray:
    """Gathered sparse MLA, K = V, sink in the denominator only (sparse_attention.py:25-60).

    q [b,m,h,d], kv [b,n,d], attn_sink [h], topk_idxs [b,m,k] int (-1 = masked).
    """
    q = np.asarray(q, F32)
    kv = np.asarray(kv, F32)
    idx_all = np.asarray(topk_idxs)
    b, m, h, d = q.shape
    sink = np.asarray(attn_sink, F32).reshape(1, 1, h, 1)
    scale = F32(softmax_scale)
    outs = []
    bidx = np.arange(b)[:, None, None]
    for start in range(0, m, chunk):
        stop = min(start + chunk, m)
        qc = q[:, start:stop]
        ic = idx_all[:, start:stop]
        kvc = kv[bidx, np.maximum(ic, 0)]                                  # [b, c, k, d]
        logits = np.matmul(qc, np.swapaxes(kvc, -1, -2)) * scale           # [b, c, h, k]
        valid = (ic >= 0)[:, :, None, :]
        logits = np.where(valid, logits, ATTN_NEG)
        mmax = logits.max(axis=-1, keepdims=True)
        mmax = np.maximum(np.maximum(mmax, sink), ATTN_NEG)
        w = np.exp(logits - mmax).astype(F32)
        w = np.where(valid, w, F32(0)).astype(F32)
        denom = w.sum(axis=-1, keepdims=True, dtype=F32) + np.exp(sink - mmax).astype(F32)
        o = np.matmul(w, kvc) / denom
        outs.append(cast(o, dtype))
    return np.concatenate(outs, axis=1)


# ---------------------------------------------------------------------------
# indexer -- deepseek_v41_mlx/indexer.py
# ---------------------------------------------------------------------------


def query_lens(start_pos: int, n: int, ratio: int) -> np.ndarray:
    """Visible compressed entries per query, (start_pos+s+1)//ratio (indexer.py:129-131)."""
    return ((start_pos + np.arange(n) + 1) // ratio).astype(np.int64)


def indexer_scores(q, index_k, w, start_pos: int, ratio: int, candidates=None) -> np.ndarray:
    """fp32 scores S[b,s,t] = sum_h relu(q.k) * w, visibility and candidate masks
    (indexer.py:123-138). q [b,n,hi,di], index_k [b,nb,di], w [b,n,hi] fp32."""
    q = np.asarray(q, F32)
    k = np.asarray(index_k, F32)
    w = np.asarray(w, F32)
    b, n, hi, di = q.shape
    nb = k.shape[1]
    dots = np.matmul(q, np.swapaxes(k, 1, 2)[:, None])                  # [b, n, hi, nb]
    scores = (np.maximum(dots, F32(0)) * w[..., None]).sum(axis=2, dtype=F32)
    lens = query_lens(start_pos, n, ratio)[:, None]
    vis = np.arange(nb)[None, :] < lens
    scores = np.where(vis[None], scores, NEG_INF).astype(F32)
    if candidates is not None:
        scores = np.where(candidates, scores, NEG_INF).astype(F32)
    return scores


def _canon(scores) -> np.ndarray:
    """-0.0 compares equal to +0.0, so both sort as one tie class."""
    s = np.asarray(scores, F32)
    return np.where(s == 0, F32(0.0), s).astype(F32)


def topk_order(scores, k: int) -> np.ndarray:
    """Positions of the k best scores, ties to the lowest index (the tie rule the
    reference leaves open -- tests/test_parity.py:17-21 -- fixed to lowest index)."""
    s = _canon(scores)
    return np.argsort(-s, axis=-1, kind="stable")[..., :k]


def topk_indices(scores, index_topk: int, lens, offset: int) -> np.ndarray:
    """Top-k, ascending position order, -1 past lens, + offset (indexer.py:140-144).

    scores [b,n,nb]; lens [n] (per query)."""
    nb = scores.shape[-1]
    k = min(index_topk, nb)
    idx = np.sort(topk_order(scores, k), axis=-1).astype(np.int64)
    lens = np.asarray(lens).reshape(1, -1, 1)
    return np.where(idx < lens, idx + offset, -1).astype(np.int32)


def select_candidate_blocks(scores, lens, topk_blocks: int, block_size: int) -> np.ndarray:
    """Level one of the two-level top-k (indexer.py:38-64). scores [b,n,nb], lens [n]."""
    scores = np.asarray(scores, F32)
    width = scores.shape[-1]
    pad = (-width) % block_size
    if pad:
        scores = np.concatenate(
            [scores, np.full((*scores.shape[:-1], pad), NEG_INF, F32)], axis=-1)
    blocks = scores.reshape(*scores.shape[:-1], -1, block_size).max(axis=-1)
    nbk = blocks.shape[-1]
    last = (np.asarray(lens, np.int64).reshape(-1, 1) - 1) // block_size       # floor division
    pin = np.arange(nbk)[None, :] == last
    blocks = np.where(pin[None], POS_INF, blocks).astype(F32)
    k = min(topk_blocks, nbk)
    top = topk_order(blocks, k)
    top_val = np.take_along_axis(blocks, top, axis=-1)
    keep = np.zeros(blocks.shape, dtype=bool)
    np.put_along_axis(keep, top, top_val > NEG_INF, axis=-1)
    return np.repeat(keep, block_size, axis=-1)[..., :width]


# ---------------------------------------------------------------------------
# window index matrix -- deepseek_v41_mlx/attention.py:40-50
# ---------------------------------------------------------------------------


def window_idx_matrix(wp: int, n: int, window: int) -> np.ndarray:
    """[n, W_eff] indices into concat(prev_window(wp), chunk(n)), -1 pads."""
    w_eff = min(window, wp + n)
    end = np.arange(n) + wp
    start = np.maximum(end - window + 1, 0)
    idx = start[:, None] + np.arange(w_eff)[None, :]
    return np.where(idx > end[:, None], -1, idx).astype(np.int32)


# ---------------------------------------------------------------------------
# config topology -- deepseek_v41_mlx/config.py:104-133
# ---------------------------------------------------------------------------


class Args:
    """The ModelArgs fields the attention path reads (config.py:35-82)."""

    def __init__(self, **kw):
        self.dim = 5120
        self.n_layers = 40
        self.n_heads = 64
        self.head_dim = 512
        self.rope_head_dim = 64
        self.q_lora_rank = 1280
        self.o_lora_rank = 1024
        self.o_groups = 8
        self.window_size = 128
        self.norm_eps = 1e-20
        self.compress_ratios = ()
        self.kv_source_layers = ()
        self.index_source_layers = ()
        self.compress_rope_theta = 160000.0
        self.candidate_source_layer = -1
        self.candidate_topk_blocks = 0
        self.candidate_block_size = 0
        self.original_seq_len = 65536
        self.rope_theta = 10000.0
        self.rope_factor = 16.0
        self.beta_fast = 32
        self.beta_slow = 1
        self.max_seq_len = 1048576
        self.index_n_heads = 32
        self.index_head_dim = 128
        self.index_topk = 512
        for k, v in kw.items():
            if not hasattr(self, k):
                raise TypeError(f"unknown arg {k}")
            setattr(self, k, v)

    def compress_ratio(self, layer_id: int) -> int:
        return int(self.compress_ratios[layer_id]) if layer_id < len(self.compress_ratios) else 0


# ---------------------------------------------------------------------------
# caches -- deepseek_v41_mlx/cache.py, compressor.py:82-88
# ---------------------------------------------------------------------------


class CompressorState:
    def __init__(self, bsz, ratio, head_dim):
        self.kv_state = np.zeros((bsz, ratio, head_dim), F32)
        self.score_state = np.full((bsz, ratio, head_dim), NEG_INF, F32)


class LayerCache:
    """cache.py:27-67. Consumers hold references to the owner's buffers."""

    def __init__(self, bsz, args: Args, layer_id, max_seq_len, dtype="f32"):
        self.window = args.window_size
        self.ratio = args.compress_ratio(layer_id)
        self.is_kv_source = layer_id in args.kv_source_layers
        self.dtype = dtype
        self.win_kv = np.zeros((bsz, self.window, args.head_dim), F32)
        self.comp_kv = None
        self.comp_state = None
        self.index_k = None
        if self.is_kv_source:
            n_comp = max_seq_len // self.ratio
            self.comp_kv = np.zeros((bsz, n_comp, args.head_dim), F32)
            if self.ratio > 1:
                self.comp_state = CompressorState(bsz, self.ratio, args.head_dim)
            if layer_id in args.index_source_layers:
                self.index_k = np.zeros((bsz, n_comp, args.index_head_dim), F32)

    def window_chrono(self, pos):
        w = self.window
        wp = min(pos, w)
        if wp == 0:
            return self.win_kv[:, :0]
        slots = (pos - wp + np.arange(wp)) % w
        return self.win_kv[:, slots]

    def write_window(self, pos, kv):
        n = kv.shape[1]
        keep = min(n, self.window)
        slots = (pos + n - keep + np.arange(keep)) % self.window
        self.win_kv[:, slots] = cast(kv[:, n - keep:], self.dtype)


class ModelCache:
    def __init__(self, args: Args, bsz=1, max_seq_len=None, dtype="f32"):
        self.max_seq_len = max_seq_len or min(args.max_seq_len, 4096)
        self.offset = 0
        self.layers = [LayerCache(bsz, args, i, self.max_seq_len, dtype)
                       for i in range(args.n_layers)]


class SharedState:
    """model.py:35-44."""

    def __init__(self):
        self.kv_src_cache = None
        self.index_src_cache = None
        self.topk_idxs = None
        self.candidates = None


# ---------------------------------------------------------------------------
# compressor -- deepseek_v41_mlx/compressor.py:46-79
# ---------------------------------------------------------------------------


def softmax(x, axis):
    x = np.asarray(x, F32)
    e = np.exp(x - x.max(axis=axis, keepdims=True)).astype(F32)
    return (e / e.sum(axis=axis, keepdims=True, dtype=F32)).astype(F32)


def compressor_pool(kv, score, start_pos, state: CompressorState, ratio, norm_w, eps, dtype):
    """The ratio>1 body after the two fp32 projections: carry-in, group, softmax pool,
    carry-out, norm (compressor.py:58-79). kv/score [b,n,d] fp32. Returns latents or None."""
    bsz, n, _ = kv.shape
    kv = np.asarray(kv, F32)
    score = np.asarray(score, F32)
    m = start_pos % ratio
    if m:
        kv = np.concatenate([state.kv_state[:bsz, :m], kv], axis=1)
        score = np.concatenate([state.score_state[:bsz, :m], score], axis=1)
    total = m + n
    g = total // ratio
    rem = total % ratio
    if rem:
        state.kv_state[:bsz, :rem] = kv[:, total - rem:]
        state.score_state[:bsz, :rem] = score[:, total - rem:]
        kv, score = kv[:, :total - rem], score[:, :total - rem]
    if g == 0:
        return None
    kv = kv.reshape(bsz, g, ratio, -1)
    score = score.reshape(bsz, g, ratio, -1)
    pooled = (kv * softmax(score, axis=2)).sum(axis=2, dtype=F32)
    return rmsnorm(cast(pooled, dtype), norm_w, eps, dtype)


def linear(x, w, dtype):
    """nn.Linear without bias in the activation dtype: fp32 accumulate, cast out."""
    return cast(np.matmul(np.asarray(x, F32), np.asarray(w, F32).T), dtype)


def compressor_forward(x, start_pos, state, p, ratio, eps, dtype):
    """Compressor.__call__ (compressor.py:46-79). p: dict with wkv, wgate, norm."""
    if ratio == 1:
        return rmsnorm(linear(x, p["wkv"], dtype), p["norm"], eps, dtype)
    xf = np.asarray(x, F32)
    kv = np.matmul(xf, np.asarray(p["wkv"], F32).T).astype(F32)
    score = np.matmul(xf, np.asarray(p["wgate"], F32).T).astype(F32)
    return compressor_pool(kv, score, start_pos, state, ratio, p["norm"], eps, dtype)


# ---------------------------------------------------------------------------
# indexer key publish + scoring -- deepseek_v41_mlx/indexer.py:89-144
# ---------------------------------------------------------------------------


def group_positions(g0: int, g: int, ratio: int) -> np.ndarray:
    """Rope positions of compressed groups g0 .. g0+g-1: a latent stands for the first token of
    its group, so group j rotates at position j * ratio (attention.py:157-161, indexer.py:100-102)."""
    return (g0 + np.arange(g)) * ratio


def publish_keys(latents, start_pos, ratio, rd, cos, sin, p, eps, dtype, cache: LayerCache):
    """Indexer.publish_keys (indexer.py:89-104)."""
    g0 = start_pos // ratio
    g = latents.shape[1]
    pos = group_positions(g0, g, ratio)
    k = rmsnorm(linear(latents, p["wk"], dtype), p["k_norm"], eps, dtype)
    k = rope_tail(k, rd, cos[pos], sin[pos], dtype=dtype)
    k = fq_fp4_ue8m0(k, 32, dtype)
    cache.index_k[:k.shape[0], g0:g0 + g] = cast(k, cache.dtype)


def index_weight_scale(hi: int, di: int, dtype: str) -> np.float32:
    """softmax_scale * n_heads**-0.5 as the activation dtype sees it: an MLX python
    scalar takes the array's dtype (indexer.py:123)."""
    return cast(np.array([di ** -0.5 * hi ** -0.5], F32), dtype)[0]


def indexer_forward(x, qr, start_pos, offset, cos, sin, index_k, shared, p, a: Args,
                    layer_flags, dtype):
    """Indexer.__call__ (indexer.py:106-144). layer_flags: (ratio, is_candidate_source,
    uses_candidates)."""
    ratio, is_cand_src, uses_cand = layer_flags
    bsz, n, _ = x.shape
    hi, di, rd = a.index_n_heads, a.index_head_dim, a.rope_head_dim
    nb = index_k.shape[1]
    q = linear(qr, p["wq_b"], dtype).reshape(bsz, n, hi, di)
    q = rope_tail(q, rd, cos[start_pos:start_pos + n], sin[start_pos:start_pos + n], dtype=dtype)
    q = fq_fp4_ue8m0(q, 32, dtype)
    w = cast(linear(x, p["weights_proj"], dtype) * index_weight_scale(hi, di, dtype), dtype)
    scores = indexer_scores(q, cast(index_k, "f32"), w, start_pos, ratio)
    lens = query_lens(start_pos, n, ratio)
    if is_cand_src:
        shared.candidates = select_candidate_blocks(scores, lens, a.candidate_topk_blocks,
                                                    a.candidate_block_size)
    elif uses_cand and shared.candidates is not None:
        scores = np.where(shared.candidates, scores, NEG_INF).astype(F32)
    return topk_indices(scores, a.index_topk, lens, offset)


# ---------------------------------------------------------------------------
# attention layer -- deepseek_v41_mlx/attention.py:53-179
# ---------------------------------------------------------------------------


class AttentionLayer:
    """Attention.__call__ restated over numpy weights (attention.py:106-179).

    params: wq_a [q_lora, dim], q_norm [q_lora], wq_b [H*D, q_lora], wkv [D, dim],
    kv_norm [D], wo_a [G*o_lora, H*D/G], wo_b [dim, G*o_lora], attn_sink [H],
    compressor {wkv, wgate?, norm}, indexer {wq_b, weights_proj, wk?, k_norm?}.
    """

    def __init__(self, layer_id: int, a: Args, params: dict, dtype: str = "f32"):
        self.layer_id = layer_id
        self.a = a
        self.p = params
        self.dtype = dtype
        self.ratio = a.compress_ratio(layer_id)
        self.is_kv_source = layer_id in a.kv_source_layers
        self.is_index_source = layer_id in a.index_source_layers
        self.owns_k = self.is_index_source and self.is_kv_source
        self.is_candidate_source = layer_id == a.candidate_source_layer
        self.uses_candidates = 0 <= a.candidate_source_layer < layer_id
        if self.ratio:
            orig_len, theta = a.original_seq_len, a.compress_rope_theta
        else:
            orig_len, theta = 0, a.rope_theta
        self.rope = (a.rope_head_dim, orig_len, theta, a.rope_factor, a.beta_fast, a.beta_slow)
        self.break_rope_inverse = False
        self.break_sink = False

    def freqs(self, upto):
        rd, orig_len, theta, factor, bf, bs = self.rope
        return precompute_freqs_cis(rd, max(upto, 64), orig_len, theta, factor, bf, bs)

    def __call__(self, x, start_pos, cache: ModelCache, shared: SharedState):
        a, p, dt = self.a, self.p, self.dtype
        bsz, n, _ = x.shape
        H, D, rd = a.n_heads, a.head_dim, a.rope_head_dim
        eps = a.norm_eps
        end_pos = start_pos + n
        cos, sin = self.freqs(end_pos)
        c_q, s_q = cos[start_pos:end_pos], sin[start_pos:end_pos]

        qr = rmsnorm(linear(x, p["wq_a"], dt), p["q_norm"], eps, dt)
        q = linear(qr, p["wq_b"], dt).reshape(bsz, n, H, D)
        q = rope_tail(q, rd, c_q, s_q, dtype=dt)

        kv = rmsnorm(linear(x, p["wkv"], dt), p["kv_norm"], eps, dt)
        kv = rope_tail(kv, rd, c_q, s_q, dtype=dt)
        kv = fq_fp8_ue8m0(kv, 32, dt)

        lc = cache.layers[self.layer_id]
        prev = lc.window_chrono(start_pos)
        wp = prev.shape[1]
        kv_all = np.concatenate([cast(prev, dt), kv], axis=1) if wp else kv
        idxs = np.broadcast_to(window_idx_matrix(wp, n, a.window_size)[None],
                               (bsz, n, min(a.window_size, wp + n)))
        lc.write_window(start_pos, kv)
        offset = wp + n

        if self.ratio:
            src = shared.kv_src_cache
            compress_len = end_pos // self.ratio
            latents = None
            if self.is_kv_source:
                latents = compressor_forward(x, start_pos, lc.comp_state, p["compressor"],
                                             self.ratio, eps, dt)
                shared.kv_src_cache = src = lc
            if self.is_index_source:
                if self.owns_k:
                    if latents is not None:
                        publish_keys(latents, start_pos, self.ratio, rd, cos, sin,
                                     p["indexer"], eps, dt, lc)
                    shared.index_src_cache = lc
                if compress_len == 0:
                    cidx = np.zeros((bsz, n, 0), np.int32)
                else:
                    index_k = shared.index_src_cache.index_k[:bsz, :compress_len]
                    cidx = indexer_forward(
                        x, qr, start_pos, offset, cos, sin, index_k, shared, p["indexer"], a,
                        (self.ratio, self.is_candidate_source, self.uses_candidates), dt)
                shared.topk_idxs = cidx
            else:
                cidx = shared.topk_idxs
            if latents is not None:
                g0 = start_pos // self.ratio
                g = latents.shape[1]
                pos = group_positions(g0, g, self.ratio)
                latents = rope_tail(latents, rd, cos[pos], sin[pos], dtype=dt)
                latents = fq_fp4_e4m3(latents, 16, dt)
                lc.comp_kv[:bsz, g0:g0 + g] = cast(latents, lc.dtype)
            if compress_len:
                comp = cast(src.comp_kv[:bsz, :compress_len], dt)
                kv_all = np.concatenate([kv_all, comp], axis=1)
                idxs = np.concatenate([idxs, cidx], axis=-1)

        sink = np.zeros_like(p["attn_sink"]) if self.break_sink else p["attn_sink"]
        o = sparse_attn(q, kv_all, sink, idxs, D ** -0.5, dtype=dt)
        if not self.break_rope_inverse:
            o = rope_tail(o, rd, c_q, s_q, inverse=True, dtype=dt)
        G, R = a.o_groups, a.o_lora_rank
        o = o.reshape(bsz, n, G, -1)
        wo_a = np.asarray(p["wo_a"], F32).reshape(G, R, -1)
        o = np.einsum("bsgd,grd->bsgr", o.astype(F32), wo_a).astype(F32)
        return linear(cast(o.reshape(bsz, n, -1), dt), p["wo_b"], dt)


class AttentionStack:
    """Attention-only stack threading SharedState top-down (model.py:35-44, 141-154):
    h <- h + attn_l(attn_norm_l(h)); the FFN, hyper-connections and engram are identity."""

    def __init__(self, a: Args, params: list, dtype: str = "f32"):
        self.a = a
        self.dtype = dtype
        self.layers = [AttentionLayer(i, a, params[i], dtype) for i in range(a.n_layers)]
        self.norms = [params[i]["attn_norm"] for i in range(a.n_layers)]

    def __call__(self, h, cache: ModelCache):
        start_pos = cache.offset
        shared = SharedState()
        for layer, nw in zip(self.layers, self.norms):
            h = cast(np.asarray(h, F32) + layer(rmsnorm(h, nw, self.a.norm_eps, self.dtype),
                                                start_pos, cache, shared), self.dtype)
        cache.offset = start_pos + h.shape[1]
        return h


# ---------------------------------------------------------------------------
# seeded synthetic parameters (shared by tests and the bench's CPU leg)
# ---------------------------------------------------------------------------


def make_params(a: Args, seed: int, dtype: str = "f32") -> list:
    """Weights N(0, 0.02), sinks N(0, 1), norm weights N(1, 0.1), drawn in a fixed
    order from numpy's default_rng(seed); bf16-rounded when dtype is bf16."""
    rng = np.random.default_rng(seed)

    def w(*shape, std=0.02):
        return cast(rng.standard_normal(shape).astype(F32) * F32(std), dtype)

    def nw(dim):
        return (F32(1.0) + rng.standard_normal(dim).astype(F32) * F32(0.1)).astype(F32)

    H, D, dim = a.n_heads, a.head_dim, a.dim
    out = []
    for i in range(a.n_layers):
        p = dict(
            attn_norm=nw(dim),
            wq_a=w(a.q_lora_rank, dim), q_norm=nw(a.q_lora_rank),
            wq_b=w(H * D, a.q_lora_rank), wkv=w(D, dim), kv_norm=nw(D),
            wo_a=w(a.o_groups * a.o_lora_rank, H * D // a.o_groups),
            wo_b=w(dim, a.o_groups * a.o_lora_rank),
            attn_sink=rng.standard_normal(H).astype(F32),
        )
        r = a.compress_ratio(i)
        if i in a.kv_source_layers:
            c = dict(wkv=w(D, dim), norm=nw(D))
            if r > 1:
                c["wgate"] = w(D, dim)
            # the ratio>1 projections run in fp32 (compressor.py:59-61)
            if r > 1:
                c["wkv"] = c["wkv"].astype(F32)
            p["compressor"] = c
        if i in a.index_source_layers:
            ix = dict(wq_b=w(a.index_n_heads * a.index_head_dim, a.q_lora_rank),
                      weights_proj=w(a.index_n_heads, dim))
            if i in a.kv_source_layers:
                ix["wk"] = w(a.index_head_dim, D)
                ix["k_norm"] = nw(a.index_head_dim)
            p["indexer"] = ix
        out.append(p)
    return out
