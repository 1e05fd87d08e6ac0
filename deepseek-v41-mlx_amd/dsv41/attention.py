"""One V4.1 attention layer (deepseek_v41_mlx/attention.py:53-179) on the GPU.

The compressor projections are torch GEMMs, and so are the other projections outside decode row
counts. At decode row counts wq_a and wkv run in one dsv41_linear_rows_pair launch, the indexer's
wq_b and weights_proj on dsv41_linear_rows, and wq_b and wo_b on dsv41_linear_rows where its
128-row tiles apply (33-64 rows at the release's widths); otherwise they stay torch GEMMs
(layers.decode_linear).
Everything between them, and the grouped block-diagonal wo_a, runs in HIP kernels:

  q      : q_norm (RMSNorm kernel); q's rope tail is applied by the attention launch as it
           loads q (no separate pass over q)
  kv     : kv_norm -> rope -> fp8 fake-quant, one fused kernel, in place
  owner  : compressor pooling kernel; index keys published into its own index_k; latents
           roped + fp4/e4m3 fake-quantized straight into its comp_kv (no staging copy)
  index  : fused q prologue, MFMA scoring, candidate blocks, top-k
  attend : one sparse-MLA kernel that reads the previous window ring, this chunk's KV and the
           most recent owner's comp_kv in place -- the reference's concatenation of the three
           (attention.py:127, 165-168) never happens -- and applies the inverse rope to the
           output tail before storing it.
  output : the grouped wo_a (dsv41_wo_a_grouped: exact products, fp32 sums, one rounding to
           x's dtype), reading the attention output and wo_a's weight in place; then wo_b.
The window ring is written after the attention kernel has read the previous window, which
is equivalent to the reference's write-before-concatenate order because the concatenated
copy held the old ring contents.

Caches held in another dtype than the activations (the reference's default: fp32 caches under a
bf16 model, cache.py:29, 72) are converted at every cache boundary, as the reference converts
them (attention.py:127, 163, 166; cache.py:67): stores compute in the activation dtype and
convert on the store, reads convert the visible rows to the activation dtype first. That costs
one copy of the visible cache per call; keeping the cache in the activation dtype reads it in
place.

The forward is chunk-general: prefill, chunked prefill and 1-token decode share one path.
"""

from __future__ import annotations

import torch

from . import _abi, fakequant
from .compressor import Compressor
from .config import ModelArgs
from .indexer import Indexer
from .layers import RMSNorm, decode_linear, decode_linear_pair, yarn_inv_freqs


# multiply-adds from which fp32 activations take the batched GEMM for wo_a (the release shape
# 8 x (4096 -> 1024) from two rows on)
_WO_A_FP32_GEMM_MACS = 1 << 26


def window_idx_matrix(wp: int, n: int, window: int, device="cuda") -> torch.Tensor:
    """[n, min(window, wp+n)] int32 indices into concat(prev window(wp), chunk(n)), -1 pads
    (attention.py:40-50)."""
    return _abi.window_idx(wp, n, window, torch.device(device))


class Attention(torch.nn.Module):
    def __init__(self, layer_id: int, args: ModelArgs, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.layer_id = layer_id
        self.dim = args.dim
        self.n_heads = args.n_heads
        self.head_dim = args.head_dim
        self.rope_head_dim = args.rope_head_dim
        self.q_lora_rank = args.q_lora_rank
        self.o_lora_rank = args.o_lora_rank
        self.n_groups = args.o_groups
        self.window_size = args.window_size
        self.ratio = args.compress_ratio(layer_id)
        self.eps = args.norm_eps
        self.softmax_scale = args.head_dim ** -0.5
        self.dtype = dtype
        self.device = torch.device(device)

        def lin(i, o):
            return torch.nn.Linear(i, o, bias=False, dtype=dtype, device=device)

        self.attn_sink = torch.nn.Parameter(torch.zeros(self.n_heads, dtype=torch.float32, device=device))
        self.wq_a = lin(self.dim, self.q_lora_rank)
        self.q_norm = RMSNorm(self.q_lora_rank, self.eps, device=device)
        self.wq_b = lin(self.q_lora_rank, self.n_heads * self.head_dim)
        self.wkv = lin(self.dim, self.head_dim)
        self.kv_norm = RMSNorm(self.head_dim, self.eps, device=device)
        self.wo_a = lin(self.n_heads * self.head_dim // self.n_groups, self.n_groups * self.o_lora_rank)
        self.wo_b = lin(self.n_groups * self.o_lora_rank, self.dim)

        self.is_kv_source = layer_id in args.kv_source_layers
        self.is_index_source = layer_id in args.index_source_layers
        if self.is_kv_source:
            self.compressor = Compressor(args, layer_id, dtype, device)
        if self.is_index_source:
            self.indexer = Indexer(args, layer_id, dtype, device)

        if self.ratio:
            orig_len, theta = args.original_seq_len, args.compress_rope_theta
        else:
            orig_len, theta = 0, args.rope_theta
        self._rope = (args.rope_head_dim, orig_len, theta, args.rope_factor, args.beta_fast,
                      args.beta_slow)
        self._freq_vec = None
        self._cos = None
        self._sin = None
        self._workspace = None
        self.requires_grad_(False)

        # test hooks (negative controls), attention.py:95-97
        self._break_rope_inverse = False
        self._break_sink = False

    def _freqs(self, upto: int):
        """Device (cos, sin) tables covering positions < upto; grown geometrically."""
        if self._cos is None or self._cos.shape[0] < upto:
            if self._freq_vec is None:
                rd, orig_len, theta, factor, bf, bs = self._rope
                self._freq_vec = torch.from_numpy(yarn_inv_freqs(rd, orig_len, theta, factor, bf, bs)).to(self.device)
            rows = max(upto, 64, 0 if self._cos is None else 2 * self._cos.shape[0])
            self._cos, self._sin = _abi.rope_table(self._freq_vec, rows)
        return self._cos, self._sin

    def _kv_prologue(self, kv, cos, sin, start_pos):
        rd = self.rope_head_dim
        if fakequant.DISABLE:
            kv = _abi.rmsnorm(kv, self.kv_norm.weight, self.eps)
            return _abi.rope_tail(kv, rd, cos, sin, start_pos, 1)
        return _abi.kv_window_prep(kv, self.kv_norm.weight, cos, sin, rd, start_pos, self.eps)

    def _write_latents(self, latents, lc, g0, cos, sin):
        rd = self.rope_head_dim
        if lc.comp_kv8 is not None:           # fp8 cache variant: fp8 QAT, stored packed
            _abi.comp_write_fp8(latents.to(self.dtype).contiguous(), lc.comp_kv8, lc.comp_ks, g0, self.ratio, cos,
                                sin, rd, lc.fp8_rb)
            return
        if lc.comp_kv4 is not None:           # packed fp4 cache: the same fp4/e4m3 QAT, stored packed
            _abi.comp_write_fp4(latents.to(self.dtype).contiguous(), lc.comp_kv4, g0, self.ratio, cos, sin, rd)
            return
        lat = latents.contiguous()
        if fakequant.DISABLE:
            lat = _abi.rope_tail(lat, rd, cos, sin, g0 * self.ratio, self.ratio)
            lc.comp_kv[:lat.shape[0], g0:g0 + lat.shape[1]] = lat
            return
        if lc.comp_kv.dtype == lat.dtype:
            _abi.comp_write(lat, lc.comp_kv, g0, self.ratio, cos, sin, rd)
            return
        # a cache in another dtype: rope + QAT in the latents' dtype, converted on the store
        # (attention.py:158-163); tables shifted so group j sits at position (g0 + j) * ratio
        staged = torch.empty_like(lat)
        p0 = g0 * self.ratio
        _abi.comp_write(lat, staged, 0, self.ratio, cos[p0:], sin[p0:], rd)
        lc.comp_kv[:lat.shape[0], g0:g0 + lat.shape[1]] = staged

    def forward(self, x: torch.Tensor, start_pos: int, cache, shared) -> torch.Tensor:
        """x [b, n, dim] (post attn_norm), absolute positions [start_pos, start_pos + n)."""
        bsz, n, _ = x.shape
        rd = self.rope_head_dim
        end_pos = start_pos + n
        cos, sin = self._freqs(end_pos)
        x = x.contiguous()

        # wq_a and wkv read the same rows: one launch at decode row counts
        qa, kv_raw = decode_linear_pair(self.wq_a, self.wkv, x)
        # queries: q's rope tail (attention.py:117) is applied by the attention launch as it loads q
        qr = self.q_norm(qa)
        q = decode_linear(self.wq_b, qr, wide_only=True).view(bsz, n, self.n_heads, self.head_dim).contiguous()

        # this chunk's window KV
        kv = self._kv_prologue(kv_raw.contiguous(), cos, sin, start_pos)

        lc = cache.layers[self.layer_id]
        wp = min(start_pos, self.window_size)
        offset = wp + n                     # compressed entries follow window + chunk
        cidx = None
        comp, n_comp, comp_kind = None, 0, "dense"
        if self.ratio:
            src = shared.kv_src_cache
            compress_len = end_pos // self.ratio
            latents = None
            if self.is_kv_source:
                latents = self.compressor(x, start_pos, lc.comp_state)
                shared.kv_src_cache = src = lc
            if self.is_index_source:
                if self.indexer.owns_k:
                    if latents is not None:
                        self.indexer.publish_keys(latents, start_pos, cos, sin, lc)
                    shared.index_src_cache = lc
                if compress_len == 0:
                    cidx = torch.zeros(bsz, n, 0, dtype=torch.int32, device=x.device)
                else:
                    index_k = shared.index_src_cache.index_keys(bsz, compress_len)
                    if isinstance(index_k, torch.Tensor) and index_k.dtype != x.dtype:
                        index_k = index_k.to(x.dtype)   # indexer.py:125 reads the keys converted
                    cidx = self.indexer(x, qr, start_pos, offset, cos, sin, index_k, shared)
                shared.topk_idxs = cidx
            else:
                cidx = shared.topk_idxs
            if latents is not None:
                self._write_latents(latents, lc, start_pos // self.ratio, cos, sin)
            if compress_len:
                (comp_kind, comp), n_comp = src.comp_source(bsz), compress_len
                if comp_kind == "dense" and comp.dtype != x.dtype:
                    comp = comp[:, :n_comp].to(x.dtype)     # attention.py:166

        sink = torch.zeros_like(self.attn_sink) if self._break_sink else self.attn_sink
        # one-token decode: the attention launch also writes the token into the ring (the slot it
        # takes is outside the token's window); a chunk writes its ring after the attention
        # (a ring held in another dtype is read converted, attention.py:127, and written after)
        ring = lc.win_kv
        if ring is not None and ring.dtype != x.dtype:
            ring = ring[:bsz].to(x.dtype)
        decode = n == 1 and ring is lc.win_kv
        sel = cidx if cidx is not None and cidx.shape[-1] else None
        rdo = 0 if self._break_rope_inverse else rd
        if lc.win_kv8 is not None:          # the packed cache: MXFP8 ring, fp4 compressed rows
            o = _abi.sparse_mla_packed(q, lc.win_kv8, kv, comp if comp_kind == "fp4" else None, n_comp, sink, sel,
                                       self.softmax_scale, self.window_size, start_pos, cos, sin, rdo,
                                       write_ring=decode, q_rd=rd)
        elif comp_kind == "fp8":
            o = _abi.sparse_mla_fp8(q, ring, kv, comp, src.comp_ks[:bsz], src.fp8_rb, n_comp, sink, sel,
                                    self.softmax_scale, self.window_size, start_pos, cos, sin, rdo, write_ring=decode,
                                    q_rd=rd)
        elif comp_kind == "fp4":
            o = _abi.sparse_mla_fp4(q, ring, kv, comp, n_comp, sink, sel, self.softmax_scale, self.window_size,
                                    start_pos, cos, sin, rdo, write_ring=decode, q_rd=rd)
        else:
            o = _abi.sparse_mla(q, ring, kv, comp, n_comp, sink, sel, self.softmax_scale, self.window_size,
                                start_pos, cos, sin, rdo, write_ring=decode, q_rd=rd)
        if not decode:
            lc.write_window(start_pos, kv)

        # grouped block-diagonal wo_a, fp32 sums cast to x's dtype, then wo_b (attention.py:176-179)
        # wo_b at 33-64 rows: 128-row tiles over 4 contraction ranges and their reduce (24.4 + 4.5
        # us at 64 rows against 28.9 us for the library; the 40-layer token 5.748 against 5.78 ms)
        return decode_linear(self.wo_b, self._wo_a(o.view(bsz, n, -1), x.dtype), wide_only=True)

    def _wo_a(self, o, out_dtype):
        g, r = self.n_groups, self.o_lora_rank
        d = o.shape[-1] // g
        rows = o.numel() // o.shape[-1]
        if o.dtype == torch.float32 and rows * o.shape[-1] * r >= _WO_A_FP32_GEMM_MACS:
            # fp32 activations at GEMM-sized shapes: one fp32 GEMM per group (the grouped kernel's
            # fp32 form is a one-thread-per-output loop, meant for small shapes)
            og = o.reshape(rows, g, d).transpose(0, 1).contiguous()                  # [g, rows, d]
            wg = self.wo_a.weight.view(g, r, d).transpose(1, 2).contiguous()         # [g, d, r]
            return torch.bmm(og, wg).transpose(0, 1).reshape(*o.shape[:-1], g * r).to(out_dtype)
        return _abi.wo_a_grouped(o, self.wo_a.weight, g, out_dtype=out_dtype)
