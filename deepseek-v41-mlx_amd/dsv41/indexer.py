"""The sparse-attention indexer (deepseek_v41_mlx/indexer.py:38-144) on the GPU.

Owners (kv source and index source) turn their pre-RoPE latents into index keys
(``publish_keys``: wk GEMM, then one fused kernel: k_norm -> rope at g*ratio -> fp4/ue8m0
fake-quant -> store into ``index_k`` in place). Every index source scores its own queries
against the most recent owner's keys, read in place:

  q = fq4(rope(wq_b(qr)))  (one fused kernel after the wq_b GEMM)
  S[b,s,t] = sum_h relu(q[b,s,h] . k[b,t]) * w[b,s,h],  w = weights_proj(x) * Di^-1/2 Hi^-1/2

on MFMA, with the visibility mask (t >= lens_s -> -inf) and, for layers after the candidate
source, the candidate mask applied in the same pass. The candidate source publishes its
block mask (``select_candidate_blocks``); the top-k kernel returns the ``index_topk`` best
positions per query in ascending order, offset into the attention's unified index space, -1
past the visible range. Decode queries of index sources other than the candidate source, on
keys of shapes it serves, take the fused form (dsv41_indexer_topk(_fp8, _mxfp4)): the scoring kernel
keeps each row range's best index_topk and a merge selects from those lists -- the same
selection, without writing the scores.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _abi, fakequant
from .config import ModelArgs
from .layers import RMSNorm, decode_linear


def _lens_tensor(lens, device) -> torch.Tensor:
    if isinstance(lens, torch.Tensor):
        return lens.reshape(-1).to(device=device, dtype=torch.int32).contiguous()
    return torch.as_tensor(np.asarray(lens).reshape(-1), dtype=torch.int32, device=device)


def select_candidate_blocks(scores: torch.Tensor, lens, topk_blocks: int,
                            block_size: int) -> torch.Tensor:
    """Level one of the two-level top-k (indexer.py:38-64). scores [b, n, nb] fp32 with
    unreachable positions at -inf; lens [n] or [n, 1]. Returns a bool mask like scores."""
    return _abi.candidate_blocks(scores.float().contiguous(), topk_blocks, block_size,
                                 _lens_tensor(lens, scores.device))


def weight_scale(n_heads: int, head_dim: int, dtype) -> float:
    """head_dim**-0.5 * n_heads**-0.5 as the activation dtype holds it: a python scalar
    multiplying an MLX array takes the array's dtype (indexer.py:123)."""
    return float(torch.tensor(head_dim ** -0.5 * n_heads ** -0.5, dtype=dtype).float())


class Indexer(torch.nn.Module):
    def __init__(self, args: ModelArgs, layer_id: int, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.layer_id = layer_id
        self.owns_k = layer_id in args.kv_source_layers
        self.ratio = args.compress_ratio(layer_id)
        self.is_candidate_source = layer_id == args.candidate_source_layer
        self.uses_candidates = 0 <= args.candidate_source_layer < layer_id
        self.candidate_topk_blocks = args.candidate_topk_blocks
        self.candidate_block_size = args.candidate_block_size
        self.n_heads = args.index_n_heads
        self.head_dim = args.index_head_dim
        self.rope_head_dim = args.rope_head_dim
        self.index_topk = args.index_topk
        self.softmax_scale = self.head_dim ** -0.5
        self.wq_b = torch.nn.Linear(args.q_lora_rank, self.n_heads * self.head_dim, bias=False,
                                    dtype=dtype, device=device)
        self.weights_proj = torch.nn.Linear(args.dim, self.n_heads, bias=False, dtype=dtype,
                                            device=device)
        if self.owns_k:
            self.wk = torch.nn.Linear(args.head_dim, self.head_dim, bias=False, dtype=dtype,
                                      device=device)
            self.k_norm = RMSNorm(self.head_dim, args.norm_eps, device=device)
        self.requires_grad_(False)

    def publish_keys(self, latents: torch.Tensor, start_pos: int, cos, sin, cache) -> None:
        """Index keys of this chunk's pre-RoPE latents into cache.index_k (indexer.py:89-104),
        or packed into an MXFP4 cache (index_k4 / index_ks)."""
        g0 = start_pos // self.ratio
        rd = self.rope_head_dim
        k_raw = self.wk(latents).contiguous()
        if cache.index_k8 is not None:
            _abi.index_key_publish_fp8(k_raw, cache.index_k8, cache.index_k8s, g0, self.ratio, self.k_norm.weight,
                                       cos, sin, rd, self.k_norm.eps, cache.fp8_rb)
            return
        if cache.index_k4 is not None:
            if fakequant.DISABLE:
                raise ValueError("an MXFP4 index cache holds fp4 fake-quantized keys; QAT is disabled")
            _abi.index_key_publish_mxfp4(k_raw, cache.index_k4, cache.index_ks, g0, self.ratio, self.k_norm.weight,
                                         cos, sin, rd, self.k_norm.eps)
            return
        if fakequant.DISABLE:
            k = _abi.rmsnorm(k_raw, self.k_norm.weight, self.k_norm.eps)
            k = _abi.rope_tail(k, rd, cos, sin, g0 * self.ratio, self.ratio)
            cache.index_k[:k.shape[0], g0:g0 + k.shape[1]] = k
            return
        if cache.index_k.dtype == k_raw.dtype:
            _abi.index_key_publish(k_raw, cache.index_k, g0, self.ratio, self.k_norm.weight, cos, sin,
                                   rd, self.k_norm.eps)
            return
        # a cache in another dtype: norm, rope and QAT in the keys' dtype, converted on the store
        # (indexer.py:104); tables shifted so group j sits at position (g0 + j) * ratio
        staged = torch.empty_like(k_raw)
        p0 = g0 * self.ratio
        _abi.index_key_publish(k_raw, staged, 0, self.ratio, self.k_norm.weight, cos[p0:], sin[p0:], rd,
                               self.k_norm.eps)
        cache.index_k[:k_raw.shape[0], g0:g0 + k_raw.shape[1]] = staged

    def forward(self, x: torch.Tensor, qr: torch.Tensor, start_pos: int, offset: int,
                cos, sin, index_k: torch.Tensor, shared) -> torch.Tensor:
        """x [b,n,dim], qr [b,n,q_lora]; index_k [b, nb, Di] (the owner's cache, in place), or
        the PackedKeys of an MXFP4 or fp8 cache (LayerCache.index_keys).
        Returns [b, n, min(index_topk, nb)] int32 indices, -1 masked."""
        bsz, n, _ = x.shape
        rd = self.rope_head_dim
        # decode rows: dsv41_linear_rows (8.8-9.2 us at 32-64 rows against 18.2-18.4 us for torch's linear)
        q = decode_linear(self.wq_b, qr).view(bsz, n, self.n_heads, self.head_dim).contiguous()
        # decode rows: dsv41_linear_rows (5120 -> 64: 17.8 us for torch's linear inside the token)
        w_raw = decode_linear(self.weights_proj, x).contiguous()
        w_scale = weight_scale(self.n_heads, self.head_dim, x.dtype)
        cand = None
        if not self.is_candidate_source and self.uses_candidates and shared.candidates is not None:
            cand = shared.candidates
        if getattr(index_k, "kind", None) == "mxfp4":
            if fakequant.DISABLE:
                raise ValueError("an MXFP4 index cache holds fp4 fake-quantized keys; QAT is disabled")
            q_mx = _abi.index_q_prep_mxfp4(q, cos, sin, rd, start_pos)
            nb = index_k.codes.shape[1]
            if not self.is_candidate_source:
                idx = _abi.indexer_topk_mxfp4(q_mx, w_raw, w_scale, index_k.codes, index_k.scales, nb, start_pos,
                                              self.ratio, self.index_topk, offset, cand)
                if idx is not None:
                    return idx
            scores = _abi.indexer_score_mxfp4(q_mx, w_raw, w_scale, index_k.codes, index_k.scales, nb, start_pos,
                                              self.ratio, cand)
        elif getattr(index_k, "kind", None) == "fp8":
            if fakequant.DISABLE:
                q = _abi.rope_tail(q, rd, cos, sin, start_pos, 1)
            else:
                _abi.index_q_prep(q, cos, sin, rd, start_pos)
            nb = index_k.codes.shape[1]
            if not self.is_candidate_source and q.dtype == torch.bfloat16:
                idx = _abi.indexer_topk_fp8(q, w_raw, w_scale, index_k.codes, index_k.scales, index_k.rb, nb, start_pos,
                                            self.ratio, self.index_topk, offset, cand)
                if idx is not None:
                    return idx
            scores = _abi.indexer_score_fp8(q, w_raw, w_scale, index_k.codes, index_k.scales, index_k.rb, nb, start_pos,
                                            self.ratio, cand)
        else:
            if fakequant.DISABLE:
                q = _abi.rope_tail(q, rd, cos, sin, start_pos, 1)
            else:
                _abi.index_q_prep(q, cos, sin, rd, start_pos)
            if not self.is_candidate_source and q.dtype == torch.bfloat16:
                # decode shapes the fused form serves: the same selection, the scores never written
                idx = _abi.indexer_topk(q, w_raw, w_scale, index_k, start_pos, self.ratio, self.index_topk, offset,
                                        cand)
                if idx is not None:
                    return idx
            scores = _abi.indexer_score(q, w_raw, w_scale, index_k, start_pos, self.ratio, cand)
        if self.is_candidate_source:
            shared.candidates = _abi.candidate_blocks(scores, self.candidate_topk_blocks,
                                                      self.candidate_block_size, None, start_pos,
                                                      self.ratio)
        return _abi.topk_select(scores, self.index_topk, start_pos, self.ratio, offset)
