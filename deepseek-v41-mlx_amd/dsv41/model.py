"""Cross-layer sharing and an attention-only stack (deepseek_v41_mlx/model.py:35-44, 141-154).

``SharedState`` is handed down the layer loop afresh every forward: kv sources publish their
``LayerCache`` (compressed KV), index-key owners publish theirs (index keys), index sources
publish their top-k selection and the candidate source its block mask; every later layer
consumes the most recent value in place. ``AttentionStack`` runs only the attention half of
each block: h <- h + attn(attn_norm(h)); MoE, hyper-connections and engram are identity.
"""

from __future__ import annotations

import torch

from . import _abi
from .attention import Attention
from .cache import ModelCache
from .config import ModelArgs
from .layers import RMSNorm


def _fused_norm_ok(h: torch.Tensor) -> bool:
    """dsv41_add_rmsnorm's row shapes: whole 16-byte chunks, at most 1,024 of them per row."""
    per = 16 // h.element_size()
    return h.shape[-1] % per == 0 and h.shape[-1] // per <= 1024 and h.data_ptr() % 16 == 0


class SharedState:
    """What attention layers hand down the stack instead of recomputing."""

    def __init__(self):
        self.kv_src_cache = None
        self.index_src_cache = None
        self.topk_idxs = None
        self.candidates = None


class AttentionStack(torch.nn.Module):
    def __init__(self, args: ModelArgs, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.args = args
        self.dtype = dtype
        self.device = torch.device(device)
        self.layers = torch.nn.ModuleList(Attention(i, args, dtype, device) for i in range(args.n_layers))
        self.norms = torch.nn.ModuleList(RMSNorm(args.dim, args.norm_eps, device=device)
                                         for _ in range(args.n_layers))
        # test hook (negative control), model.py:111-112, 145-152
        self._break_sharing = False

    def make_cache(self, bsz: int = 1, max_seq_len: int | None = None, dtype=None, *, index_format: str = "dense",
                   cache_format: str = "dense", fp8_block_rows: int = 1) -> ModelCache:
        """The reference's Model.make_cache (model.py:117-119) takes the cache dtype, fp32 by
        default; here it defaults to the stack's own dtype, whose caches the kernels read in
        place. Any other dtype is converted at each cache boundary, as the reference does."""
        return ModelCache(self.args, bsz, max_seq_len, self.dtype if dtype is None else dtype, self.device,
                          index_format, cache_format, fp8_block_rows)

    def forward(self, h: torch.Tensor, cache: ModelCache) -> torch.Tensor:
        """h [b, n, dim] continues the sequence at cache.offset; advances the cache."""
        start_pos = cache.offset
        shared = SharedState()
        # each block's residual add is fused with the next block's attn_norm (dsv41_add_rmsnorm):
        # the same two ops, bit for bit, in one pass over h, which is updated in place (a copy of
        # the caller's tensor)
        h = h.contiguous().clone()
        delta = None
        for attn, norm in zip(self.layers, self.norms):
            use = shared
            if self._break_sharing and not attn.is_kv_source and attn.ratio:
                use = SharedState()
                use.kv_src_cache = shared.kv_src_cache
                use.index_src_cache = shared.index_src_cache
                use.topk_idxs = (torch.full_like(shared.topk_idxs, -1)
                                 if shared.topk_idxs is not None else None)
            if delta is None:
                x = norm(h)
            elif _fused_norm_ok(h):
                x = _abi.add_rmsnorm(h, delta.contiguous(), norm.weight, norm.eps)
            else:
                h.add_(delta)
                x = norm(h)
            delta = attn(x, start_pos, cache, use)
        if delta is not None:
            h = h + delta
        cache.offset = start_pos + h.shape[1]
        return h
