"""Cross-layer sharing and an attention-only stack (deepseek_v41_mlx/model.py:35-44, 141-154).

``SharedState`` is handed down the layer loop afresh every forward: kv sources publish their
``LayerCache`` (compressed KV), index-key owners publish theirs (index keys), index sources
publish their top-k selection and the candidate source its block mask; every later layer
consumes the most recent value in place. ``AttentionStack`` runs only the attention half of
each block: h <- h + attn(attn_norm(h)); MoE, hyper-connections and engram are identity.
"""

from __future__ import annotations

import torch

from .attention import Attention
from .cache import ModelCache
from .config import ModelArgs
from .layers import RMSNorm


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
        for attn, norm in zip(self.layers, self.norms):
            use = shared
            if self._break_sharing and not attn.is_kv_source and attn.ratio:
                use = SharedState()
                use.kv_src_cache = shared.kv_src_cache
                use.index_src_cache = shared.index_src_cache
                use.topk_idxs = (torch.full_like(shared.topk_idxs, -1)
                                 if shared.topk_idxs is not None else None)
            h = h + attn(norm(h), start_pos, cache, use)
        cache.offset = start_pos + h.shape[1]
        return h
