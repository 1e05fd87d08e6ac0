"""Gathered sparse MLA (deepseek_v41_mlx/sparse_attention.py:34-60) on the GPU.

* ``kv`` is one shared vector per position: key and value are the same row;
* an index of -1 (or >= kv.shape[1]) contributes nothing;
* ``attn_sink`` enters the softmax denominator only (no value row);
* a row with no valid index yields zeros (the -1e30 max floor).

``chunk`` is accepted for signature compatibility; the kernel streams the index list in
32-row tiles and never materializes the gathered block.
"""

from __future__ import annotations

import torch

from . import _abi

NEG_INF = -1e30


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor,
                topk_idxs: torch.Tensor, softmax_scale: float, chunk: int = 256) -> torch.Tensor:
    """q [b,m,h,d], kv [b,n,d], attn_sink [h] fp32, topk_idxs [b,m,k] int32 -> [b,m,h,d]."""
    del chunk
    return _abi.sparse_attn(q.contiguous(), kv.contiguous(), attn_sink.float().contiguous(),
                            topk_idxs.to(torch.int32).contiguous(), softmax_scale)
