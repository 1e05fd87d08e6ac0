"""The decode hot path of one compressing attention layer as a fixed-shape step.

One step = indexer scoring of every visible compressed entry (MFMA) -> top-k selection ->
sparse MLA over the window ring, this token's KV and the selected compressed entries, with
the inverse rope on the output -- i.e. attention.py:143-175 minus the projections, the
cache writes and the fake-quant prologues, which are per-token elementwise work.

All outputs and scratch are allocated once, so a step issues exactly three kernels (four
when the attention splits its index list) and can be captured in a HIP graph.
"""

from __future__ import annotations

import torch

from . import _abi


class SparseDecodeStep:
    def __init__(self, bsz: int, heads: int, head_dim: int, rd: int, index_heads: int,
                 index_dim: int, nb: int, index_topk: int, window: int, start_pos: int,
                 ratio: int, dtype=torch.bfloat16, device="cuda"):
        self.bsz, self.heads, self.head_dim, self.rd = bsz, heads, head_dim, rd
        self.index_heads, self.index_dim = index_heads, index_dim
        self.nb, self.topk, self.window = nb, index_topk, window
        self.start_pos, self.ratio = start_pos, ratio
        self.dtype = dtype
        self.wp = min(start_pos, window)
        self.offset = self.wp + 1
        self.k = min(index_topk, nb)
        self.scores = torch.empty(bsz, 1, nb, dtype=torch.float32, device=device)
        self.out = torch.empty(bsz, 1, heads, head_dim, dtype=dtype, device=device)
        rows = min(window, self.wp + 1) + self.k
        ws = _abi.mla_workspace_bytes(bsz, 1, heads, head_dim, rows, dtype)
        self.workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=device)

    def __call__(self, q, index_q, w_raw, w_scale, index_k, comp_kv, win_kv, chunk_kv, sink,
                 cos, sin):
        """q [b,1,H,D]; index_q [b,1,Hi,Di] (already roped + fake-quantized); w_raw [b,1,Hi];
        index_k / comp_kv: the owner's caches ([b, >=nb, *] views, read in place);
        win_kv [b, window, D] ring of the previous tokens; chunk_kv [b,1,D] this token's KV."""
        _abi.indexer_score(index_q, w_raw, w_scale, index_k[:, :self.nb], self.start_pos, self.ratio,
                           None, out=self.scores)
        idx = _abi.topk_select(self.scores, self.topk, self.start_pos, self.ratio, self.offset)
        _abi.sparse_mla(q, win_kv, chunk_kv, comp_kv, self.nb, sink, idx, self.head_dim ** -0.5,
                        self.window, self.start_pos, cos, sin, self.rd, out=self.out,
                        workspace=self.workspace)
        return self.out, idx
