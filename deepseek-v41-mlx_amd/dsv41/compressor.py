"""Learned KV compression (deepseek_v41_mlx/compressor.py:36-88) on the GPU.

* ratio > 1 (owner layers): ``kv = x @ wkv^T`` and ``score = x @ wgate^T`` in fp32 (the two
  projections are torch GEMMs), then one HIP kernel prepends the carried partial group,
  pools every completed group with a per-channel softmax over the ratio axis, RMSNorms the
  pooled vector and stores the new remainder back into ``CompressorState``;
* ratio == 1: a plain projection followed by the norm.

The result is the **pre-RoPE, pre-quantization** latent ``[b, g, head_dim]`` for the groups this
chunk closes (indices start_pos // ratio ..), or None when no group closes.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _abi
from .config import ModelArgs
from .layers import RMSNorm


class Compressor(torch.nn.Module):
    def __init__(self, args: ModelArgs, layer_id: int, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        self.ratio = args.compress_ratio(layer_id)
        self.head_dim = args.head_dim
        self.norm = RMSNorm(args.head_dim, args.norm_eps, device=device)
        # ratio > 1 pools in fp32, so its projections are held in fp32 (compressor.py:59-61)
        wdt = torch.float32 if self.ratio > 1 else dtype
        self.wkv = torch.nn.Linear(args.dim, args.head_dim, bias=False, dtype=wdt, device=device)
        if self.ratio > 1:
            self.wgate = torch.nn.Linear(args.dim, args.head_dim, bias=False, dtype=torch.float32,
                                         device=device)
        self.requires_grad_(False)

    def forward(self, x: torch.Tensor, start_pos: int, comp_state) -> torch.Tensor | None:
        if self.ratio == 1:
            return self.norm(self.wkv(x))
        xf = x.float()
        kv = F.linear(xf, self.wkv.weight)
        score = F.linear(xf, self.wgate.weight)
        return _abi.compress_pool(kv, score, comp_state.kv_state, comp_state.score_state,
                                  self.norm.weight, self.ratio, start_pos, self.norm.eps, x.dtype)


class CompressorState:
    """The open group's per-token kv/score rows, fp32 (compressor.py:82-88)."""

    def __init__(self, bsz: int, ratio: int, head_dim: int, device="cuda"):
        self.kv_state = torch.zeros(bsz, ratio, head_dim, dtype=torch.float32, device=device)
        self.score_state = torch.full((bsz, ratio, head_dim), float("-inf"), dtype=torch.float32,
                                      device=device)
