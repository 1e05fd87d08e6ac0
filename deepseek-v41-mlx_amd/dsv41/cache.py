"""Incremental attention state in HBM (deepseek_v41_mlx/cache.py:27-78).

Per layer:

* ``win_kv`` -- every layer: a ring of ``window_size`` KV rows, position p at slot p % window;
* ``comp_kv`` -- kv-source (owner) layers only: one latent per completed group, append-only;
  consumer layers never copy it: they read the most recent owner's buffer in place through
  ``SharedState.kv_src_cache``;
* ``comp_state`` -- ratio > 1 owners: the fp32 kv/score rows of the open group;
* ``index_k`` -- owners that are also index sources: the indexer's key cache, read in place
  by every index source below them.

All buffers are plain torch device tensors with the reference's attribute names, so callers
that snapshot and restore them (generate.py:18-44) work unchanged. The attention kernels
require ``dtype`` to equal the activation dtype.
"""

from __future__ import annotations

import torch

from . import _abi
from .compressor import CompressorState
from .config import ModelArgs


class LayerCache:
    def __init__(self, bsz: int, args: ModelArgs, layer_id: int, max_seq_len: int,
                 dtype=torch.float32, device="cuda"):
        self.window = args.window_size
        self.ratio = args.compress_ratio(layer_id)
        self.is_kv_source = layer_id in args.kv_source_layers
        self.dtype = dtype
        self.win_kv = torch.zeros(bsz, self.window, args.head_dim, dtype=dtype, device=device)
        self.comp_kv = None
        self.comp_state = None
        self.index_k = None
        if self.is_kv_source:
            n_comp = max_seq_len // self.ratio
            self.comp_kv = torch.zeros(bsz, n_comp, args.head_dim, dtype=dtype, device=device)
            if self.ratio > 1:
                self.comp_state = CompressorState(bsz, self.ratio, args.head_dim, device)
            if layer_id in args.index_source_layers:
                self.index_k = torch.zeros(bsz, n_comp, args.index_head_dim, dtype=dtype,
                                           device=device)

    def window_chrono(self, pos: int) -> torch.Tensor:
        """The ring in chronological order: positions [pos - Wp, pos), Wp = min(pos, window)."""
        w = self.window
        wp = min(pos, w)
        slots = (torch.arange(wp, device=self.win_kv.device) + (pos - wp)) % w
        return self.win_kv[:, slots]

    def write_window(self, pos: int, kv: torch.Tensor) -> None:
        """Write chunk KV at positions [pos, pos+n) into the ring (cache.py:61-67)."""
        _abi.window_write(self.win_kv, kv.to(self.dtype).contiguous(), pos)


class ModelCache:
    def __init__(self, args: ModelArgs, bsz: int = 1, max_seq_len: int | None = None,
                 dtype=torch.float32, device="cuda"):
        self.max_seq_len = max_seq_len or min(args.max_seq_len, 4096)
        self.offset = 0
        self.layers = [LayerCache(bsz, args, i, self.max_seq_len, dtype, device)
                       for i in range(args.n_layers)]
        self.engram_ids = None
