"""Incremental attention state in HBM (deepseek_v41_mlx/cache.py:27-78).

Per layer:

* ``win_kv`` -- every layer: a ring of ``window_size`` KV rows, position p at slot p % window;
* ``comp_kv`` -- kv-source (owner) layers only: one latent per completed group, append-only;
  consumer layers never copy it: they read the most recent owner's buffer in place through
  ``SharedState.kv_src_cache``;
* ``comp_state`` -- ratio > 1 owners: the fp32 kv/score rows of the open group;
* ``index_k`` -- owners that are also index sources: the indexer's key cache, read in place
  by every index source below them. With ``index_format="mxfp4"`` the keys -- fp4
  fake-quantized by construction (indexer.py:100-104) -- are held losslessly packed instead:
  ``index_k4`` (e2m1 codes, [b, n, Di/2] bytes) and ``index_ks`` (ue8m0 block scales,
  [b, n, Di/32] bytes), and ``index_k`` is None.

``cache_format="fp8"`` is the fp8 cache variant: the compressed KV and the index keys are
stored as e4m3fn codes with one ue8m0 scale byte per 32 channels of each row (``comp_kv8`` /
``comp_ks``, ``index_k8`` / ``index_k8s``; ``comp_kv`` and ``index_k`` are None), written with
fake_quant_fp8_ue8m0's formula in place of the reference's fp4 QAT at those two stores and
dequantized in-kernel. The window ring stays in ``dtype``.

``cache_format="fp4"`` holds the compressed KV -- fp4/e4m3 fake-quantized by construction
(attention.py:157-163) -- losslessly packed: ``comp_kv4``, rows of d/2 bytes of e2m1 codes then
d/16 e4m3 scale bytes (288 bytes for 512 channels; ``comp_kv`` is None). The index keys follow
``index_format`` (MXFP4 is their lossless packed form), the window ring stays in ``dtype``.
``cache_format="packed"`` adds the window ring in its lossless packed form: ``win_kv8``, MXFP8
rows of d e4m3fn codes then d/32 ue8m0 scale bytes (528 bytes for 512 channels; ``win_kv`` is
None), for window KV that carries the fp8 QAT of attention.py:120-122. The packed stores encode
their QAT, so with the QAT switched off they quantize at the store.

All buffers are plain torch device tensors with the reference's attribute names. The kernels
update them in place, so a snapshot must copy: ``lc.win_kv[:]`` -- which in MLX pins the
pre-step value (generate.py:18-44) -- is a view in torch. ``snapshot(cache)`` and
``restore(cache, snap)`` are the torch counterparts of generate.py's ``_cache_snapshot`` /
``_cache_restore``: they copy every buffer of every format, and restore writes back into the
same tensors, so references to them (a captured HIP graph, a consumer's view) stay valid.

``dtype`` defaults to fp32, the reference's default (cache.py:29, 72). The attention layer
converts at every boundary of a cache held in another dtype than its activations, as the
reference does (attention.py:127, 163, 166); a cache in the activation dtype is read in place.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _abi
from .compressor import CompressorState
from .config import ModelArgs


INDEX_FORMATS = ("dense", "mxfp4")
CACHE_FORMATS = ("dense", "fp8", "fp4", "packed")


class PackedKeys:
    """Index keys of a packed cache as the indexer takes them: kind "mxfp4" or "fp8", the code
    and scale views of rows [:bsz, :n], and the rows one scale byte covers (rb: 1, or 32 for an
    fp8 cache of 32 x 32 blocks)."""

    def __init__(self, kind: str, codes: torch.Tensor, scales: torch.Tensor, rb: int = 1):
        self.kind, self.codes, self.scales, self.rb = kind, codes, scales, rb

    @property
    def shape(self):
        return self.codes.shape


class LayerCache:
    def __init__(self, bsz: int, args: ModelArgs, layer_id: int, max_seq_len: int,
                 dtype=torch.float32, device="cuda", index_format: str = "dense", cache_format: str = "dense",
                 fp8_block_rows: int = 1):
        if index_format not in INDEX_FORMATS:
            raise ValueError(f"index_format must be one of {INDEX_FORMATS}, got {index_format!r}")
        if cache_format not in CACHE_FORMATS:
            raise ValueError(f"cache_format must be one of {CACHE_FORMATS}, got {cache_format!r}")
        if fp8_block_rows not in (1, 32):
            raise ValueError(f"fp8_block_rows must be 1 or 32, got {fp8_block_rows}")
        fp8 = cache_format == "fp8"
        # fp8 caches: one ue8m0 scale byte per 32 channels of every fp8_rb rows (32: 32 x 32 blocks)
        self.fp8_rb = fp8_block_rows if fp8 else 1
        self.window = args.window_size
        self.ratio = args.compress_ratio(layer_id)
        self.is_kv_source = layer_id in args.kv_source_layers
        self.dtype = dtype
        self.win_kv = self.win_kv8 = None
        if cache_format == "packed":
            self.win_kv8 = torch.zeros(bsz, self.window, _abi.mxfp8_row_bytes(args.head_dim), dtype=torch.uint8,
                                       device=device)
        else:
            self.win_kv = torch.zeros(bsz, self.window, args.head_dim, dtype=dtype, device=device)
        self.comp_kv = None
        self.comp_state = None
        self.index_k = None
        self.index_k4 = None
        self.index_ks = None
        self.comp_kv8 = self.comp_ks = self.index_k8 = self.index_k8s = None
        self.comp_kv4 = None
        if self.is_kv_source:
            n_comp = max_seq_len // self.ratio
            d = args.head_dim
            n_blk = -(-n_comp // self.fp8_rb)
            if fp8:
                self.comp_kv8 = torch.zeros(bsz, n_comp, d, dtype=torch.uint8, device=device)
                self.comp_ks = torch.zeros(bsz, n_blk, d // 32, dtype=torch.uint8, device=device)
            elif cache_format in ("fp4", "packed"):
                self.comp_kv4 = torch.zeros(bsz, n_comp, _abi.fp4_row_bytes(d), dtype=torch.uint8, device=device)
            else:
                self.comp_kv = torch.zeros(bsz, n_comp, d, dtype=dtype, device=device)
            if self.ratio > 1:
                self.comp_state = CompressorState(bsz, self.ratio, args.head_dim, device)
            if layer_id in args.index_source_layers:
                di = args.index_head_dim
                if fp8:
                    self.index_k8 = torch.zeros(bsz, n_comp, di, dtype=torch.uint8, device=device)
                    self.index_k8s = torch.zeros(bsz, n_blk, di // 32, dtype=torch.uint8, device=device)
                elif index_format == "mxfp4":
                    self.index_k4 = torch.zeros(bsz, n_comp, di // 2, dtype=torch.uint8, device=device)
                    self.index_ks = torch.zeros(bsz, n_comp, di // 32, dtype=torch.uint8, device=device)
                else:
                    self.index_k = torch.zeros(bsz, n_comp, di, dtype=dtype, device=device)

    def index_keys(self, bsz: int, n: int):
        """The first n keys of rows [:bsz] in the form the indexer takes: a dense view, or the
        PackedKeys of an MXFP4 or fp8 cache."""
        if self.index_k4 is not None:
            return PackedKeys("mxfp4", self.index_k4[:bsz, :n], self.index_ks[:bsz, :n])
        if self.index_k8 is not None:
            return PackedKeys("fp8", self.index_k8[:bsz, :n], self.index_k8s[:bsz, :-(-n // self.fp8_rb)], self.fp8_rb)
        return self.index_k[:bsz, :n]

    def comp_source(self, bsz: int):
        """The compressed cache of rows [:bsz] as the attention reads it: (kind, tensor), kind
        "dense", "fp8" (codes; the scales are ``comp_ks``) or "fp4" (packed rows)."""
        if self.comp_kv8 is not None:
            return "fp8", self.comp_kv8[:bsz]
        if self.comp_kv4 is not None:
            return "fp4", self.comp_kv4[:bsz]
        return "dense", self.comp_kv[:bsz]

    def ring(self):
        """The window ring as the attention reads it: (kind, tensor), kind "dense" or "mxfp8"."""
        return ("mxfp8", self.win_kv8) if self.win_kv8 is not None else ("dense", self.win_kv)

    def window_chrono(self, pos: int) -> torch.Tensor:
        """The ring in chronological order: positions [pos - Wp, pos), Wp = min(pos, window).
        Rows of the packed ring come back as their uint8 MXFP8 rows."""
        w = self.window
        if self.win_kv8 is not None:
            wp = min(pos, w)
            slots = (torch.arange(wp, device=self.win_kv8.device) + (pos - wp)) % w
            return self.win_kv8[:, slots]
        wp = min(pos, w)
        slots = (torch.arange(wp, device=self.win_kv.device) + (pos - wp)) % w
        return self.win_kv[:, slots]

    def write_window(self, pos: int, kv: torch.Tensor) -> None:
        """Write chunk KV at positions [pos, pos+n) into the ring (cache.py:61-67)."""
        if self.win_kv8 is not None:
            _abi.window_write_mxfp8(self.win_kv8, kv.to(self.dtype).contiguous(), pos)
        else:
            _abi.window_write(self.win_kv, kv.to(self.dtype).contiguous(), pos)


class ModelCache:
    def __init__(self, args: ModelArgs, bsz: int = 1, max_seq_len: int | None = None,
                 dtype=torch.float32, device="cuda", index_format: str = "dense", cache_format: str = "dense",
                 fp8_block_rows: int = 1):
        self.max_seq_len = max_seq_len or min(args.max_seq_len, 4096)
        self.offset = 0
        self.layers = [LayerCache(bsz, args, i, self.max_seq_len, dtype, device, index_format, cache_format,
                                  fp8_block_rows)
                       for i in range(args.n_layers)]
        # token ids the engram hasher reads back (cache.py:77-78); host memory, as there
        self.engram_ids = (np.zeros((bsz, self.max_seq_len), dtype=np.int64)
                           if args.engram_layer_ids else None)


_BUFFERS = ("win_kv", "comp_kv", "index_k", "index_k4", "index_ks", "comp_kv8", "comp_ks", "index_k8", "index_k8s",
            "comp_kv4", "win_kv8")


def snapshot(cache: ModelCache):
    """Copies of every cache buffer and the offset (generate.py:18-30 takes the same state)."""
    layers = []
    for lc in cache.layers:
        bufs = {name: getattr(lc, name).clone() for name in _BUFFERS if getattr(lc, name) is not None}
        cs = lc.comp_state
        state = (cs.kv_state.clone(), cs.score_state.clone()) if cs is not None else None
        layers.append((bufs, state))
    eng = cache.engram_ids.copy() if cache.engram_ids is not None else None
    return cache.offset, layers, eng


def restore(cache: ModelCache, snap) -> None:
    """Write a snapshot back (generate.py:33-44), into the same tensors."""
    offset, layers, eng = snap
    if len(layers) != len(cache.layers):
        raise ValueError(f"snapshot of {len(layers)} layers for a cache of {len(cache.layers)}")
    cache.offset = offset
    for lc, (bufs, state) in zip(cache.layers, layers):
        for name, t in bufs.items():
            getattr(lc, name).copy_(t)
        if state is not None:
            lc.comp_state.kv_state.copy_(state[0])
            lc.comp_state.score_state.copy_(state[1])
    if eng is not None:
        cache.engram_ids[...] = eng

