"""Shared test helpers: the parity configs, seeded inputs, weight loading, metrics."""

from __future__ import annotations

import numpy as np

from oracle import cpu_ref as R

SEED_BASE = 20261201

# C1: tiny fp32 parity config -- 4 attention layers, hidden 256, 4 heads, KV latent 64 incl.
# a 16-channel rope tail, indexer 2 x 32, ratio 4, top-k 16, layer 0 owns the cache and the
# index keys, layers 1-3 consume. YaRN is exercised (original_seq_len 64 < 144 positions).
C1 = dict(dim=256, n_layers=4, n_heads=4, head_dim=64, rope_head_dim=16, q_lora_rank=64,
          o_lora_rank=32, o_groups=2, window_size=128, compress_ratios=(4, 4, 4, 4),
          kv_source_layers=(0,), index_source_layers=(0,), index_n_heads=2, index_head_dim=32,
          index_topk=16, rope_theta=10000.0, compress_rope_theta=10000.0, original_seq_len=64,
          rope_factor=4.0, max_seq_len=256)

# A tiny topology with every sharing role: a window-only layer (0), an owner (1), a
# consumer (2), an index source without keys that is the candidate source (3), a consumer
# (4) and a candidate consumer (5); window 8 so the ring wraps.
TOPO = dict(dim=64, n_layers=6, n_heads=4, head_dim=64, rope_head_dim=16, q_lora_rank=32,
            o_lora_rank=16, o_groups=2, window_size=8, compress_ratios=(0, 4, 4, 4, 4, 4),
            kv_source_layers=(1,), index_source_layers=(1, 3, 5), candidate_source_layer=3,
            candidate_topk_blocks=3, candidate_block_size=2, index_n_heads=4, index_head_dim=32,
            index_topk=4, rope_theta=10000.0, compress_rope_theta=40000.0, original_seq_len=64,
            rope_factor=4.0, max_seq_len=128)

# The 40-layer sharing topology of the C4 decode config at toy sizes: window-only layers 0-1,
# owners 2/8/14/20, index sources 2..36 (24-36 score against layer 20's keys under its
# candidate mask, which keeps 3 of 5 blocks here), ratio 4, window 8 (the ring wraps).
C4_TOY = dict(dim=64, n_layers=40, n_heads=4, head_dim=64, rope_head_dim=16, q_lora_rank=32,
              o_lora_rank=16, o_groups=2, window_size=8, compress_ratios=(0, 0) + (4,) * 38,
              kv_source_layers=(2, 8, 14, 20), index_source_layers=(2, 8, 14, 20, 24, 28, 32, 36),
              candidate_source_layer=20, candidate_topk_blocks=3, candidate_block_size=2,
              index_n_heads=16, index_head_dim=32, index_topk=4, rope_theta=10000.0,
              compress_rope_theta=40000.0, original_seq_len=64, rope_factor=4.0, max_seq_len=128)


# The release's compression ratios at toy size -- the sharing pattern of the reference test's own
# configuration (tests/test_parity.py:77-83): window-only layers 0-1; a ratio-2 owner (2) with two
# consumers (3, 4); a ratio-1 owner (5) that is also the candidate source (3 blocks of 2); a
# ratio-1 consumer (6); and a ratio-1 index source without keys (7) that scores layer 5's keys
# under layer 5's candidate mask. Window 8, so the ring wraps; top-4 of up to 40 entries.
RELEASE_TOY = dict(dim=64, n_layers=8, n_heads=4, head_dim=64, rope_head_dim=16, q_lora_rank=32,
                   o_lora_rank=16, o_groups=4, window_size=8, compress_ratios=(0, 0, 2, 2, 2, 1, 1, 1),
                   kv_source_layers=(2, 5), index_source_layers=(2, 5, 7), candidate_source_layer=5,
                   candidate_topk_blocks=3, candidate_block_size=2, index_n_heads=8, index_head_dim=32,
                   index_topk=4, rope_theta=10000.0, compress_rope_theta=40000.0, original_seq_len=64,
                   rope_factor=4.0, max_seq_len=128)


def args(cfg: dict) -> R.Args:
    return R.Args(**cfg)


def rel_max_diff(a, b) -> float:
    """max |a - b| / max |b| (the reference test's metric, tests/test_parity.py:238-240)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-9))


def max_abs(a, b) -> float:
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


def to_np(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


# ---------------------------------------------------------------- torch-side loading


def _set(param, arr):
    import torch
    param.data.copy_(torch.as_tensor(np.asarray(arr, np.float32)).to(param.dtype))


def load_attention(attn, p: dict) -> None:
    """Copy one layer's oracle parameters (oracle.cpu_ref.make_params) into a dsv41 Attention."""
    for name in ("wq_a", "wq_b", "wkv", "wo_a", "wo_b"):
        _set(getattr(attn, name).weight, p[name])
    _set(attn.q_norm.weight, p["q_norm"])
    _set(attn.kv_norm.weight, p["kv_norm"])
    _set(attn.attn_sink, p["attn_sink"])
    if "compressor" in p:
        c = p["compressor"]
        _set(attn.compressor.wkv.weight, c["wkv"])
        _set(attn.compressor.norm.weight, c["norm"])
        if "wgate" in c:
            _set(attn.compressor.wgate.weight, c["wgate"])
    if "indexer" in p:
        ix = p["indexer"]
        _set(attn.indexer.wq_b.weight, ix["wq_b"])
        _set(attn.indexer.weights_proj.weight, ix["weights_proj"])
        if "wk" in ix:
            _set(attn.indexer.wk.weight, ix["wk"])
            _set(attn.indexer.k_norm.weight, ix["k_norm"])


def load_stack(stack, params: list) -> None:
    for attn, norm, p in zip(stack.layers, stack.norms, params):
        load_attention(attn, p)
        _set(norm.weight, p["attn_norm"])


def model_args(cfg: dict):
    from dsv41.config import ModelArgs
    return ModelArgs(**cfg)
