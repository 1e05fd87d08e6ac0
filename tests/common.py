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


# ---------------------------------------------------------------- bf16 attention check

# bf16 attention outputs are held to the 2e-2 relative gate, and to two per-head bounds at the
# kernels' own error level (bf16 rounding of the softmax weights fed to the PV product and of the
# output), which a sink in the wrong place, a dropped list row or a shifted window exceed even
# where they stay inside 2e-2 of max |o|:
#   * per-head scale: alpha_h = <got_h, want_h> / <want_h, want_h>, over every query and channel
#     of head h, within ATTN_ALPHA of 1 -- a sink that enters a head's denominator wrongly
#     scales that head's whole output. The kernels normalize by the sum of the bf16 weights they
#     multiply, so rounding only moves weight between rows; where one row dominates a head that
#     moves the fit by up to one bf16 half-ulp, 2^-8, the bound (over many rows it averages out:
#     ~2e-4 at 640 rows);
#   * per-head max error within ATTN_HEAD_REL of that head's own max |want_h|.
ATTN_ALPHA = 2.0 ** -8
ATTN_HEAD_REL = 1.5e-2


def attn_metrics(got, want):
    """(max |got - want| / max |want|, max_h |alpha_h - 1|, max_h per-head relative max error)
    over arrays [..., heads, channels]."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    h = g.shape[-2]
    g2 = np.moveaxis(g, -2, 0).reshape(h, -1)
    w2 = np.moveaxis(w, -2, 0).reshape(h, -1)
    ww = (w2 * w2).sum(1)
    live = ww > 0
    alpha = np.where(live, (g2 * w2).sum(1) / np.where(live, ww, 1.0), 1.0)
    head_max = np.abs(w2).max(1)
    err = np.abs(g2 - w2).max(1)
    head_err = np.where(live, err / np.where(live, head_max, 1.0), err)
    return rel_max_diff(g, w), float(np.abs(alpha - 1).max()), float(head_err.max())


def attn_close(got, want) -> bool:
    rel, a, e = attn_metrics(got, want)
    return rel < 2e-2 and a <= ATTN_ALPHA and e <= ATTN_HEAD_REL


def assert_attn_close(got, want, what=""):
    rel, a, e = attn_metrics(got, want)
    assert rel < 2e-2 and a <= ATTN_ALPHA and e <= ATTN_HEAD_REL, \
        f"{what} rel {rel:.3e} |alpha-1| {a:.3e} head err {e:.3e}"


def attn_controls(idx, sink, window_rows=0):
    """Planted mistakes for the bf16 attention check, as changed oracle inputs: (name, idx, sink).
    idx [b, m, k] with the window rows first (window_rows of them) when window_rows > 0.

    * the sink zeroed;
    * the sink counted once per split of two (its weight doubled: sink + ln 2);
    * the last valid list row of every query dropped;
    * the window read one row early: its rows' indices minus one (the oldest row that has just
      left the window in, the newest row out)."""
    idx = np.asarray(idx)
    yield "sink zeroed", idx, np.zeros_like(sink)
    yield "sink once per split", idx, (sink + np.log(2.0)).astype(np.float32)
    dropped = idx.copy()
    valid = dropped >= 0
    last = dropped.shape[-1] - 1 - np.argmax(valid[..., ::-1], axis=-1)
    has = valid.any(-1)
    bi, mi = np.nonzero(has)
    dropped[bi, mi, last[bi, mi]] = -1
    yield "one list row dropped", dropped, sink
    if window_rows:
        shifted = idx.copy()
        win = shifted[..., :window_rows]
        shifted[..., :window_rows] = np.where(win >= 0, win - 1, -1)
        yield "window shifted by one", shifted, sink
