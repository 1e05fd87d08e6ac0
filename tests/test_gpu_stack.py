"""The 40-layer decode step (dsv41.step.StackDecodeStep) of the C4 sharing topology.

* Toy size: the kernels-only step reproduces, bit for bit, every per-layer attention output
  and every cache write of the full ``AttentionStack`` forward (projections included) for the
  same decode token -- the per-layer kernel inputs are recorded from that forward.
* Full size (batch 64, 65,536-token context -> 16,384 entries, 64 heads x 512, indexer
  64 x 128, top-512, 40 layers): sampled rows of a window-only layer, the last index source
  (layer 36: its own queries against layer 20's keys under layer 20's candidate mask) and a
  consumer (layer 39) against the oracle -- scores within 1e-5 of max |S|, top-k bit-exact
  given those scores, outputs within the bf16 attention check (2e-2 relative plus per-head bounds).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from common import C4_TOY, RELEASE_TOY, SEED_BASE, args, assert_attn_close, load_stack, model_args, to_np
from oracle import cpu_ref as R

pytestmark = pytest.mark.gpu
F32 = np.float32


def _clone_cache(cache):
    import copy
    from dsv41.cache import _BUFFERS
    c = copy.copy(cache)
    c.layers = []
    for lc in cache.layers:
        n = copy.copy(lc)
        for name in _BUFFERS:
            t = getattr(lc, name)
            setattr(n, name, None if t is None else t.clone())
        c.layers.append(n)
    return c


def _record_decode(stack, h, cache):
    """Run one forward of the stack and record the kernel inputs of each layer."""
    from dsv41 import _abi
    recs = [dict() for _ in stack.layers]
    layer = [0]
    orig = {n: getattr(_abi, n) for n in ("sparse_mla", "indexer_score", "comp_write", "index_key_publish",
                                          "indexer_score_mxfp4", "index_key_publish_mxfp4", "sparse_mla_fp8",
                                          "indexer_score_fp8", "comp_write_fp8", "index_key_publish_fp8",
                                          "indexer_topk", "indexer_topk_fp8", "indexer_topk_mxfp4", "sparse_mla_fp4",
                                          "comp_write_fp4", "sparse_mla_packed")}

    def sparse_mla(q, win_kv, chunk_kv, comp_kv, n_comp, attn_sink, idx, *a, **k):
        r = recs[layer[0]]
        r.update(q=q.clone(), kv=chunk_kv.clone(), sink=attn_sink.clone())
        o = orig["sparse_mla"](q, win_kv, chunk_kv, comp_kv, n_comp, attn_sink, idx, *a, **k)
        r["out"] = o.clone()
        layer[0] += 1
        return o

    def indexer_score(q, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q=q.clone(), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_score"](q, w_raw, w_scale, *a, **k)

    def sparse_mla_fp8(q, win_kv, chunk_kv, comp8, comp_scale, scale_rb, n_comp, attn_sink, idx, *a, **k):
        r = recs[layer[0]]
        r.update(q=q.clone(), kv=chunk_kv.clone(), sink=attn_sink.clone())
        o = orig["sparse_mla_fp8"](q, win_kv, chunk_kv, comp8, comp_scale, scale_rb, n_comp, attn_sink, idx, *a, **k)
        r["out"] = o.clone()
        layer[0] += 1
        return o

    def sparse_mla_fp4(q, win_kv, chunk_kv, comp4, n_comp, attn_sink, idx, *a, **k):
        r = recs[layer[0]]
        r.update(q=q.clone(), kv=chunk_kv.clone(), sink=attn_sink.clone())
        o = orig["sparse_mla_fp4"](q, win_kv, chunk_kv, comp4, n_comp, attn_sink, idx, *a, **k)
        r["out"] = o.clone()
        layer[0] += 1
        return o

    def sparse_mla_packed(q, win_kv8, chunk_kv, comp4, n_comp, attn_sink, idx, *a, **k):
        r = recs[layer[0]]
        r.update(q=q.clone(), kv=chunk_kv.clone(), sink=attn_sink.clone())
        o = orig["sparse_mla_packed"](q, win_kv8, chunk_kv, comp4, n_comp, attn_sink, idx, *a, **k)
        r["out"] = o.clone()
        layer[0] += 1
        return o

    def comp_write_fp4(latents, *a, **k):
        recs[layer[0]]["latent"] = latents.clone()
        return orig["comp_write_fp4"](latents, *a, **k)

    def indexer_topk(q, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q=q.clone(), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_topk"](q, w_raw, w_scale, *a, **k)

    def indexer_topk_mxfp4(q_mx, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q_mx=tuple(t.clone() for t in q_mx), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_topk_mxfp4"](q_mx, w_raw, w_scale, *a, **k)

    def indexer_topk_fp8(q, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q=q.clone(), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_topk_fp8"](q, w_raw, w_scale, *a, **k)

    def indexer_score_fp8(q, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q=q.clone(), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_score_fp8"](q, w_raw, w_scale, *a, **k)

    def comp_write_fp8(latents, *a, **k):
        recs[layer[0]]["latent"] = latents.clone()
        return orig["comp_write_fp8"](latents, *a, **k)

    def index_key_publish_fp8(k_raw, codes, scales, g0, ratio, norm_w, *a, **k):
        recs[layer[0]].update(k_raw=k_raw.clone(), k_norm=norm_w.clone())
        return orig["index_key_publish_fp8"](k_raw, codes, scales, g0, ratio, norm_w, *a, **k)

    def indexer_score_mxfp4(q_mx, w_raw, w_scale, *a, **k):
        recs[layer[0]].update(index_q_mx=tuple(t.clone() for t in q_mx), w_raw=w_raw.clone(), w_scale=w_scale)
        return orig["indexer_score_mxfp4"](q_mx, w_raw, w_scale, *a, **k)

    def index_key_publish_mxfp4(k_raw, k_codes, k_scales, g0, ratio, norm_w, *a, **k):
        recs[layer[0]].update(k_raw=k_raw.clone(), k_norm=norm_w.clone())
        return orig["index_key_publish_mxfp4"](k_raw, k_codes, k_scales, g0, ratio, norm_w, *a, **k)

    def comp_write(latents, *a, **k):
        recs[layer[0]]["latent"] = latents.clone()
        return orig["comp_write"](latents, *a, **k)

    def index_key_publish(k_raw, index_k, g0, ratio, norm_w, *a, **k):
        recs[layer[0]].update(k_raw=k_raw.clone(), k_norm=norm_w.clone())
        return orig["index_key_publish"](k_raw, index_k, g0, ratio, norm_w, *a, **k)

    for n, f in (("sparse_mla", sparse_mla), ("indexer_score", indexer_score), ("comp_write", comp_write),
                 ("index_key_publish", index_key_publish), ("indexer_score_mxfp4", indexer_score_mxfp4),
                 ("index_key_publish_mxfp4", index_key_publish_mxfp4), ("sparse_mla_fp8", sparse_mla_fp8),
                 ("indexer_score_fp8", indexer_score_fp8), ("comp_write_fp8", comp_write_fp8),
                 ("index_key_publish_fp8", index_key_publish_fp8), ("indexer_topk", indexer_topk),
                 ("indexer_topk_fp8", indexer_topk_fp8), ("indexer_topk_mxfp4", indexer_topk_mxfp4),
                 ("sparse_mla_fp4", sparse_mla_fp4), ("comp_write_fp4", comp_write_fp4),
                 ("sparse_mla_packed", sparse_mla_packed)):
        setattr(_abi, n, f)
    try:
        stack(h, cache)
    finally:
        for n, f in orig.items():
            setattr(_abi, n, f)
    assert layer[0] == len(stack.layers)
    return recs


@pytest.mark.parametrize("topology,index_format,T", [
    ("c4", "dense", 40), ("c4", "mxfp4", 40), ("c4", "fp8", 40), ("c4", "fp4", 40), ("c4", "packed", 40),
    ("release", "dense", 40), ("release", "dense", 39), ("release", "fp8", 40), ("release", "mxfp4", 39),
    ("release", "fp4", 39), ("release", "packed", 40)])
def test_stack_step_reproduces_attention_stack(gpu, topology, index_format, T):
    """Toy C4 topology (ratio 4) or the release's ratios (0,0,2,2,2,1,1,1) in bf16: T-1 prefill
    tokens, then the decode token at position T-1. At T = 40 it completes a group at every ratio
    (owners write a latent and a key); at T = 39 the ratio-2 group stays open (its compressor
    state carries) while the ratio-1 owner writes. Dense or MXFP4 index caches, the fp8 cache
    variant (fp8 compressed KV and index keys), the packed fp4 compressed KV with MXFP4 index
    keys ("fp4"), and that with an MXFP8 window ring ("packed"). The packed formats use the widths
    their kernels take (128-channel index keys; fp8 and fp4 latents of 512)."""
    from dsv41.model import AttentionStack
    from dsv41.step import StackDecodeStep
    base = C4_TOY if topology == "c4" else RELEASE_TOY
    # MXFP4 index caches: the fp4 MFMA kernels take 16/32/64 heads of 128 channels
    cfg = dict(base, index_head_dim=128, index_n_heads=16) if index_format == "mxfp4" else base
    if index_format in ("fp8", "fp4", "packed"):
        cfg = dict(base, index_head_dim=128, head_dim=512, rope_head_dim=64)
    if index_format in ("fp4", "packed"):
        cfg = dict(cfg, index_n_heads=16)
    a = args(cfg)
    st = AttentionStack(model_args(cfg), torch.bfloat16, gpu)
    load_stack(st, R.make_params(a, SEED_BASE + 40, "bf16"))
    rng = np.random.default_rng(SEED_BASE + 40)
    b = 2
    h = torch.from_numpy(rng.standard_normal((b, T, a.dim)).astype(F32)).to(gpu).to(torch.bfloat16)
    if index_format == "fp8":
        cache = st.make_cache(b, a.max_seq_len, cache_format="fp8")
    elif index_format in ("fp4", "packed"):
        cache = st.make_cache(b, a.max_seq_len, index_format="mxfp4", cache_format=index_format)
    else:
        cache = st.make_cache(b, a.max_seq_len, index_format=index_format)
    st(h[:, :T - 1], cache)
    before = _clone_cache(cache)
    recs = _record_decode(st, h[:, T - 1:], cache)
    step = StackDecodeStep(model_args(cfg), b, T - 1, torch.bfloat16, gpu)
    outs = step(before, recs)
    torch.cuda.synchronize()
    for l, (o, r) in enumerate(zip(outs, recs)):
        assert torch.equal(o, r["out"]), f"layer {l} output"
    from dsv41.cache import _BUFFERS
    for l, (g, w) in enumerate(zip(before.layers, cache.layers)):
        for name in _BUFFERS:
            x, y = getattr(g, name), getattr(w, name)
            assert (x is None) == (y is None)
            if x is not None:
                assert torch.equal(x, y), f"layer {l} {name}"
    # the candidate mask is live at this size: layers after the source use it, and it drops blocks
    if topology == "c4":
        assert step.plan[20].candidate_source and step.plan[24].uses_candidates
    else:
        assert step.plan[5].candidate_source and step.plan[7].uses_candidates
        assert [p.ratio for p in step.plan] == [0, 0, 2, 2, 2, 1, 1, 1]


def c4_args(**over):
    from dsv41.config import ModelArgs
    cfg = dict(n_layers=40, compress_ratios=(0, 0) + (4,) * 38, kv_source_layers=(2, 8, 14, 20),
               index_source_layers=(2, 8, 14, 20, 24, 28, 32, 36), candidate_source_layer=20,
               candidate_topk_blocks=2048, candidate_block_size=8, index_n_heads=64, index_head_dim=128,
               index_topk=512, window_size=128, n_heads=64, head_dim=512, rope_head_dim=64,
               compress_rope_theta=160000.0, original_seq_len=65536, rope_factor=16.0, max_seq_len=65536)
    cfg.update(over)
    return ModelArgs(**cfg)


def c4_inputs(a, b, gen, device):
    """Per-layer decode inputs of the C4 config: q / kv N(0,1)/sqrt(576) bf16, sinks N(0,1),
    index queries fp4-fake-quantized N(0,1), head weights N(0,1) bf16, owner latents and raw
    keys N(0,1)."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    s = 576 ** -0.5
    bf = torch.bfloat16
    H, D, Hi, Di = a.n_heads, a.head_dim, a.index_n_heads, a.index_head_dim
    rn = lambda *shape: torch.randn(*shape, generator=gen, device=device)   # noqa: E731
    ins = []
    for l in range(a.n_layers):
        x = dict(q=(rn(b, 1, H, D) * s).to(bf), kv=(rn(b, 1, D) * s).to(bf), sink=rn(H))
        if a.compress_ratio(l) and l in a.index_source_layers:
            x["index_q"] = _abi.fq_fp4_ue8m0(rn(b, 1, Hi, Di).to(bf))
            x["w_raw"] = rn(b, 1, Hi).to(bf)
            x["w_scale"] = weight_scale(Hi, Di, bf)
        if l in a.kv_source_layers:
            x["latent"] = rn(b, 1, D).to(bf)
            if l in a.index_source_layers:
                x["k_raw"] = rn(b, 1, Di).to(bf)
                x["k_norm"] = torch.ones(Di, device=device)
        ins.append(x)
    return ins


def c4_fill_cache(cache, gen):
    """Window rings and compressed caches N(0,1)/sqrt(576), index keys fp4-fake-quantized N(0,1)."""
    from dsv41 import _abi
    s = 576 ** -0.5
    for lc in cache.layers:
        for t in (lc.win_kv, lc.comp_kv):
            if t is not None:
                t.copy_(torch.randn(t.shape, generator=gen, device=t.device) * s)
        if lc.index_k is not None:
            lc.index_k.copy_(torch.randn(lc.index_k.shape, generator=gen, device=lc.index_k.device))
            _abi.fq_fp4_ue8m0(lc.index_k, out=lc.index_k)


def _oracle_layer_out(a, q_row, win_before, kv_row, comp_row, idx_row, sink, start_pos, ratio):
    """Oracle attention output of one batch row: q's rope tail (the step applies it as the
    attention loads q), attention over concat(window chrono, chunk, comp), then the inverse rope
    of the layer's table."""
    W = a.window_size
    wp = min(start_pos, W)
    slots = (start_pos - wp + np.arange(wp)) % W
    parts = [win_before[slots], kv_row]
    if comp_row is not None:
        parts.append(comp_row)
    kv_all = np.concatenate(parts, axis=0)[None]
    widx = R.window_idx_matrix(wp, 1, W)[None]
    full = widx if idx_row is None else np.concatenate([widx, idx_row[None, None]], -1)
    orig, theta = (a.original_seq_len, a.compress_rope_theta) if ratio else (0, a.rope_theta)
    rc, rs = R.precompute_freqs_cis(a.rope_head_dim, start_pos + 1, orig, theta, a.rope_factor, a.beta_fast,
                                    a.beta_slow)
    q = R.rope_tail(q_row[None, None], a.rope_head_dim, rc[[start_pos]], rs[[start_pos]], dtype="bf16")
    o = R.sparse_attn(q, kv_all, sink, full, a.head_dim ** -0.5, dtype="bf16")
    return R.rope_tail(o, a.rope_head_dim, rc[[start_pos]], rs[[start_pos]], inverse=True, dtype="bf16")[0, 0]


def test_c4_full_size_sampled_rows(gpu):
    from dsv41 import _abi
    from dsv41.cache import ModelCache
    from dsv41.step import StackDecodeStep
    a = c4_args()
    B, sp, r = 64, 65535, 4
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 4)
    cache = ModelCache(a, B, 65536, torch.bfloat16, gpu)
    c4_fill_cache(cache, gen)
    ins = c4_inputs(a, B, gen, gpu)
    rows = (0, 37, 63)
    layers = (0, 36, 39)
    win_before = {(l, b): to_np(cache.layers[l].win_kv[b]) for l in layers for b in rows}
    step = StackDecodeStep(a, B, sp, torch.bfloat16, gpu)
    outs = step(cache, ins)
    torch.cuda.synchronize()
    nb = (sp + 1) // r
    lens = R.query_lens(sp, 1, r)
    f = lambda t: t.float().cpu().numpy()   # noqa: E731
    # layer 36 selects with the fused indexer + top-k form, which writes no scores: its scores
    # come from indexer_score with the same inputs and the candidate mask layer 20 published
    assert step.plan[36].fused_idx is not None and step.candidates is not None
    got_s = to_np(_abi.indexer_score(ins[36]["index_q"], ins[36]["w_raw"], ins[36]["w_scale"],
                                     cache.layers[20].index_k[:B, :nb], sp, r, step.candidates))
    idx36 = step.plan[36].idx.cpu().numpy()
    for b in rows:
        keys20 = f(cache.layers[20].index_k[b, :nb])[None]
        w20 = R.cast(f(ins[20]["w_raw"][b:b + 1]) * F32(ins[20]["w_scale"]), "bf16")
        s20 = R.indexer_scores(f(ins[20]["index_q"][b:b + 1]), keys20, w20, sp, r)
        cand = R.select_candidate_blocks(s20, lens, a.candidate_topk_blocks, a.candidate_block_size)
        w36 = R.cast(f(ins[36]["w_raw"][b:b + 1]) * F32(ins[36]["w_scale"]), "bf16")
        want = R.indexer_scores(f(ins[36]["index_q"][b:b + 1]), keys20, w36, sp, r, cand)
        assert np.abs(got_s[b:b + 1] - want).max() <= 1e-5 * np.abs(want).max(), f"scores row {b}"
        want_i = R.topk_indices(got_s[b:b + 1], a.index_topk, lens, min(sp, a.window_size) + 1)
        assert np.array_equal(idx36[b:b + 1], want_i), f"top-k row {b}"
        comp20 = f(cache.layers[20].comp_kv[b, :nb])
        for l in layers:
            ratio = a.compress_ratio(l)
            o = _oracle_layer_out(a, f(ins[l]["q"][b, 0]), win_before[(l, b)], f(ins[l]["kv"][b]),
                                  comp20 if ratio else None, idx36[b, 0] if ratio else None, f(ins[l]["sink"]),
                                  sp, ratio)
            assert_attn_close(to_np(outs[l][b, 0]), o, f"layer {l} row {b}")


def test_stack_step_graph_replays(gpu):
    """The 40-layer step captured in a HIP graph: every replay, with eager work and host
    synchronizations between replays, reproduces the eager step bit for bit (outputs and the
    fused top-k of the last index source). Top-128 over 4,096 entries at B=16 takes the fused
    indexer + top-k form on every index source but the candidate source; the step's writes (ring
    slot, owner latent and key) store the same values on every replay."""
    from dsv41.cache import ModelCache
    from dsv41.step import StackDecodeStep
    a = c4_args(index_topk=128, candidate_topk_blocks=256, max_seq_len=16384)
    B, sp = 16, 16383
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 9)
    cache = ModelCache(a, B, 16384, torch.bfloat16, gpu)
    c4_fill_cache(cache, gen)
    ins = c4_inputs(a, B, gen, gpu)
    step = StackDecodeStep(a, B, sp, torch.bfloat16, gpu)
    assert sum(p.fused_idx is not None for p in step.plan) == 7
    want = [o.clone() for o in step(cache, ins)]
    want_idx = step.plan[36].idx.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(cache, ins)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step(cache, ins)
    for rep in range(3):
        for o in outs:
            o.zero_()
        step.plan[36].idx.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for l, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), (rep, l)
        assert torch.equal(step.plan[36].idx, want_idx), rep


@pytest.mark.parametrize("cache_format", ["dense", "fp8"])
def test_cache_snapshot_restore_replays_a_decode_step(gpu, cache_format):
    """The torch counterpart of generate.py's snapshot / retry: after 39 prefill tokens, snapshot
    the cache, run the decode token (it completes a group: owners write a latent and a key, every
    layer writes its ring slot and the compressor state moves), restore, and run the same token
    again: the same outputs, and the same cache afterwards."""
    from dsv41.cache import restore, snapshot
    from dsv41.model import AttentionStack
    cfg = C4_TOY if cache_format == "dense" else dict(C4_TOY, index_head_dim=128, head_dim=512, rope_head_dim=64)
    a = args(cfg)
    st = AttentionStack(model_args(cfg), torch.bfloat16, gpu)
    load_stack(st, R.make_params(a, SEED_BASE + 41, "bf16"))
    rng = np.random.default_rng(SEED_BASE + 41)
    b, T = 2, 40
    h = torch.from_numpy(rng.standard_normal((b, T, a.dim)).astype(F32)).to(gpu).to(torch.bfloat16)
    cache = st.make_cache(b, a.max_seq_len, cache_format=cache_format) if cache_format == "fp8" else \
        st.make_cache(b, a.max_seq_len)
    st(h[:, :T - 1], cache)
    snap = snapshot(cache)
    first = st(h[:, T - 1:], cache).clone()
    after = snapshot(cache)
    restore(cache, snap)
    second = st(h[:, T - 1:], cache)
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    assert cache.offset == after[0]
    for l, (lc, (bufs, state)) in enumerate(zip(cache.layers, after[1])):
        for name, t in bufs.items():
            assert torch.equal(getattr(lc, name), t), f"layer {l} {name}"
        if state is not None:
            assert torch.equal(lc.comp_state.kv_state, state[0]) and torch.equal(lc.comp_state.score_state,
                                                                                 state[1]), f"layer {l} state"


# Scores of the block-scaled fp4 x fp8 MFMA against the exact scores: the instruction sums its
# 128 exact products to a few 1e-5 of the result's magnitude (a one-wave probe on the box), so
# the scores carry that error; the dequantizing fp8 scorer is exact.
MXQ_FP8_TOL = 1e-4


def c5_fill_cache(cache, gen):
    """fp8 caches of 32 x 32 blocks: e4m3 codes uniform over the finite codes, ue8m0 block scales
    2^U{-4..4} (bytes 123..131); window rings N(0,1)/sqrt(576) bf16."""
    s = 576 ** -0.5
    for lc in cache.layers:
        lc.win_kv.copy_(torch.randn(lc.win_kv.shape, generator=gen, device=lc.win_kv.device) * s)
        for codes, scales in ((lc.comp_kv8, lc.comp_ks), (lc.index_k8, lc.index_k8s)):
            if codes is None:
                continue
            c = torch.randint(0, 256, codes.shape, generator=gen, device=codes.device, dtype=torch.int32)
            codes.copy_(torch.where((c & 0x7F) == 0x7F, c ^ 1, c).to(torch.uint8))
            scales.copy_(torch.randint(123, 132, scales.shape, generator=gen, device=scales.device,
                                       dtype=torch.int32).to(torch.uint8))


@pytest.mark.parametrize("scorer", ["exact", "mxq"])
def test_c5_fp8_block_cache_full_size_sampled_rows(gpu, scorer):
    """The fp8 40-layer decode step as the fp8 cache variant's configuration states it: batch 16,
    131,072-token context (32,768 compressed entries), top-1,024, compressed KV and index keys as
    e4m3 in 32 x 32 blocks with ue8m0 scales 2^-4..2^4, dequantized in-kernel. Sampled rows of a
    window-only layer, the candidate source (layer 20), the last index source (layer 36: its
    queries against layer 20's keys under layer 20's candidate mask, which keeps 2,048 of 4,096
    blocks) and a consumer (39) against the oracle on the dequantized caches.

    scorer "exact" (the default form: bf16 queries, keys dequantized in-kernel, exact products,
    fp32 sums): scores within 1e-5 max|S|, and the candidate mask and the top-k of layers 20 and
    36 bit-exact against the oracle's selection over the oracle's own fp32 scores (indexer.py:
    134-144), outputs within the bf16 attention check.
    scorer "mxq" (opt-in: MXFP4 queries on the block-scaled fp4 x fp8 MFMA, whose sums carry a few
    1e-5 max|S|): scores within MXQ_FP8_TOL max|S|, the selection bit-exact given its own scores,
    and against the exact scores it may differ only by swaps among entries within that error of
    the k-th score."""
    from dsv41 import _abi
    from dsv41.cache import ModelCache
    from dsv41.step import StackDecodeStep
    a = c4_args(index_topk=1024, max_seq_len=131072)
    B, sp, r = 16, 131071, 4
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 5)
    cache = ModelCache(a, B, 131072, torch.bfloat16, gpu, cache_format="fp8", fp8_block_rows=32)
    c5_fill_cache(cache, gen)
    ins = c4_inputs(a, B, gen, gpu)
    ident = (torch.ones(sp + 1, 32, device=gpu), torch.zeros(sp + 1, 32, device=gpu))
    if scorer == "mxq":
        for l, x in enumerate(ins):
            if "index_q" in x:                   # the same fp4 values in MXFP4 form
                x["index_q_mx"] = _abi.index_q_prep_mxfp4(x["index_q"], *ident, 64, sp)
    rows = (0, 9, 15)
    layers = (0, 36, 39)
    win_before = {(l, b): to_np(cache.layers[l].win_kv[b]) for l in layers for b in rows}
    step = StackDecodeStep(a, B, sp, torch.bfloat16, gpu)
    print(f"[c5] 40-layer fp8 step, B=16, nb=32768, scorer {scorer}", flush=True)
    outs = step(cache, ins)
    torch.cuda.synchronize()
    nb = (sp + 1) // r
    lens = R.query_lens(sp, 1, r)
    off = min(sp, a.window_size) + 1
    K = a.index_topk
    f = lambda t: t.float().cpu().numpy()   # noqa: E731
    l20 = cache.layers[20]
    assert l20.fp8_rb == 32 and step.candidates is not None
    if scorer == "mxq":
        tol = MXQ_FP8_TOL
        score = lambda l, cand=None: to_np(_abi.indexer_score_mxq_fp8(   # noqa: E731
            ins[l]["index_q_mx"], ins[l]["w_raw"], ins[l]["w_scale"], l20.index_k8[:B], l20.index_k8s[:B], 32, nb,
            sp, r, cand))
    else:
        tol = 1e-5
        score = lambda l, cand=None: to_np(_abi.indexer_score_fp8(   # noqa: E731
            ins[l]["index_q"], ins[l]["w_raw"], ins[l]["w_scale"], l20.index_k8[:B], l20.index_k8s[:B], 32, nb, sp,
            r, cand))
    # the scores the step's kernels formed (the same kernel on the same inputs gives the same bits)
    got20 = score(20)
    got_s = score(36, step.candidates)
    cand_gpu = step.candidates.cpu().numpy()
    idx20 = step.plan[20].idx.cpu().numpy()
    idx36 = step.plan[36].idx.cpu().numpy()
    swaps = 0
    for b in rows:
        keys20 = R.dequant_fp8_cache(l20.index_k8[b:b + 1].cpu().numpy(), l20.index_k8s[b:b + 1].cpu().numpy(),
                                     32)[:, :nb]
        w20 = R.cast(f(ins[20]["w_raw"][b:b + 1]) * F32(ins[20]["w_scale"]), "bf16")
        s20 = R.indexer_scores(f(ins[20]["index_q"][b:b + 1]), keys20, w20, sp, r)
        assert np.abs(got20[b:b + 1] - s20).max() <= tol * np.abs(s20).max(), f"layer 20 scores row {b}"
        # given the GPU's own scores the selection is always bit-exact
        cand_own = R.select_candidate_blocks(got20[b:b + 1], lens, a.candidate_topk_blocks, a.candidate_block_size)
        assert np.array_equal(cand_gpu[b:b + 1], cand_own), f"candidate mask row {b}"
        assert np.array_equal(idx20[b:b + 1], R.topk_indices(got20[b:b + 1], K, lens, off)), f"layer 20 top-k {b}"
        assert 0 < cand_own.mean() < 1                           # the mask is live
        cand = R.select_candidate_blocks(s20, lens, a.candidate_topk_blocks, a.candidate_block_size)
        w36 = R.cast(f(ins[36]["w_raw"][b:b + 1]) * F32(ins[36]["w_scale"]), "bf16")
        want = R.indexer_scores(f(ins[36]["index_q"][b:b + 1]), keys20, w36, sp, r, cand)
        fin = np.isfinite(want)
        if scorer == "exact":
            # the reference's rule on the oracle's exact fp32 scores, bit for bit
            assert np.array_equal(cand_gpu[b:b + 1], cand), f"candidate mask vs exact scores row {b}"
            assert np.array_equal(idx20[b:b + 1], R.topk_indices(s20, K, lens, off)), f"layer 20 exact top-k {b}"
        assert np.array_equal(np.isfinite(got_s[b:b + 1]), np.isfinite(R.indexer_scores(
            f(ins[36]["index_q"][b:b + 1]), keys20, w36, sp, r, cand_own))), f"mask row {b}"
        if np.array_equal(cand_own, cand):
            assert np.abs(got_s[b:b + 1][fin] - want[fin]).max() <= tol * np.abs(want[fin]).max(), f"scores row {b}"
        assert np.array_equal(idx36[b:b + 1], R.topk_indices(got_s[b:b + 1], K, lens, off)), f"top-k row {b}"
        want_i = R.topk_indices(want, K, lens, off)
        if scorer == "exact":
            assert np.array_equal(idx36[b:b + 1], want_i), f"layer 36 exact top-k row {b}"
        else:
            got_pos = idx36[b, 0][idx36[b, 0] >= 0] - off
            want_pos = want_i[0, 0][want_i[0, 0] >= 0] - off
            diff = np.setxor1d(got_pos, want_pos)
            if diff.size:
                kth = np.sort(want[0, 0][fin[0, 0]])[::-1][K - 1]
                band = tol * np.abs(want[fin]).max()
                assert np.all(np.abs(want[0, 0][diff] - kth) <= 2 * band), f"layer 36 swaps beyond the error, row {b}"
            swaps += diff.size // 2
        comp20 = R.dequant_fp8_cache(l20.comp_kv8[b:b + 1].cpu().numpy(), l20.comp_ks[b:b + 1].cpu().numpy(),
                                     32)[0, :nb]
        for l in layers:
            ratio = a.compress_ratio(l)
            o = _oracle_layer_out(a, f(ins[l]["q"][b, 0]), win_before[(l, b)], f(ins[l]["kv"][b]),
                                  comp20 if ratio else None, idx36[b, 0] if ratio else None, f(ins[l]["sink"]),
                                  sp, ratio)
            assert_attn_close(to_np(outs[l][b, 0]), o, f"layer {l} row {b}")
    print(f"[c5] scorer {scorer}: {swaps} top-k swaps against the exact scores over {len(rows)} rows", flush=True)
