"""Layer- and stack-level parity of the dsv41 path against the oracle, plus the C2 decode step.

* C1 (tiny fp32, 4 layers, 128-token prefill then 16 decode steps): QAT simulation off on
  both sides at 1e-5 max-abs (the strict pass), on at 5e-3 relative (the reference's own
  threshold for the QAT-on pass, tests/test_parity.py:721-722: midpoint flips).
* TOPO (every sharing role incl. candidates, ring wraps): the same two passes, GPU decode vs
  GPU prefill tail, chunked vs single forward, and the negative controls of
  tests/test_parity.py:736-760 (broken sink / rope inverse / sharing must move the output).
* C2 (bf16, batch 32, 4096 compressed entries, top-512, 64 heads x 512): the decode step --
  scores within 1e-5 of the float32 contraction, top-k bit-exact given those scores,
  attention output within the bf16 attention check (2e-2 relative plus per-head bounds).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from common import (C1, RELEASE_TOY, SEED_BASE, TOPO, args, assert_attn_close, load_stack, max_abs, model_args,
                    rel_max_diff, to_np)
from oracle import cpu_ref as R

pytestmark = pytest.mark.gpu
F32 = np.float32


def _stacks(cfg, dt, seed, device):
    from dsv41.model import AttentionStack
    a = args(cfg)
    params = R.make_params(a, seed, dt)
    st = AttentionStack(model_args(cfg), {"f32": torch.float32, "bf16": torch.bfloat16}[dt], device)
    load_stack(st, params)
    return a, st, R.AttentionStack(a, params, dt)


def _qat(enabled: bool):
    import dsv41.fakequant as FQ
    FQ.DISABLE = not enabled
    R.DISABLE_FAKE_QUANT = not enabled


@pytest.fixture
def qat_restore():
    yield
    _qat(True)


def _run(model, h, cache, splits, to_dev):
    """Feed h[:, s:e] chunk by chunk; to_dev=None runs the oracle on numpy arrays."""
    outs = []
    for s, e in splits:
        chunk = np.ascontiguousarray(h[:, s:e])
        outs.append(to_np(model(to_dev(chunk), cache)) if to_dev is not None else model(chunk, cache))
    return np.concatenate(outs, axis=1)


@pytest.mark.parametrize("qat", [False, True], ids=["qat-off", "qat-on"])
def test_c1_prefill_then_decode(gpu, qat, qat_restore):
    _qat(qat)
    a, st, ost = _stacks(C1, "f32", SEED_BASE, gpu)
    rng = np.random.default_rng(SEED_BASE)
    T = 128 + 16
    h = rng.standard_normal((1, T, a.dim)).astype(F32)
    splits = [(0, 128)] + [(t, t + 1) for t in range(128, T)]
    want = _run(ost, h, R.ModelCache(a, 1, a.max_seq_len), splits, None)
    got = _run(st, h, st.make_cache(1, a.max_seq_len), splits, lambda x: torch.from_numpy(x).to(gpu))
    if qat:
        assert rel_max_diff(got, want) < 5e-3
    else:
        assert max_abs(got, want) < 1e-5, f"max abs {max_abs(got, want):.3e}"


@pytest.mark.parametrize("topology", ["topo", "release"])
@pytest.mark.parametrize("qat", [False, True], ids=["qat-off", "qat-on"])
def test_topology_battery(gpu, qat, topology, qat_restore):
    """TOPO (ratio 4, every sharing role) or the release's ratios (0,0,2,2,2,1,1,1): ratio-2
    pooling with remainders carried across odd chunk cuts, and the ratio-1 compressor branch,
    writes and key publishes at every position."""
    _qat(qat)
    cfg = TOPO if topology == "topo" else RELEASE_TOY
    a, st, ost = _stacks(cfg, "f32", SEED_BASE + 3, gpu)
    rng = np.random.default_rng(SEED_BASE + 3)
    T = 40
    h = rng.standard_normal((2, T, a.dim)).astype(F32)
    dev = lambda x: torch.from_numpy(x).to(gpu)   # noqa: E731
    full_o = _run(ost, h, R.ModelCache(a, 2, a.max_seq_len), [(0, T)], None)
    full_g = _run(st, h, st.make_cache(2, a.max_seq_len), [(0, T)], dev)
    dec = [(0, 32)] + [(t, t + 1) for t in range(32, T)]
    dec_g = _run(st, h, st.make_cache(2, a.max_seq_len), dec, dev)
    chunks = [(0, 13), (13, 14), (14, 27), (27, 31), (31, T)]
    chk_g = _run(st, h, st.make_cache(2, a.max_seq_len), chunks, dev)
    if qat:
        tol = lambda g, w: rel_max_diff(g, w) < 5e-3          # noqa: E731
    elif topology == "topo":
        tol = lambda g, w: max_abs(g, w) < 1e-5                # noqa: E731
    else:   # 8 residual layers: outputs reach |h| ~ 5, so the fp32 bar is relative
        tol = lambda g, w: rel_max_diff(g, w) < 1e-5           # noqa: E731
    assert tol(full_g, full_o), f"prefill vs oracle {max_abs(full_g, full_o):.3e}"
    assert tol(dec_g, full_o), f"decode vs oracle prefill {max_abs(dec_g, full_o):.3e}"
    assert tol(chk_g, full_o), f"chunked vs oracle {max_abs(chk_g, full_o):.3e}"


@pytest.mark.parametrize("cache_format", ["fp4", "packed"])
def test_packed_cache_stack_equals_dense_cache(gpu, cache_format):
    """The release topology in bf16 (512-channel latents) over a packed fp4 compressed cache
    ("fp4") and also an MXFP8 window ring ("packed"): every output of a chunked prefill and the
    decode steps after it is bit-identical to the run over the dense cache, each owner's packed
    rows decode to its dense rows and each packed ring to the dense ring (the packed forms are
    lossless for the QAT values attention.py:120-122 and 157-163 store)."""
    cfg = dict(RELEASE_TOY, head_dim=512, rope_head_dim=64, index_head_dim=128)
    a, st, _ = _stacks(cfg, "bf16", SEED_BASE + 6, gpu)
    rng = np.random.default_rng(SEED_BASE + 6)
    T = 44
    h = rng.standard_normal((2, T, a.dim)).astype(F32)
    dev = lambda x: torch.from_numpy(x).to(gpu).to(torch.bfloat16)   # noqa: E731
    splits = [(0, 17), (17, 30)] + [(t, t + 1) for t in range(30, T)]
    c16 = st.make_cache(2, a.max_seq_len)
    c4 = st.make_cache(2, a.max_seq_len, cache_format=cache_format)
    o16 = _run(st, h, c16, splits, dev)
    o4 = _run(st, h, c4, splits, dev)
    assert np.array_equal(o4.view(np.uint32), o16.view(np.uint32))
    for l in a.kv_source_layers:
        n = T // a.compress_ratios[l]
        assert c4.layers[l].comp_kv is None and c16.layers[l].comp_kv4 is None
        got = R.fp4_e4m3_decode(c4.layers[l].comp_kv4[:, :n].cpu().numpy())
        assert np.array_equal(got.view(np.uint32), to_np(c16.layers[l].comp_kv[:, :n]).view(np.uint32)), l
    for l, (lp, ld) in enumerate(zip(c4.layers, c16.layers)):
        if cache_format == "packed":
            assert lp.win_kv is None
            got = R.mxfp8_decode(lp.win_kv8.cpu().numpy())
            assert np.array_equal(got.view(np.uint32), to_np(ld.win_kv).view(np.uint32)), l
        else:
            assert lp.win_kv8 is None and torch.equal(lp.win_kv, ld.win_kv)


@pytest.mark.parametrize("topology", ["topo", "release"])
@pytest.mark.parametrize("qat", [False, True], ids=["qat-off", "qat-on"])
def test_bf16_stack_over_default_fp32_cache(gpu, topology, qat, qat_restore):
    """The reference's default cache dtype under a bf16 model: ModelCache(args, bsz, max_seq_len)
    holds fp32 buffers (cache.py:29, 72; stream.py:71 builds it so) and the layer converts at
    every cache boundary (attention.py:127, 163, 166; cache.py:67). A chunked prefill with odd
    cuts and decode steps past the ring wrap give outputs bit-identical to the run over bf16
    caches, and every fp32 buffer holds the bf16 run's values exactly (a bf16 value widens
    exactly, so both runs read the same numbers)."""
    from dsv41.cache import ModelCache
    _qat(qat)
    cfg = TOPO if topology == "topo" else RELEASE_TOY
    a, st, _ = _stacks(cfg, "bf16", SEED_BASE + 7, gpu)
    rng = np.random.default_rng(SEED_BASE + 7)
    T = 40
    h = rng.standard_normal((2, T, a.dim)).astype(F32)
    dev = lambda x: torch.from_numpy(x).to(gpu).to(torch.bfloat16)   # noqa: E731
    splits = [(0, 13), (13, 27)] + [(t, t + 1) for t in range(27, T)]
    c32 = ModelCache(model_args(cfg), 2, a.max_seq_len, device=gpu)
    c16 = st.make_cache(2, a.max_seq_len)
    assert c32.layers[0].win_kv.dtype == torch.float32 and c16.layers[0].win_kv.dtype == torch.bfloat16
    o16 = _run(st, h, c16, splits, dev)
    o32 = _run(st, h, c32, splits, dev)
    assert np.array_equal(o32.view(np.uint32), o16.view(np.uint32))
    checked = 0
    for l, (w, n) in enumerate(zip(c32.layers, c16.layers)):
        for name in ("win_kv", "comp_kv", "index_k"):
            x, y = getattr(w, name), getattr(n, name)
            assert (x is None) == (y is None), (l, name)
            if x is not None:
                assert x.dtype == torch.float32 and torch.equal(x, y.float()), (l, name)
                checked += 1
        if w.comp_state is not None:
            assert torch.equal(w.comp_state.kv_state, n.comp_state.kv_state)
            assert torch.equal(w.comp_state.score_state, n.comp_state.score_state)
    assert checked >= len(c32.layers) + 2 * len(a.kv_source_layers) - 1


def test_negative_controls_move_the_output(gpu):
    a, st, _ = _stacks(TOPO, "f32", SEED_BASE + 4, gpu)
    rng = np.random.default_rng(SEED_BASE + 4)
    h = torch.from_numpy(rng.standard_normal((2, 30, a.dim)).astype(F32)).to(gpu)
    base = to_np(st(h, st.make_cache(2, a.max_seq_len)))

    def broken(setup, teardown):
        setup()
        try:
            return rel_max_diff(to_np(st(h, st.make_cache(2, a.max_seq_len))), base)
        finally:
            teardown()

    for attr in ("_break_sink", "_break_rope_inverse"):
        d = broken(lambda: [setattr(l, attr, True) for l in st.layers],
                   lambda: [setattr(l, attr, False) for l in st.layers])
        assert d > 1e-3, attr
    d = broken(lambda: setattr(st, "_break_sharing", True), lambda: setattr(st, "_break_sharing", False))
    assert d > 1e-3
    assert max_abs(to_np(st(h, st.make_cache(2, a.max_seq_len))), base) == 0.0


def c2_inputs(nb=4096, start=16384, seed=SEED_BASE + 1, b=32):
    """C2: batch 32, 16,384-token context -> 4,096 compressed entries, 64 heads x 512 (rope 64),
    indexer 64 x 128, top-512, window 128. Cache and queries N(0,1)/sqrt(576); sinks N(0,1);
    index queries/keys are fp4 fake-quantized N(0,1), head weights N(0,1) in bf16. Drawn in
    this fixed order from one seeded CPU generator."""
    g = torch.Generator("cpu").manual_seed(seed)
    H, D, Hi, Di, W = 64, 512, 64, 128, 128
    s = 576 ** -0.5
    t = {}
    t["q"] = (torch.randn(b, 1, H, D, generator=g) * s).to(torch.bfloat16)
    t["win"] = (torch.randn(b, W, D, generator=g) * s).to(torch.bfloat16)
    t["chunk"] = (torch.randn(b, 1, D, generator=g) * s).to(torch.bfloat16)
    t["comp"] = (torch.randn(b, nb, D, generator=g) * s).to(torch.bfloat16)
    t["iq"] = torch.from_numpy(R.fq_fp4_ue8m0(torch.randn(b, 1, Hi, Di, generator=g).numpy(), 32, "bf16")).to(torch.bfloat16)
    t["ik"] = torch.from_numpy(R.fq_fp4_ue8m0(torch.randn(b, nb, Di, generator=g).numpy(), 32, "bf16")).to(torch.bfloat16)
    t["w"] = torch.randn(b, 1, Hi, generator=g).to(torch.bfloat16)
    t["sink"] = torch.randn(H, generator=g)
    return t, dict(H=H, D=D, Hi=Hi, Di=Di, W=W, nb=nb, start=start, K=512, rd=64, r=4)


def test_c2_decode_step(gpu):
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis
    from dsv41.step import SparseDecodeStep
    t, c = c2_inputs()
    b = t["q"].shape[0]
    d = {k: v.to(gpu) for k, v in t.items()}
    cos, sin = precompute_freqs_cis(c["rd"], c["start"] + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    step = SparseDecodeStep(b, c["H"], c["D"], c["rd"], c["Hi"], c["Di"], c["nb"], c["K"], c["W"], c["start"],
                            c["r"], torch.bfloat16, gpu, fused=False)     # two calls: the scores are kept
    ws = weight_scale(c["Hi"], c["Di"], torch.bfloat16)
    out, idx = step(d["q"], d["iq"], d["w"], ws, d["ik"], d["comp"], d["win"], d["chunk"], d["sink"], cos, sin)
    torch.cuda.synchronize()
    f = lambda x: x.float().numpy()   # noqa: E731
    # scores
    w = R.cast(f(t["w"]) * np.float32(ws), "bf16")
    want_s = R.indexer_scores(f(t["iq"]), f(t["ik"]), w, c["start"], c["r"])
    got_s = to_np(step.scores)
    assert np.abs(got_s - want_s).max() <= 1e-5 * np.abs(want_s).max()
    # top-k bit-exact given the GPU's scores
    lens = R.query_lens(c["start"], 1, c["r"])
    wp = min(c["start"], c["W"])
    want_i = R.topk_indices(got_s, c["K"], lens, wp + 1)
    assert np.array_equal(idx.cpu().numpy(), want_i)
    # attention over concat(window, chunk, comp) with the reference's index layout
    slots = (c["start"] - wp + np.arange(wp)) % c["W"]
    kv_all = np.concatenate([f(t["win"])[:, slots], f(t["chunk"]), f(t["comp"])], axis=1)
    widx = np.broadcast_to(R.window_idx_matrix(wp, 1, c["W"])[None], (b, 1, min(c["W"], wp + 1)))
    rc, rs = R.precompute_freqs_cis(c["rd"], c["start"] + 1, 65536, 160000.0, 16.0, 32, 1)
    qr = R.rope_tail(f(t["q"]), c["rd"], rc[[c["start"]]], rs[[c["start"]]], dtype="bf16")   # q's rope, in-launch
    o = R.sparse_attn(qr, kv_all, f(t["sink"]), np.concatenate([widx, want_i], -1), c["D"] ** -0.5, dtype="bf16")
    want_o = R.rope_tail(o, c["rd"], rc[[c["start"]]], rs[[c["start"]]], inverse=True, dtype="bf16")
    assert_attn_close(to_np(out), want_o)


def test_bs32_ctx64k_decode_step_sampled_rows(gpu):
    """The bench's decode workload at full size (batch 32, 65,536 tokens -> 16,384 compressed
    entries, top-512, window 128), through the fused step the bench times: sampled batch rows
    against the oracle -- scores (two-call form) within 1e-5 of max |S|, the fused selection
    bit-exact to the oracle's top-k of the GPU scores, attention within the bf16 attention check."""
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis
    from dsv41.step import SparseDecodeStep
    b, nb, start, K = 32, 16384, 65536, 512
    H, D, Hi, Di, W, rd, r = 64, 512, 64, 128, 128, 64, 4
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 64)
    rn = lambda *s: torch.randn(*s, generator=g, device=gpu)   # noqa: E731
    sc = 576 ** -0.5
    # index queries and keys on the e2m1 grid times 1/4, as the fp4 index cache holds them
    grid = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], device=gpu) * 0.25
    fp4 = lambda *s: grid[torch.randint(0, 16, s, generator=g, device=gpu)].bfloat16()   # noqa: E731
    q, win, chunk = (rn(b, 1, H, D) * sc).bfloat16(), (rn(b, W, D) * sc).bfloat16(), (rn(b, 1, D) * sc).bfloat16()
    comp = (rn(b, nb, D) * sc).bfloat16()
    iq, ik = fp4(b, 1, Hi, Di), fp4(b, nb, Di)
    w, sink = rn(b, 1, Hi).bfloat16(), rn(H)
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    ws = weight_scale(Hi, Di, torch.bfloat16)
    fused = SparseDecodeStep(b, H, D, rd, Hi, Di, nb, K, W, start, r, torch.bfloat16, gpu)
    two = SparseDecodeStep(b, H, D, rd, Hi, Di, nb, K, W, start, r, torch.bfloat16, gpu, fused=False)
    assert fused.fused
    out, idx = fused(q, iq, w, ws, ik, comp, win, chunk, sink, cos, sin)
    two(q, iq, w, ws, ik, comp, win, chunk, sink, cos, sin)
    torch.cuda.synchronize()
    rows = [0, 13, 31]
    f = lambda x: x[rows].float().cpu().numpy()   # noqa: E731
    wq = R.cast(f(w) * np.float32(ws), "bf16")
    want_s = R.indexer_scores(f(iq), f(ik), wq, start, r)
    got_s = to_np(two.scores)[rows]
    assert np.abs(got_s - want_s).max() <= 1e-5 * np.abs(want_s).max()
    wp = min(start, W)
    want_i = R.topk_indices(got_s, K, R.query_lens(start, 1, r), wp + 1)
    assert np.array_equal(idx.cpu().numpy()[rows], want_i)
    slots = (start - wp + np.arange(wp)) % W
    kv_all = np.concatenate([f(win)[:, slots], f(chunk), f(comp)], axis=1)
    widx = np.broadcast_to(R.window_idx_matrix(wp, 1, W)[None], (len(rows), 1, min(W, wp + 1)))
    rc, rs = R.precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1)
    qr = R.rope_tail(f(q), rd, rc[[start]], rs[[start]], dtype="bf16")
    o = R.sparse_attn(qr, kv_all, sink.cpu().numpy(), np.concatenate([widx, want_i], -1), D ** -0.5, dtype="bf16")
    want_o = R.rope_tail(o, rd, rc[[start]], rs[[start]], inverse=True, dtype="bf16")
    assert_attn_close(to_np(out)[rows], want_o)


@pytest.mark.parametrize("b,nb,K,start", [
    (32, 16384, 512, 65535),     # bs32, 64K context: 8 row ranges of 2048 per query
    (64, 16384, 512, 65535),     # B=64: 4 ranges of 4096
    (32, 4096, 128, 16386),      # ranges of 512, top-128; 3 tokens of the next group still open
    (16, 32768, 512, 131071),    # 16 ranges of 2048: a merge over 8,192 candidates per query
    (256, 8192, 128, 32767),     # 512 (query, head group) units: the attention's unsplit plan
])
def test_decode_step_fused_equals_two_calls(gpu, b, nb, K, start):
    """The decode step with the fused indexer + top-k form selects exactly what indexer_score +
    topk_select select, so its attention output is bit-equal as well."""
    from dsv41.layers import precompute_freqs_cis
    from dsv41.step import SparseDecodeStep
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 41)
    H, D, Hi, Di, W, rd, r = 64, 512, 64, 128, 128, 64, 4
    rn = lambda *s: torch.randn(*s, generator=g, device=gpu)   # noqa: E731
    sc = 576 ** -0.5
    q, win, chunk = (rn(b, 1, H, D) * sc).bfloat16(), (rn(b, W, D) * sc).bfloat16(), (rn(b, 1, D) * sc).bfloat16()
    comp = (rn(b, nb, D) * sc).bfloat16()
    iq, ik, w, sink = rn(b, 1, Hi, Di).bfloat16(), rn(b, nb, Di).bfloat16(), rn(b, 1, Hi).bfloat16(), rn(H)
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    fused = SparseDecodeStep(b, H, D, rd, Hi, Di, nb, K, W, start, r, torch.bfloat16, gpu)
    two = SparseDecodeStep(b, H, D, rd, Hi, Di, nb, K, W, start, r, torch.bfloat16, gpu, fused=False)
    assert fused.fused and not two.fused
    o1, i1 = fused(q, iq, w, 0.01, ik, comp, win, chunk, sink, cos, sin)
    o2, i2 = two(q, iq, w, 0.01, ik, comp, win, chunk, sink, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2)
    assert torch.equal(o1, o2)


def test_decode_step_graph_replays(gpu):
    """The bs32 / 64K decode step (fused indexer + top-k, sparse MLA with its split combine)
    captured in a HIP graph over two input sets: every replay, with eager work and host
    synchronizations between replays, equals the eager step bit for bit."""
    from dsv41.layers import precompute_freqs_cis
    from dsv41.step import SparseDecodeStep
    b, nb, K, start = 32, 16384, 512, 65535
    H, D, Hi, Di, W, rd, r = 64, 512, 64, 128, 128, 64, 4
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 42)
    rn = lambda *s: torch.randn(*s, generator=g, device=gpu)   # noqa: E731
    sc = 576 ** -0.5
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    sets, steps = [], []
    for _ in range(2):
        sets.append(dict(q=(rn(b, 1, H, D) * sc).bfloat16(), win=(rn(b, W, D) * sc).bfloat16(),
                         chunk=(rn(b, 1, D) * sc).bfloat16(), comp=(rn(b, nb, D) * sc).bfloat16(),
                         iq=rn(b, 1, Hi, Di).bfloat16(), ik=rn(b, nb, Di).bfloat16(), w=rn(b, 1, Hi).bfloat16(),
                         sink=rn(H)))
        steps.append(SparseDecodeStep(b, H, D, rd, Hi, Di, nb, K, W, start, r, torch.bfloat16, gpu))

    def run(i):
        d = sets[i]
        return steps[i](d["q"], d["iq"], d["w"], 0.01, d["ik"], d["comp"], d["win"], d["chunk"], d["sink"], cos, sin)

    want = [tuple(t.clone() for t in run(i)) for i in range(2)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(0)
        run(1)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = [run(0), run(1)]
    for rep in range(3):
        for st in steps:
            st.out.zero_()
            st.idx.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i in range(2):
            assert steps[i].fused
            assert torch.equal(got[i][1], want[i][1]), (rep, i)
            assert torch.equal(got[i][0], want[i][0]), (rep, i)
