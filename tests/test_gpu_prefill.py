"""Chunked causal prefill at full size through the HIP path (the prefill plans of the indexer,
top-k and sparse-MLA kernels), checked against the oracle on sampled query rows and through
size-independent properties on every row.

* C3: B=1, an 8,192-token chunk after 32,768 tokens (nb = 10,240 compressed entries at ratio 4),
  64 heads x 512 (rope 64), indexer 64 x 128, top-2,048, window 128: 2,176-entry lists per
  query. Sampled rows: scores within 1e-5 of max |S|, top-k bit-exact given those scores,
  attention output within the bf16 attention check (2e-2 relative plus per-head bounds). Every row: the selection is a valid top-2,048 of its
  scores (no unselected visible score above a selected one), ascending, offset, in range.
* The longest list one prefill workgroup stages: 512 queries whose lists hold exactly 2,304
  entries (128 window rows + top-2,176), some of them masked (-1).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from common import SEED_BASE, assert_attn_close, to_np
from oracle import cpu_ref as R

pytestmark = pytest.mark.gpu
F32 = np.float32

H, D, RD, HI, DI, W, RATIO = 64, 512, 64, 64, 128, 128, 4
YARN = (65536, 160000.0, 16.0, 32, 1)      # original_seq_len, theta, factor, beta_fast, beta_slow


def _inputs(gen, device, n, prior, nb):
    """q / chunk / window ring / compressed cache N(0,1)/sqrt(576) bf16; index queries and keys
    fp4-fake-quantized N(0,1) (the values indexer.py:100-104, 119-121 store); head weights N(0,1)
    bf16; sinks N(0,1). Drawn in this order from one seeded generator on the GPU."""
    from dsv41 import _abi
    s = 576 ** -0.5
    bf = torch.bfloat16
    rn = lambda *shape: torch.randn(*shape, generator=gen, device=device)   # noqa: E731
    t = dict(q=(rn(1, n, H, D) * s).to(bf), chunk=(rn(1, n, D) * s).to(bf), win=(rn(1, W, D) * s).to(bf),
             comp=(rn(1, nb, D) * s).to(bf))
    t["iq"] = _abi.fq_fp4_ue8m0(rn(1, n, HI, DI).to(bf))
    t["ik"] = _abi.fq_fp4_ue8m0(rn(1, nb, DI).to(bf))
    t["w"] = rn(1, n, HI).to(bf)
    t["sink"] = rn(H)
    return t


def _oracle_rows(t, rows, idx_rows, n, prior):
    """Oracle attention output of the sampled query rows of batch 0: the kv sources in the
    reference's layout concat(window chrono, chunk, compressed) and each row's index list
    (window part from window_idx_matrix, then its top-k), inverse rope at its position."""
    f = lambda x: x.float().cpu().numpy()   # noqa: E731
    wp = min(prior, W)
    slots = (prior - wp + np.arange(wp)) % W
    kv_all = np.concatenate([f(t["win"][0])[slots], f(t["chunk"][0]), f(t["comp"][0])], axis=0)[None]
    widx = R.window_idx_matrix(wp, n, W)
    end = prior + n
    rc, rs = R.precompute_freqs_cis(RD, end, *YARN)
    q = f(t["q"][0])
    sink = f(t["sink"])
    out = {}
    for s, ir in zip(rows, idx_rows):
        full = np.concatenate([widx[s], ir])[None, None].astype(np.int32)
        o = R.sparse_attn(q[s][None, None], kv_all, sink, full, D ** -0.5, dtype="bf16")
        p = prior + s
        out[s] = R.rope_tail(o, RD, rc[[p]], rs[[p]], inverse=True, dtype="bf16")[0, 0]
    return out


def test_c3_chunked_prefill_full_size(gpu):
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis
    n, prior, K = 8192, 32768, 2048
    end = prior + n
    nb = end // RATIO
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 3)
    t = _inputs(gen, gpu, n, prior, nb)
    ws = weight_scale(HI, DI, torch.bfloat16)
    cos, sin = precompute_freqs_cis(RD, end, *YARN, device=gpu)
    offset = min(prior, W) + n

    print("[c3] indexer_score n=8192 nb=10240", flush=True)
    scores = _abi.indexer_score(t["iq"], t["w"], ws, t["ik"], prior, RATIO)
    print("[c3] topk_select k=2048", flush=True)
    idx = _abi.topk_select(scores, K, prior, RATIO, offset)
    print("[c3] sparse_mla 2176-entry lists", flush=True)
    out = _abi.sparse_mla(t["q"], t["win"], t["chunk"], t["comp"], nb, t["sink"], idx, D ** -0.5, W, prior,
                          cos, sin, RD)
    torch.cuda.synchronize()
    assert _abi.mla_workspace_bytes(1, n, H, D, W + K, torch.bfloat16) == 0     # the prefill plan, no split

    # ---- every row: a valid top-K of its own scores, ascending, offset, inside visibility
    lens = (prior + torch.arange(n, device=gpu) + 1) // RATIO                    # [n]
    assert (lens >= K).all()                                                     # no row runs short
    sel = idx[0].long() - offset                                                 # [n, K]
    assert (sel >= 0).all() and (sel < lens[:, None]).all()
    assert (sel[:, 1:] > sel[:, :-1]).all()
    s0 = scores[0]
    chosen = torch.zeros_like(s0, dtype=torch.bool).scatter_(1, sel, True)
    min_sel = torch.where(chosen, s0, torch.full_like(s0, float("inf"))).amin(1)
    max_rest = torch.where(chosen, torch.full_like(s0, float("-inf")), s0).amax(1)
    assert (min_sel >= max_rest).all(), "an unselected score beats a selected one"
    vis = torch.arange(nb, device=gpu)[None, :] < lens[:, None]
    assert torch.isfinite(s0[vis]).all() and torch.isneginf(s0[~vis]).all()
    assert torch.isfinite(out.float()).all()

    # ---- sampled rows against the oracle
    rows = (0, 1, 2047, 4096, 6143, 8190, 8191)
    f = lambda x: x.float().cpu().numpy()   # noqa: E731
    ik = f(t["ik"])
    got_s = to_np(scores[0, list(rows)])
    want_i = []
    for j, s in enumerate(rows):
        w = R.cast(f(t["w"][:, s:s + 1]) * F32(ws), "bf16")
        want = R.indexer_scores(f(t["iq"][:, s:s + 1]), ik, w, prior + s, RATIO)[0, 0]
        vis = np.isfinite(want)                          # entries past visibility are -inf on both
        assert np.array_equal(np.isneginf(got_s[j]), ~vis), f"visibility row {s}"
        assert np.abs(got_s[j][vis] - want[vis]).max() <= 1e-5 * np.abs(want[vis]).max(), f"scores row {s}"
        lens_s = R.query_lens(prior + s, 1, RATIO)
        wi = R.topk_indices(got_s[j][None, None], K, lens_s, offset)[0, 0]
        assert np.array_equal(idx[0, s].cpu().numpy(), wi), f"top-k row {s}"
        want_i.append(wi)
    want_o = _oracle_rows(t, rows, want_i, n, prior)
    for s in rows:
        assert_attn_close(to_np(out[0, s]), want_o[s], f"output row {s}")


def test_prefill_lists_at_the_workgroup_limit(gpu):
    """512 queries (the prefill plan: one 64-head workgroup per query, no split) whose lists hold
    exactly 2,304 entries, the most one workgroup stages: the 128-row window and a top-2,176
    selection of random scores, which also selects entries past each query's visibility (those
    become -1, masked)."""
    from dsv41 import _abi
    from dsv41.layers import precompute_freqs_cis
    n, prior, K = 512, 32768, 2176
    end = prior + n
    nb = end // RATIO
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 5)
    t = _inputs(gen, gpu, n, prior, nb)
    cos, sin = precompute_freqs_cis(RD, end, *YARN, device=gpu)
    offset = min(prior, W) + n
    assert min(W, min(prior, W) + n) + K == 2304
    assert _abi.mla_workspace_bytes(1, n, H, D, 2304, torch.bfloat16) == 0
    # scores that favour the newest entries, so rows near the chunk start select past their
    # visibility (-1 after masking) while later rows see them
    sc = torch.randn(1, n, nb, generator=gen, device=gpu) + torch.linspace(0, 3, nb, device=gpu)
    idx = _abi.topk_select(sc, K, prior, RATIO, offset)
    print("[kmax] sparse_mla 512 queries x 2304 entries", flush=True)
    out = _abi.sparse_mla(t["q"], t["win"], t["chunk"], t["comp"], nb, t["sink"], idx, D ** -0.5, W, prior,
                          cos, sin, RD)
    torch.cuda.synchronize()
    masked = (idx[0] < 0).sum(1)
    assert masked[0] > 0 and masked[-1] == 0          # both kinds of row occur
    assert torch.isfinite(out.float()).all()
    rows = (0, 1, 255, 510, 511)
    want_o = _oracle_rows(t, rows, [idx[0, s].cpu().numpy() for s in rows], n, prior)
    for s in rows:
        assert_attn_close(to_np(out[0, s]), want_o[s], f"output row {s}")
