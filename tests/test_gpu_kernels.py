"""Kernel-level parity: each HIP entry point against the CPU oracle on the same seeded inputs.

Bars: bit-exact for index work (top-k, candidate blocks, window indices) and for the
fake-quants given identical inputs; 1e-5 max-abs for fp32 attention; for bf16 attention 2e-2
relative (max |a-b| / max |b|) plus per-head bounds at the kernels' own error level (a per-head
least-squares scale within 2^-8 of 1, per-head max error within 1.5e-2 of that head's max; the
check is shown to reject a misplaced sink, a dropped row and a shifted window). Fused kernels that end in a fake-quant are compared
allowing rare one-step rounding flips, which fp32 noise of ~1e-7 upstream of a rounding
midpoint legitimately causes (the reference's own test hits the same thing,
tests/test_parity.py:712-722); the flip rate and size are bounded in the test.
"""

from __future__ import annotations

import os
import zlib

import numpy as np
import pytest
import torch

from common import SEED_BASE, assert_attn_close, attn_close, attn_controls, attn_metrics, max_abs, rel_max_diff, to_np
from oracle import cpu_ref as R

pytestmark = pytest.mark.gpu
F32 = np.float32
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "fakequant_kat.npz")

DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def dev(x, dt="f32", device="cuda"):
    return torch.as_tensor(np.asarray(x, F32)).to(device=device, dtype=DT[dt]).contiguous()


def rng_for(name):
    return np.random.default_rng(zlib.crc32(name.encode()))


def assert_fq_close(got, want, max_flip_frac=2e-3, step_rel=0.26):
    """Equal except for rare single-step flips (each at most one grid step of its row)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = got != want
    frac = bad.mean()
    assert frac <= max_flip_frac, f"{frac:.2e} of values differ"
    if bad.any():
        rowmax = np.abs(want).max(axis=-1, keepdims=True)
        rowmax = np.broadcast_to(rowmax, want.shape)
        assert np.all(np.abs(got - want)[bad] <= step_rel * rowmax[bad])


# ------------------------------------------------------------------ fake-quant


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fake_quants_bit_exact(gpu, dt):
    from dsv41 import _abi
    d = np.load(GOLDEN)
    xs = [d["x0"], d["x1"], d["x2"], rng_for("fq").standard_normal((512, 512)).astype(F32) * 3]
    for x in xs:
        xin = R.cast(x, dt)
        for fn, ref, blk in ((_abi.fq_fp8_ue8m0, R.fq_fp8_ue8m0, 32), (_abi.fq_fp4_ue8m0, R.fq_fp4_ue8m0, 32),
                             (_abi.fq_fp4_e4m3, R.fq_fp4_e4m3, 16)):
            got = to_np(fn(dev(xin, dt), blk))
            want = ref(xin, blk, dt)
            assert np.array_equal(got, want), f"{fn.__name__} {dt} shape {x.shape}"


def test_fake_quant_golden_on_gpu(gpu):
    from dsv41 import _abi
    d = np.load(GOLDEN)
    for n in range(3):
        x = dev(d[f"x{n}"])
        assert np.array_equal(to_np(_abi.fq_fp8_ue8m0(x, 32)), d[f"fp8_ue8m0_{n}"])
        assert np.array_equal(to_np(_abi.fq_fp4_ue8m0(x, 32)), d[f"fp4_ue8m0_{n}"])
        assert np.array_equal(to_np(_abi.fq_fp4_e4m3(x, 16)), d[f"fp4_e4m3_{n}"])


# ------------------------------------------------------------------ rope, norm, tables


def test_rope_table_matches_oracle(gpu):
    from dsv41 import layers
    for args in [(16, 300, 64, 10000.0, 4.0, 32, 1), (64, 70000, 65536, 160000.0, 16.0, 32, 1)]:
        cos, sin = layers.precompute_freqs_cis(*args, device=gpu)
        rc, rs = R.precompute_freqs_cis(*args)
        assert max_abs(to_np(cos), rc) < 2e-6 and max_abs(to_np(sin), rs) < 2e-6


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rope_tail_and_rmsnorm(gpu, dt):
    from dsv41 import _abi
    rng = rng_for("rope" + dt)
    rc, rs = R.precompute_freqs_cis(64, 512, 65536, 160000.0, 16.0, 32, 1)
    cos, sin = dev(rc), dev(rs)
    x = R.cast(rng.standard_normal((2, 37, 8, 512)).astype(F32), dt)
    for inverse in (False, True):
        got = to_np(_abi.rope_tail(dev(x, dt), 64, cos, sin, 100, 3, inverse))
        pos = 100 + 3 * np.arange(37)
        want = R.rope_tail(x, 64, rc[pos], rs[pos], inverse, dt)
        # bit-exact: products and sums rounded separately, as the reference's float32 ops do
        assert np.array_equal(got, want), f"rope_tail {dt} inverse={inverse}"
    w = (1 + 0.1 * rng.standard_normal(1280)).astype(F32)
    y = R.cast(rng.standard_normal((33, 1280)).astype(F32) * 4, dt)
    got = to_np(_abi.rmsnorm(dev(y, dt), dev(w), 1e-20))
    want = R.rmsnorm(y, w, 1e-20, dt)
    assert (max_abs(got, want) < 1e-5) if dt == "f32" else (rel_max_diff(got, want) < 1e-2)


@pytest.mark.parametrize("dt,dim", [("bf16", 5120), ("bf16", 8192), ("bf16", 1280), ("bf16", 64), ("bf16", 1000),
                                    ("f32", 4096), ("f32", 1280), ("f32", 5120)])
def test_rmsnorm_rows_and_fused_residual_add(gpu, dt, dim):
    """dsv41_rmsnorm against the oracle over every launch form (rows held in registers for up to
    1,024 16-byte chunks; the strided kernel for 1,000 bf16 and 5,120 fp32 channels), in place
    too; dsv41_add_rmsnorm (the block's residual add and the next attn_norm) bit for bit equal to
    torch's add followed by dsv41_rmsnorm, h updated in place, on the shapes it takes."""
    from dsv41 import _abi
    rng = rng_for(f"norm{dt}{dim}")
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(F32)
    for rows in (1, 33, 64):
        y = R.cast(rng.standard_normal((rows, dim)).astype(F32) * 4, dt)
        got = to_np(_abi.rmsnorm(dev(y, dt), dev(w), 1e-20))
        want = R.rmsnorm(y, w, 1e-20, dt)
        assert (max_abs(got, want) < 1e-5) if dt == "f32" else (rel_max_diff(got, want) < 1e-2), rows
        x = dev(y, dt)
        assert torch.equal(_abi.rmsnorm(x, dev(w), 1e-20, out=x), dev(got, dt)), "in place"
        per = 16 // (4 if dt == "f32" else 2)
        if dim % per or dim // per > 1024:
            continue
        h = dev(y, dt)
        delta = dev(R.cast(rng.standard_normal((rows, dim)).astype(F32), dt), dt)
        h_want = h + delta
        n_want = _abi.rmsnorm(h_want, dev(w), 1e-20)
        n_got = _abi.add_rmsnorm(h, delta, dev(w), 1e-20)
        torch.cuda.synchronize()
        assert torch.equal(h, h_want), "h + delta"
        assert torch.equal(n_got, n_want), "norm of the sum"


# ------------------------------------------------------------------ fused window / cache writes


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_kv_window_prep_and_ring_write(gpu, dt):
    from dsv41 import _abi
    rng = rng_for("kvw" + dt)
    rc, rs = R.precompute_freqs_cis(64, 400, 65536, 160000.0, 16.0, 32, 1)
    b, n, d, start = 3, 21, 512, 300
    kv = R.cast(rng.standard_normal((b, n, d)).astype(F32), dt)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(F32)
    t = dev(kv, dt)
    _abi.kv_window_prep(t, dev(w), dev(rc), dev(rs), 64, start, 1e-20)
    pos = start + np.arange(n)
    want = R.fq_fp8_ue8m0(R.rope_tail(R.rmsnorm(kv, w, 1e-20, dt), 64, rc[pos], rs[pos], dtype=dt), 32, dt)
    assert_fq_close(to_np(t), want)
    # ring write: last min(n, W) rows to slots p % W
    ring = torch.zeros(b, 16, d, dtype=DT[dt], device=gpu)
    _abi.window_write(ring, t, start)
    want_ring = np.zeros((b, 16, d), F32)
    got_t = to_np(t)
    for j in range(n - 16, n):
        want_ring[:, (start + j) % 16] = got_t[:, j]
    assert np.array_equal(to_np(ring), want_ring)


@pytest.mark.parametrize("wp,n,window", [(0, 7, 8), (8, 13, 8), (128, 1, 128), (50, 300, 128)])
def test_window_idx(gpu, wp, n, window):
    from dsv41.attention import window_idx_matrix
    assert np.array_equal(window_idx_matrix(wp, n, window, gpu).cpu().numpy(), R.window_idx_matrix(wp, n, window))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_compress_pool_chunked(gpu, dt):
    from dsv41 import _abi
    rng = rng_for("pool" + dt)
    b, d, r = 2, 512, 4
    kv = rng.standard_normal((b, 45, d)).astype(F32)
    sc = rng.standard_normal((b, 45, d)).astype(F32)
    nw = (1 + 0.1 * rng.standard_normal(d)).astype(F32)
    st = R.CompressorState(b, r, d)
    ks, ss = dev(st.kv_state), dev(st.score_state)
    pos = 0
    for n in (3, 1, 1, 14, 2, 24):
        want = R.compressor_pool(kv[:, pos:pos + n], sc[:, pos:pos + n], pos, st, r, nw, 1e-20, dt)
        got = _abi.compress_pool(dev(kv[:, pos:pos + n]), dev(sc[:, pos:pos + n]), ks, ss, dev(nw), r, pos,
                                 1e-20, DT[dt])
        assert (want is None) == (got is None), f"chunk at {pos}"
        if want is not None:
            g = to_np(got)
            assert (max_abs(g, want) < 1e-5) if dt == "f32" else (rel_max_diff(g, want) < 1e-2), f"chunk at {pos}"
        rem = (pos + n) % r
        assert np.array_equal(to_np(ks)[:, :rem], st.kv_state[:, :rem])
        assert np.array_equal(to_np(ss)[:, :rem], st.score_state[:, :rem])
        pos += n


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_comp_write_and_index_key_publish(gpu, dt):
    from dsv41 import _abi
    rng = rng_for("cw" + dt)
    rc, rs = R.precompute_freqs_cis(64, 2048, 65536, 160000.0, 16.0, 32, 1)
    b, g, d, di, g0, r = 2, 9, 512, 128, 100, 4
    lat = R.cast(rng.standard_normal((b, g, d)).astype(F32), dt)
    comp = torch.zeros(b, 256, d, dtype=DT[dt], device=gpu)
    _abi.comp_write(dev(lat, dt), comp, g0, r, dev(rc), dev(rs), 64)
    pos = (g0 + np.arange(g)) * r
    want = R.fq_fp4_e4m3(R.rope_tail(lat, 64, rc[pos], rs[pos], dtype=dt), 16, dt)
    got = to_np(comp)
    assert_fq_close(got[:, g0:g0 + g], want)
    assert not got[:, :g0].any() and not got[:, g0 + g:].any()
    kr = R.cast(rng.standard_normal((b, g, di)).astype(F32), dt)
    nw = (1 + 0.1 * rng.standard_normal(di)).astype(F32)
    ik = torch.zeros(b, 256, di, dtype=DT[dt], device=gpu)
    _abi.index_key_publish(dev(kr, dt), ik, g0, r, dev(nw), dev(rc), dev(rs), 64, 1e-20)
    want = R.fq_fp4_ue8m0(R.rope_tail(R.rmsnorm(kr, nw, 1e-20, dt), 64, rc[pos], rs[pos], dtype=dt), 32, dt)
    assert_fq_close(to_np(ik)[:, g0:g0 + g], want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_index_q_prep(gpu, dt):
    from dsv41 import _abi
    rng = rng_for("iq" + dt)
    rc, rs = R.precompute_freqs_cis(64, 600, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((2, 5, 64, 128)).astype(F32), dt)
    t = dev(q, dt)
    _abi.index_q_prep(t, dev(rc), dev(rs), 64, 500)
    pos = 500 + np.arange(5)
    want = R.fq_fp4_ue8m0(R.rope_tail(q, 64, rc[pos], rs[pos], dtype=dt), 32, dt)
    assert_fq_close(to_np(t), want)


# ------------------------------------------------------------------ indexer scoring


@pytest.mark.parametrize("dt,hi,di,b,n,nb,start,use_cand", [
    ("f32", 2, 32, 1, 128, 32, 0, False),          # C1 prefill
    ("f32", 2, 32, 1, 1, 36, 143, True),           # C1 decode
    ("bf16", 64, 128, 4, 1, 4096, 16383, False),    # C2-shaped decode
    ("bf16", 64, 128, 1, 96, 1000, 3900, True),    # prefill chunk, causal + candidates
    ("bf16", 32, 128, 2, 3, 777, 3100, False),     # released model's 32 index heads
    ("bf16", 64, 128, 2, 40, 3000, 11000, False),  # prefill kernel: 8 queries per workgroup, 2 row ranges
    ("bf16", 32, 128, 1, 13, 700, 2500, False),    # prefill kernel: a partial query group (idle waves)
    ("bf16", 16, 128, 3, 9, 300, 100, False),      # prefill kernel: most rows past visibility
    ("bf16", 64, 128, 2, 1, 50, 199, False),       # decode kernel: fewer rows than one 8-wave sweep
    ("bf16", 16, 128, 3, 2, 3000, 4000, True),     # decode kernel: workgroups wholly past visibility
    ("bf16", 32, 128, 5, 1, 20000, 79999, True),   # decode kernel: 40 row ranges, candidates
    ("bf16", 8, 32, 2, 5, 40, 30, True),           # 8 heads, one padded 16-head tile (the reference test's count)
    ("bf16", 24, 64, 2, 1, 900, 3500, False),      # 24 heads: two tiles, the second half padding
    ("bf16", 100, 128, 1, 2, 500, 1900, False),    # 100 heads: eight tiles, register kernel
])
def test_indexer_score(gpu, dt, hi, di, b, n, nb, start, use_cand):
    from dsv41 import _abi
    rng = rng_for(f"idx{dt}{hi}{n}{nb}")
    r = 4
    q = R.fq_fp4_ue8m0(rng.standard_normal((b, n, hi, di)).astype(F32), 32, dt)
    k = R.fq_fp4_ue8m0(rng.standard_normal((b, nb + 5, di)).astype(F32), 32, dt)
    w_raw = R.cast(rng.standard_normal((b, n, hi)).astype(F32), dt)
    scale = R.index_weight_scale(hi, di, dt)
    cand = (rng.random((b, n, nb)) < 0.7) if use_cand else None
    kt = dev(k, dt)
    got = _abi.indexer_score(dev(q, dt), dev(w_raw, dt), scale, kt[:, :nb], start, r,
                             torch.as_tensor(cand).to(gpu) if use_cand else None)
    w = R.cast(w_raw * scale, dt)
    want = R.indexer_scores(q, k[:, :nb], w, start, r, cand)
    g = to_np(got)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(g), fin) and np.array_equal(g[~fin], want[~fin])
    assert np.abs(g[fin] - want[fin]).max() <= 1e-5 * max(np.abs(want[fin]).max(), 1.0)


@pytest.mark.parametrize("b,n,h,nb,start,rb,pad", [
    (16, 1, 64, 32768, 131071, 32, False), (3, 5, 32, 1000, 3990, 1, False), (2, 40, 16, 700, 2700, 32, False),
    (16, 1, 64, 32768, 131071, 32, True),  # 16-byte scale rows: the staged-copy decode kernel
    (3, 5, 32, 1000, 3990, 1, True), (2, 40, 16, 700, 2700, 32, True), (2, 1, 64, 50, 199, 1, True),
    (4, 2, 64, 9000, 35000, 1, True)])
def test_indexer_score_fp8_keys(gpu, b, n, h, nb, start, rb, pad):
    """fp8 index keys dequantized in-kernel: bit-identical to the bf16 path on the dequantized
    keys, and within the bf16 path's tolerance of the oracle. `pad` rounds the scale rows up to a
    multiple of 16 bytes (the layout the staged-copy kernel takes; otherwise the register kernel)."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    rng = rng_for(f"idx8{b}{n}{nb}")
    d, r = 128, 4
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 0.3, "bf16")
    w_raw = R.cast(rng.standard_normal((b, n, h)).astype(F32), "bf16")
    codes = rng.integers(0, 256, size=(b, nb + 3, d), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] ^= 0x01
    nblk = -(-(nb + 3) // rb)
    scales = rng.integers(123, 132, size=(b, (nblk + 3) // 4 * 4 if pad else nblk, d // 32), dtype=np.uint8)
    keys = R.dequant_fp8_cache(codes, scales, rb)
    scale = weight_scale(h, d, torch.bfloat16)
    got8 = _abi.indexer_score_fp8(dev(q, "bf16"), dev(w_raw, "bf16"), scale, torch.as_tensor(codes).to(gpu),
                                  torch.as_tensor(scales).to(gpu), rb, nb, start, r)
    got16 = _abi.indexer_score(dev(q, "bf16"), dev(w_raw, "bf16"), scale, dev(keys[:, :nb], "bf16"), start, r)
    assert torch.equal(got8, got16)
    w = R.cast(w_raw * scale, "bf16")
    want = R.indexer_scores(q, keys[:, :nb], w, start, r)
    g = to_np(got8)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(g), fin)
    assert np.abs(g[fin] - want[fin]).max() <= 1e-5 * max(np.abs(want[fin]).max(), 1.0)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fp8_cache_writers(gpu, dt):
    """The fp8-variant writers store fake_quant_fp8_ue8m0 of the roped latent (and of the normed,
    roped key) packed: decoded, bit-equal to the GPU's own rope + fp8 fake-quant, and within the
    fake-quant flip tolerance of the oracle; untouched rows stay zero."""
    from dsv41 import _abi
    rng = rng_for("w8" + dt)
    rc, rs = R.precompute_freqs_cis(64, 2048, 65536, 160000.0, 16.0, 32, 1)
    b, g, d, di, g0, r = 2, 7, 512, 128, 90, 4
    pos = (g0 + np.arange(g)) * r
    lat = R.cast(rng.standard_normal((b, g, d)).astype(F32) * 2, dt)
    codes = torch.zeros(b, 128, d, dtype=torch.uint8, device=gpu)
    scales = torch.zeros(b, 128, d // 32, dtype=torch.uint8, device=gpu)
    _abi.comp_write_fp8(dev(lat, dt), codes, scales, g0, r, dev(rc), dev(rs), 64)
    roped = _abi.rope_tail(dev(lat, dt), 64, dev(rc), dev(rs), g0 * r, r)     # positions (g0 + j) * r
    dense = to_np(_abi.fq_fp8_ue8m0(roped))
    torch.cuda.synchronize()
    c, sc = codes.cpu().numpy(), scales.cpu().numpy()
    got = R.dequant_fp8_cache(c[:, g0:g0 + g], sc[:, g0:g0 + g], 1)
    assert np.array_equal(got.view(np.uint32), dense.view(np.uint32))
    assert_fq_close(got, R.fq_fp8_ue8m0(R.rope_tail(lat, 64, rc[pos], rs[pos], dtype=dt), 32, dt))
    assert not c[:, :g0].any() and not c[:, g0 + g:].any() and not sc[:, g0 + g:].any()
    kr = R.cast(rng.standard_normal((b, g, di)).astype(F32), dt)
    nw = (1 + 0.1 * rng.standard_normal(di)).astype(F32)
    kc = torch.zeros(b, 128, di, dtype=torch.uint8, device=gpu)
    ks = torch.zeros(b, 128, di // 32, dtype=torch.uint8, device=gpu)
    _abi.index_key_publish_fp8(dev(kr, dt), kc, ks, g0, r, dev(nw), dev(rc), dev(rs), 64, 1e-20)
    want = R.fq_fp8_ue8m0(R.rope_tail(R.rmsnorm(kr, nw, 1e-20, dt), 64, rc[pos], rs[pos], dtype=dt), 32, dt)
    got = R.dequant_fp8_cache(kc.cpu().numpy()[:, g0:g0 + g], ks.cpu().numpy()[:, g0:g0 + g], 1)
    assert_fq_close(got, want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_index_key_publish_mxfp4_decodes_to_the_dense_publish(gpu, dt):
    """The MXFP4 key writer stores the dense writer's values losslessly: decoded, its bytes
    equal dsv41_index_key_publish's output bit for bit; untouched groups stay zero."""
    from dsv41 import _abi
    rng = rng_for("kmx" + dt)
    rc, rs = R.precompute_freqs_cis(64, 2048, 65536, 160000.0, 16.0, 32, 1)
    b, g, di, g0, r = 3, 11, 128, 70, 4
    kr = R.cast(rng.standard_normal((b, g, di)).astype(F32) * 2, dt)
    nw = (1 + 0.1 * rng.standard_normal(di)).astype(F32)
    dense = torch.zeros(b, 128, di, dtype=DT[dt], device=gpu)
    _abi.index_key_publish(dev(kr, dt), dense, g0, r, dev(nw), dev(rc), dev(rs), 64, 1e-20)
    codes = torch.zeros(b, 128, di // 2, dtype=torch.uint8, device=gpu)
    scales = torch.zeros(b, 128, di // 32, dtype=torch.uint8, device=gpu)
    _abi.index_key_publish_mxfp4(dev(kr, dt), codes, scales, g0, r, dev(nw), dev(rc), dev(rs), 64, 1e-20)
    torch.cuda.synchronize()
    c, sc = codes.cpu().numpy(), scales.cpu().numpy()
    got = R.mxfp4_decode(c[:, g0:g0 + g], sc[:, g0:g0 + g])
    want = to_np(dense)[:, g0:g0 + g]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not c[:, :g0].any() and not c[:, g0 + g:].any() and not sc[:, g0 + g:].any()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_index_q_prep_mxfp4_decodes_to_the_dense_prep(gpu, dt):
    """The MXFP4 query prologue holds exactly dsv41_index_q_prep's values, and leaves q as is."""
    from dsv41 import _abi
    rng = rng_for("qmx" + dt)
    b, n, h, d, rd, start = 2, 5, 32, 128, 64, 3000
    rc, rs = R.precompute_freqs_cis(rd, start + n, 65536, 160000.0, 16.0, 32, 1)
    q = dev(R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 3, dt), dt)
    keep = q.clone()
    codes, scales = _abi.index_q_prep_mxfp4(q, dev(rc), dev(rs), rd, start)
    assert torch.equal(q, keep)
    dense = _abi.index_q_prep(q.clone(), dev(rc), dev(rs), rd, start)
    got = R.mxfp4_decode(codes.cpu().numpy(), scales.cpu().numpy())
    assert np.array_equal(got.view(np.uint32), to_np(dense).view(np.uint32))


@pytest.mark.parametrize("b,n,h,nb,start,use_cand", [
    (32, 1, 64, 16384, 65536, False),    # the bs32 / 64K decode shape
    (4, 1, 64, 4096, 16383, True),
    (1, 96, 64, 1000, 3900, True),       # prefill chunk: causal + candidates
    (2, 3, 32, 777, 3100, False),        # 32 index heads
    (3, 2, 16, 333, 1300, False),
])
def test_indexer_score_mxfp4(gpu, b, n, h, nb, start, use_cand):
    """MXFP4 query and keys, block-scaled fp4 MFMA: within 1e-5 of max |S| of the oracle (and of
    the bf16 kernel) on the same fake-quantized values; masks and -inf identical."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    rng = rng_for(f"idxmx{b}{n}{h}{nb}")
    d, r = 128, 4
    q = R.fq_fp4_ue8m0(rng.standard_normal((b, n, h, d)).astype(F32), 32, "bf16")
    k = R.fq_fp4_ue8m0(rng.standard_normal((b, nb + 5, d)).astype(F32) * 3, 32, "bf16")
    qc, qs = R.mxfp4_encode(q)
    kc, ks = R.mxfp4_encode(k)
    assert np.array_equal(R.mxfp4_decode(kc, ks), k) and np.array_equal(R.mxfp4_decode(qc, qs), q)
    w_raw = R.cast(rng.standard_normal((b, n, h)).astype(F32), "bf16")
    scale = weight_scale(h, d, torch.bfloat16)
    cand = (rng.random((b, n, nb)) < 0.7) if use_cand else None
    ct = torch.as_tensor(cand).to(gpu) if use_cand else None
    t = lambda a: torch.as_tensor(a).to(gpu)   # noqa: E731
    got = _abi.indexer_score_mxfp4((t(qc), t(qs)), dev(w_raw, "bf16"), scale, t(kc), t(ks), nb, start, r, ct)
    w = R.cast(w_raw * scale, "bf16")
    want = R.indexer_scores(q, k[:, :nb], w, start, r, cand)
    g = to_np(got)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(g), fin) and np.array_equal(g[~fin], want[~fin])
    tol = 1e-5 * max(np.abs(want[fin]).max(), 1.0)
    assert np.abs(g[fin] - want[fin]).max() <= tol
    dense = to_np(_abi.indexer_score(dev(q, "bf16"), dev(w_raw, "bf16"), scale, dev(k[:, :nb], "bf16"), start, r, ct))
    assert np.array_equal(np.isfinite(dense), fin) and np.abs(dense[fin] - g[fin]).max() <= tol


@pytest.mark.parametrize("b,n,h,nb,topk,start,use_cand", [
    (32, 1, 64, 16384, 512, 65535, False),   # bs32 decode: 8 row ranges of 2048
    (64, 1, 64, 16384, 512, 65535, False),   # 4 ranges of 4096
    (32, 1, 32, 16384, 512, 65535, True),    # candidate-masked consumer, 32 index heads
    (8, 4, 16, 16384, 512, 20000, False),    # causal rows: ranges past visibility list -inf entries
    (16, 4, 64, 16384, 512, 40000, True),    # 4 queries per row and a candidate mask: ranges of 4096
    (3, 9, 32, 8000, 256, 30000, True),      # 9 queries per row (served with a mask), a partial last range
])
def test_indexer_topk_fused_equals_two_calls(gpu, b, n, h, nb, topk, start, use_cand):
    """The fused decode form (per-range best-k lists, then a merge) returns exactly the top-k of
    indexer_score's scores."""
    from dsv41 import _abi
    rng = rng_for(f"fused{b}{n}{h}{use_cand}")
    d, r = 128, 4
    q = dev(R.fq_fp4_ue8m0(rng.standard_normal((b, n, h, d)).astype(F32), 32, "bf16"), "bf16")
    k = dev(R.fq_fp4_ue8m0(rng.standard_normal((b, nb, d)).astype(F32), 32, "bf16"), "bf16")
    w = dev(rng.standard_normal((b, n, h)).astype(F32), "bf16")
    cand = torch.as_tensor(rng.random((b, n, nb)) < 0.7).to(gpu) if use_cand else None
    scale = R.index_weight_scale(h, d, "bf16")
    off = 129
    assert _abi.indexer_topk_workspace_bytes(b, n, h, d, nb, topk, use_cand) > 0
    fused = _abi.indexer_topk(q, w, scale, k, start, r, topk, off, cand)
    two = _abi.topk_select(_abi.indexer_score(q, w, scale, k, start, r, cand), topk, start, r, off)
    assert torch.equal(fused, two)


@pytest.mark.parametrize("b,n,h,nb,topk,start,rb,use_cand", [
    (16, 1, 64, 32768, 512, 131071, 32, False),    # bs16, 128K context, scales per 32 x 32 block
    (8, 4, 16, 16384, 512, 20000, 1, False),       # causal rows, per-row scales, ranges past visibility
    (32, 1, 32, 16384, 512, 65535, 1, True),       # candidate-masked consumer
])
def test_indexer_topk_fp8_equals_two_calls(gpu, b, n, h, nb, topk, start, rb, use_cand):
    """The fused form over fp8 keys selects exactly what indexer_score_fp8 + topk_select select."""
    from dsv41 import _abi
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 47)
    q = (torch.randn(b, n, h, 128, generator=g, device=gpu) * 0.3).bfloat16()
    w = torch.randn(b, n, h, generator=g, device=gpu).bfloat16()
    codes = torch.randint(0, 256, (b, nb, 128), generator=g, device=gpu, dtype=torch.int32)
    codes = torch.where((codes & 0x7F) == 0x7F, codes ^ 1, codes).to(torch.uint8)     # no NaN codes
    nblk = -(-nb // rb)
    scales = torch.randint(123, 132, (b, (nblk + 3) // 4 * 4, 4), generator=g, device=gpu,
                           dtype=torch.int32).to(torch.uint8)
    cand = (torch.rand(b, n, nb, generator=g, device=gpu) < 0.7) if use_cand else None
    fused = _abi.indexer_topk_fp8(q, w, 0.01, codes, scales, rb, nb, start, 4, topk, 129, cand)
    assert fused is not None
    scores = _abi.indexer_score_fp8(q, w, 0.01, codes, scales, rb, nb, start, 4, cand)
    assert torch.equal(fused, _abi.topk_select(scores, topk, start, 4, 129))


@pytest.mark.parametrize("b,n,h,nb,topk,start,use_cand", [
    (32, 1, 64, 16384, 512, 65535, False),   # bs32 decode over an MXFP4 index cache
    (8, 4, 16, 16384, 512, 20000, False),    # causal rows, ranges past visibility
    (32, 1, 32, 16384, 512, 65535, True),    # candidate-masked consumer
    (2, 1, 64, 256, 64, 1024, False),        # one range
    (16, 4, 64, 16384, 512, 40000, True),    # 4 queries per row and a candidate mask
])
def test_indexer_topk_mxfp4_equals_two_calls(gpu, b, n, h, nb, topk, start, use_cand):
    """The fused form over MXFP4 query and keys selects exactly what indexer_score_mxfp4 +
    topk_select select."""
    from dsv41 import _abi
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 48)
    rb = lambda lo, hi, *s: torch.randint(lo, hi, s, generator=g, device=gpu, dtype=torch.int32).to(torch.uint8)  # noqa: E731
    q_mx = (rb(0, 256, b, n, h, 64), rb(120, 132, b, n, h, 4))
    kc, ks = rb(0, 256, b, nb, 64), rb(120, 132, b, nb, 4)
    w = torch.randn(b, n, h, generator=g, device=gpu).bfloat16()
    cand = (torch.rand(b, n, nb, generator=g, device=gpu) < 0.7) if use_cand else None
    fused = _abi.indexer_topk_mxfp4(q_mx, w, 0.01, kc, ks, nb, start, 4, topk, 129, cand)
    assert fused is not None
    scores = _abi.indexer_score_mxfp4(q_mx, w, 0.01, kc, ks, nb, start, 4, cand)
    assert torch.equal(fused, _abi.topk_select(scores, topk, start, 4, 129))


def test_indexer_topk_shared_workspace(gpu):
    """One workspace through a sequence of fused calls of different shapes (query counts, row
    ranges, k, candidate masks, ranges past visibility): every call equals the two-call form."""
    from dsv41 import _abi
    shapes = [(32, 1, 64, 16384, 512, 65535, False), (8, 4, 16, 16384, 512, 20000, False),
              (32, 1, 32, 16384, 512, 65535, True), (2, 1, 64, 256, 64, 1024, False),
              (16, 1, 64, 32768, 512, 131071, False)]
    need = [_abi.indexer_topk_workspace_bytes(b, n, h, 128, nb, k, c) for b, n, h, nb, k, _, c in shapes]
    assert min(need) > 0
    ws = torch.empty(max(need), dtype=torch.uint8, device=gpu)
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 43)
    for rep in range(2):
        for b, n, h, nb, k, start, use_cand in shapes:
            q = torch.randn(b, n, h, 128, generator=g, device=gpu).bfloat16()
            keys = torch.randn(b, nb, 128, generator=g, device=gpu).bfloat16()
            w = torch.randn(b, n, h, generator=g, device=gpu).bfloat16()
            cand = (torch.rand(b, n, nb, generator=g, device=gpu) < 0.7) if use_cand else None
            fused = _abi.indexer_topk(q, w, 0.01, keys, start, 4, k, 129, cand, workspace=ws)
            two = _abi.topk_select(_abi.indexer_score(q, w, 0.01, keys, start, 4, cand), k, start, 4, 129)
            assert torch.equal(fused, two), (rep, b, n, h, nb, k)


# ------------------------------------------------------------------ top-k and candidates


def _score_sets(rng, b, n, nb):
    yield rng.standard_normal((b, n, nb)).astype(F32)
    yield rng.choice(np.array([-np.inf, -1.0, -0.0, 0.0, 0.5, 0.5, 2.0], F32), size=(b, n, nb))
    z = np.zeros((b, n, nb), F32)
    z[..., ::3] = -0.0
    yield z
    yield np.round(rng.standard_normal((b, n, nb)) * 4).astype(F32)


@pytest.mark.parametrize("b,n,nb,topk,start,r", [(2, 3, 40, 16, 100, 4), (4, 1, 4096, 512, 16383, 4),
                                                  (1, 64, 1000, 256, 3000, 4), (2, 1, 16384, 512, 65535, 4),
                                                  (1, 2, 300, 512, 1199, 4), (1, 5, 2049, 2048, 8191, 4),
                                                  (1, 2, 32768, 2048, 131071, 4), (1, 3, 5001, 700, 20003, 4),
                                                  (1, 1, 40000, 1000, 159999, 4), (1, 1, 20000, 5000, 79999, 4),
                                                  (2, 3, 16390, 512, 65559, 4), (1, 2, 20481, 64, 81923, 4),
                                                  (16, 1, 32768, 1024, 131071, 4)])
def test_topk_bit_exact(gpu, b, n, nb, topk, start, r):
    """Rows over 16384 scores with k <= 2048 take the two-stage form (chunk lists, then a merge);
    (2, 3, 16390, ...) and (1, 2, 20481, ...) give it a last chunk shorter than k and rows that are
    not 16-byte multiples; k above 512 takes 8,192-entry chunks (the 32,768 / 40,000 rows, C5's
    16 x 32,768 at k = 1,024). The one-stage entry point must agree bit for bit on those rows too."""
    import ctypes
    from dsv41 import _abi
    rng = rng_for(f"topk{nb}{n}")
    two_stage = _abi.topk_workspace_bytes(b * n, nb, topk) > 0
    for s in _score_sets(rng, b, n, nb):
        lens = R.query_lens(start, n, r)
        s = np.where(np.arange(nb)[None, None] < lens[None, :, None], s, -np.inf).astype(F32)
        off = 129
        st = dev(s)
        got = _abi.topk_select(st, topk, start, r, off)
        want = R.topk_indices(s, topk, lens, off)
        assert np.array_equal(got.cpu().numpy(), want), f"nb={nb} topk={topk}"
        if two_stage:
            one = torch.empty_like(got)
            rc = _abi.lib().dsv41_topk_select(ctypes.c_void_p(st.data_ptr()), ctypes.c_void_p(one.data_ptr()),
                                              b * n, n, nb, topk, start, r, off,
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == 0 and torch.equal(one, got)


@pytest.mark.parametrize("b,n,nb,tb,bs,start,r", [(2, 3, 40, 3, 2, 100, 4), (1, 7, 333, 20, 8, 1200, 4),
                                                   (2, 1, 16384, 2048, 8, 65535, 4), (1, 4, 64, 100, 3, 0, 1),
                                                   (2, 2, 32768, 1024, 8, 131071, 4),    # 4096 blocks, vector path
                                                   (1, 3, 65536, 2048, 8, 262140, 4)])   # 8192 blocks
def test_candidate_blocks_bit_exact(gpu, b, n, nb, tb, bs, start, r):
    from dsv41 import _abi
    from dsv41.indexer import select_candidate_blocks
    rng = rng_for(f"cand{nb}{n}")
    for s in _score_sets(rng, b, n, nb):
        lens = R.query_lens(start, n, r)
        s = np.where(np.arange(nb)[None, None] < lens[None, :, None], s, -np.inf).astype(F32)
        got = _abi.candidate_blocks(dev(s), tb, bs, None, start, r).cpu().numpy()
        want = R.select_candidate_blocks(s, lens, tb, bs)
        assert np.array_equal(got, want)
        got2 = select_candidate_blocks(dev(s), lens, tb, bs).cpu().numpy()
        assert np.array_equal(got2, want)


# ------------------------------------------------------------------ sparse attention


@pytest.mark.parametrize("dt,b,m,h,d,nkv,k", [
    ("f32", 1, 128, 4, 64, 160, 144),      # C1-sized prefill
    ("f32", 2, 3, 6, 512, 300, 70),
    ("bf16", 2, 5, 64, 512, 900, 300),     # prefill-shaped: 64 heads per workgroup
    ("bf16", 32, 1, 64, 512, 4224, 640),   # C2 decode: split index lists + combine
    ("bf16", 3, 2, 16, 576, 200, 97),      # head_dim 576 (512 + 64 reading)
    ("bf16", 1, 4, 4, 64, 50, 33),         # heads < 16 (masked head tile)
    ("bf16", 1, 640, 64, 512, 2000, 96),   # >= 512 queries: the prefill kernel
    ("bf16", 2, 300, 48, 128, 700, 130),   # prefill kernel, partial 64-head group
    ("bf16", 1, 520, 64, 512, 100, 20),    # prefill kernel, one step (pipelined order's edges)
    ("bf16", 1, 512, 64, 256, 300, 50),    # prefill kernel, two steps
    ("bf16", 1, 1, 16, 576, 41000, 40000),  # 18 splits: partials beyond the combine's register set
])
def test_sparse_attn(gpu, dt, b, m, h, d, nkv, k):
    from dsv41.sparse_attention import sparse_attn
    rng = rng_for(f"sa{dt}{b}{m}{h}{d}")
    # logits with std ~2 after the softmax scale: a peaked distribution, not a flat one
    q = R.cast(rng.standard_normal((b, m, h, d)).astype(F32) * 2, dt)
    kv = R.cast(rng.standard_normal((b, nkv, d)).astype(F32), dt)
    sink = rng.standard_normal(h).astype(F32)
    idx = rng.integers(-1, nkv + 3, size=(b, m, k)).astype(np.int32)   # includes -1 and >= nkv
    idx[0, 0, :] = -1                                                   # all-masked row
    got = to_np(sparse_attn(dev(q, dt), dev(kv, dt), dev(sink), torch.as_tensor(idx).to(gpu), d ** -0.5))
    want = R.sparse_attn(q, kv, sink, np.where(idx < nkv, idx, -1), d ** -0.5, dtype=dt)
    assert np.all(got[0, 0] == 0)
    if dt == "f32":
        assert max_abs(got, want) < 1e-5
    else:
        assert_attn_close(got, want)


def _concat_reference(win, chunk, comp, n_comp, start, window):
    """What attention.py:124-168 materializes: concat(prev window chrono, chunk, comp)."""
    wp = min(start, window)
    slots = (start - wp + np.arange(wp)) % window
    return np.concatenate([win[:, slots], chunk, comp[:, :n_comp]], axis=1)


@pytest.mark.parametrize("dt,b,n,h,d,window,start,n_comp,k", [
    ("f32", 1, 1, 4, 64, 128, 143, 36, 16),       # C1 decode
    ("f32", 2, 20, 4, 64, 8, 30, 12, 4),          # chunk longer than part of the ring
    ("bf16", 32, 1, 64, 512, 128, 16383, 4096, 512),
    ("bf16", 1, 40, 64, 512, 16, 100, 35, 24),
    ("bf16", 2, 1, 64, 512, 128, 5, 0, 0),        # window only, ring still filling
    ("bf16", 3, 1, 64, 512, 128, 0, 0, 0),        # the first token: an empty ring, its own row and the sink
    ("f32", 2, 1, 4, 64, 8, 0, 0, 0),
    ("bf16", 1, 600, 64, 512, 16, 200, 150, 64),  # >= 512 queries: the 64-head two-role prefill kernel
    ("bf16", 2, 300, 96, 512, 128, 1000, 300, 128),   # 96 heads: its second workgroup has one idle tile
    ("bf16", 2, 300, 64, 512, 128, 1000, 300, 128),   # two batch rows through the two-role kernel
    ("bf16", 1, 520, 128, 512, 128, 3000, 700, 96),   # 128 heads: two head groups per query
])
def test_sparse_mla_in_place_sources(gpu, dt, b, n, h, d, window, start, n_comp, k):
    from dsv41 import _abi
    rng = rng_for(f"mla{dt}{b}{n}{start}")
    rd = 16 if d == 64 else 64
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 2, dt)
    win = R.cast(rng.standard_normal((b, window, d)).astype(F32), dt)
    chunk = R.cast(rng.standard_normal((b, n, d)).astype(F32), dt)
    comp = R.cast(rng.standard_normal((b, n_comp + 7, d)).astype(F32), dt)
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    lens = R.query_lens(start, n, 4)
    cidx = None
    if k:
        cidx = np.sort(rng.integers(0, max(n_comp, 1), size=(b, n, k)), axis=-1)
        cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
    got = _abi.sparse_mla(dev(q, dt), dev(win, dt), dev(chunk, dt), dev(comp, dt) if n_comp else None, n_comp,
                          dev(sink), torch.as_tensor(cidx).to(gpu) if k else None, d ** -0.5, window, start,
                          dev(rc), dev(rs), rd)
    kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
    widx = np.broadcast_to(R.window_idx_matrix(wp, n, window)[None], (b, n, min(window, wp + n)))
    idxs = np.concatenate([widx, cidx], axis=-1) if k else widx
    o = R.sparse_attn(q, kv_all, sink, idxs, d ** -0.5, dtype=dt)
    pos = start + np.arange(n)
    want = R.rope_tail(o, rd, rc[pos], rs[pos], inverse=True, dtype=dt)
    g = to_np(got)
    if dt == "f32":
        assert max_abs(g, want) < 1e-5
    else:
        assert_attn_close(g, want)


@pytest.mark.parametrize("plan,b,n,start,n_comp,k", [
    ("decode split", 32, 1, 16383, 4096, 512),     # C2: the list split across workgroups + combine
    ("prefill two-role", 1, 600, 1000, 250, 128),  # >= 512 queries: mla_roles_kernel, no split
])
def test_bf16_attention_check_rejects_planted_mistakes(gpu, plan, b, n, start, n_comp, k):
    """The check every bf16 attention test uses (2e-2 of max |o| plus the per-head scale and
    per-head error bounds of tests/common.py) accepts the kernel and rejects the oracle
    recomputed with each planted mistake -- sink zeroed, sink counted once per split, one list
    row dropped, the window read one row early -- on data at the release scale (q and KV
    N(0,1)/sqrt(576), sinks N(0,1): flat softmax weights over the list, where a sink moves a
    head's output by e^sink / rows, well inside 2e-2 of max |o|). Both directions: the kernel's
    output against each changed oracle, and each changed oracle against the oracle
    (sparse_attention.py:51-57; kernel.py:352-383)."""
    from dsv41 import _abi
    h, d, window, rd = 64, 512, 128, 64
    rng = rng_for(f"ctl{plan}")
    s = 576 ** -0.5
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * s, "bf16")
    win = R.cast(rng.standard_normal((b, window, d)).astype(F32) * s, "bf16")
    chunk = R.cast(rng.standard_normal((b, n, d)).astype(F32) * s, "bf16")
    comp = R.cast(rng.standard_normal((b, n_comp, d)).astype(F32) * s, "bf16")
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    lens = R.query_lens(start, n, 4)
    cidx = np.sort(np.stack([np.stack([rng.choice(max(int(min(lens[i], n_comp)), k), k, replace=False)
                                       for i in range(n)]) for _ in range(b)]), axis=-1)
    cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
    got = to_np(_abi.sparse_mla(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), dev(comp, "bf16"), n_comp,
                                dev(sink), torch.as_tensor(cidx).to(gpu), d ** -0.5, window, start, dev(rc), dev(rs),
                                rd))
    kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
    weff = min(window, wp + n)
    widx = np.broadcast_to(R.window_idx_matrix(wp, n, window)[None], (b, n, weff))
    idxs = np.concatenate([widx, cidx], axis=-1)
    pos = start + np.arange(n)

    def oracle(ix, sk):
        o = R.sparse_attn(q, kv_all, sk, ix, d ** -0.5, dtype="bf16")
        return R.rope_tail(o, rd, rc[pos], rs[pos], inverse=True, dtype="bf16")

    want = oracle(idxs, sink)
    m = attn_metrics(got, want)
    print(f"[{plan}] kernel vs oracle: rel {m[0]:.3e} |alpha-1| {m[1]:.3e} head err {m[2]:.3e}", flush=True)
    assert attn_close(got, want)
    for name, ix, sk in attn_controls(idxs, sink, window_rows=weff):
        bad = oracle(ix, sk)
        m1, m2 = attn_metrics(got, bad), attn_metrics(bad, want)
        print(f"[{plan}] {name}: kernel vs changed oracle rel {m1[0]:.3e} |alpha-1| {m1[1]:.3e} head err "
              f"{m1[2]:.3e}; changed vs oracle rel {m2[0]:.3e}", flush=True)
        assert not attn_close(got, bad), name
        assert not attn_close(bad, want), name


def test_sparse_mla_split_lists_reuse_workspace(gpu):
    """Decode lists split 14 ways and merged: one workspace serves consecutive calls (different
    data, then a smaller batch)."""
    from dsv41 import _abi
    d, h, window, start, rd = 512, 64, 128, 40000, 64
    rc, rs = R.precompute_freqs_cis(rd, start + 2, 65536, 160000.0, 16.0, 32, 1)
    n_comp, k = 9000, 2000                    # 2128 rows per query: 16 splits at batch 8
    ws = None
    for call, b in enumerate((8, 8, 3)):
        rng = rng_for(f"mlaws{call}")
        q = R.cast(rng.standard_normal((b, 1, h, d)).astype(F32) * 2, "bf16")
        win = R.cast(rng.standard_normal((b, window, d)).astype(F32), "bf16")
        chunk = R.cast(rng.standard_normal((b, 1, d)).astype(F32), "bf16")
        comp = R.cast(rng.standard_normal((b, n_comp, d)).astype(F32), "bf16")
        sink = rng.standard_normal(h).astype(F32)
        cidx = np.sort(rng.integers(0, n_comp, size=(b, 1, k)), axis=-1)
        cidx[:, :, ::7] = -1
        cidx = np.where(cidx >= 0, cidx + window + 1, -1).astype(np.int32)
        nbytes = _abi.mla_workspace_bytes(b, 1, h, d, window + k, torch.bfloat16)
        assert nbytes > 0
        if ws is None:
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
        assert ws.numel() >= nbytes
        got = _abi.sparse_mla(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), dev(comp, "bf16"), n_comp,
                              dev(sink), torch.as_tensor(cidx).to(gpu), d ** -0.5, window, start, dev(rc), dev(rs),
                              rd, workspace=ws)
        torch.cuda.synchronize()
        kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
        widx = np.broadcast_to(R.window_idx_matrix(window, 1, window)[None], (b, 1, window))
        o = R.sparse_attn(q, kv_all, sink, np.concatenate([widx, cidx], axis=-1), d ** -0.5, dtype="bf16")
        want = R.rope_tail(o, rd, rc[[start]], rs[[start]], inverse=True, dtype="bf16")
        assert_attn_close(to_np(got), want, f"call {call}")


def _fp8_cache(rng, b, rows, d, rb):
    """e4m3 codes (the two NaN codes avoided) and ue8m0 block scales 2^-4 .. 2^4."""
    codes = rng.integers(0, 256, size=(b, rows, d), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] ^= 0x01
    scales = rng.integers(123, 132, size=(b, -(-rows // rb), d // 32), dtype=np.uint8)
    return codes, scales


@pytest.mark.parametrize("b,n,window,start,n_comp,k,rb", [
    (8, 1, 128, 40000, 9000, 1000, 32),     # decode, split index lists, 32x32-block scales
    (16, 1, 128, 131071, 4000, 1024, 32),   # the fp8-cache decode shape (batch 16, top-1024), smaller cache
    (1, 600, 16, 200, 150, 64, 1),          # >= 512 queries: the 64-head plan; per-row scales
])
def test_sparse_mla_fp8_cache_equals_bf16_on_dequantized_cache(gpu, b, n, window, start, n_comp, k, rb):
    """fp8 compressed cache dequantized in-kernel: bit-identical to the bf16 path on the
    dequantized cache (e4m3 x 2^k is exact in bf16) and within the bf16 tolerance of the oracle."""
    from dsv41 import _abi
    rng = rng_for(f"mla8{b}{n}{start}")
    h, d, rd = 64, 512, 64
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 2, "bf16")
    win = R.cast(rng.standard_normal((b, window, d)).astype(F32), "bf16")
    chunk = R.cast(rng.standard_normal((b, n, d)).astype(F32), "bf16")
    codes, scales = _fp8_cache(rng, b, n_comp + 5, d, rb)
    comp = R.dequant_fp8_cache(codes, scales, rb)
    assert np.array_equal(R.cast(comp, "bf16"), comp)
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    lens = R.query_lens(start, n, 4)
    cidx = np.sort(rng.integers(0, n_comp, size=(b, n, k)), axis=-1)
    cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
    cidx[:, :, ::5] = -1
    idx_t = torch.as_tensor(cidx).to(gpu)
    args = (d ** -0.5, window, start, dev(rc), dev(rs), rd)
    got8 = _abi.sparse_mla_fp8(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), torch.as_tensor(codes).to(gpu),
                               torch.as_tensor(scales).to(gpu), rb, n_comp, dev(sink), idx_t, *args)
    got16 = _abi.sparse_mla(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), dev(comp, "bf16"), n_comp,
                            dev(sink), idx_t, *args)
    assert torch.equal(got8, got16)
    kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
    widx = np.broadcast_to(R.window_idx_matrix(wp, n, window)[None], (b, n, min(window, wp + n)))
    o = R.sparse_attn(q, kv_all, sink, np.concatenate([widx, cidx], axis=-1), d ** -0.5, dtype="bf16")
    pos = start + np.arange(n)
    want = R.rope_tail(o, rd, rc[pos], rs[pos], inverse=True, dtype="bf16")
    assert_attn_close(to_np(got8), want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_comp_write_fp4_packs_the_comp_write_values(gpu, dt):
    """The packed fp4 writer stores the oracle's encoding of the GPU's own roped latents, byte
    for byte; decoded, those rows are bit-equal to what the dense comp_write stores; rows outside
    the written groups stay zero."""
    from dsv41 import _abi
    rng = rng_for("w4" + dt)
    rc, rs = R.precompute_freqs_cis(64, 2048, 65536, 160000.0, 16.0, 32, 1)
    b, g, d, g0, r = 3, 11, 512, 77, 4
    lat = R.cast(rng.standard_normal((b, g, d)).astype(F32) * 2, dt)
    lat[0, 0, :16] = 0.0                               # a zero block: the floor scale
    lat[1, 2, 32:48] *= 1e-2                           # a small block: a subnormal e4m3 scale
    row = _abi.fp4_row_bytes(d)
    assert row == 288
    packed = torch.zeros(b, 128, row, dtype=torch.uint8, device=gpu)
    _abi.comp_write_fp4(dev(lat, dt), packed, g0, r, dev(rc), dev(rs), 64)
    dense = torch.zeros(b, 128, d, dtype=DT[dt], device=gpu)
    _abi.comp_write(dev(lat, dt), dense, g0, r, dev(rc), dev(rs), 64)
    roped = to_np(_abi.rope_tail(dev(lat, dt), 64, dev(rc), dev(rs), g0 * r, r))
    torch.cuda.synchronize()
    p = packed.cpu().numpy()
    assert np.array_equal(p[:, g0:g0 + g], R.fp4_e4m3_encode(roped))
    got = R.fp4_e4m3_decode(p[:, g0:g0 + g])
    assert np.array_equal(got.view(np.uint32), to_np(dense)[:, g0:g0 + g].view(np.uint32))
    assert not p[:, :g0].any() and not p[:, g0 + g:].any()
    assert p[0, g0, 256] == 0x01 and 0x01 < p[1, g0 + 2, 258] < 0x08     # the floor and a subnormal scale


def _fp4_cache(rng, b, rows, d):
    """Packed fp4 rows: uniform random code bytes and e4m3 scale bytes 2^-5 .. 2^3 (no NaN)."""
    codes = rng.integers(0, 256, size=(b, rows, d // 2), dtype=np.uint8)
    scales = rng.integers(0x10, 0x58, size=(b, rows, d // 16), dtype=np.uint8)
    return np.concatenate([codes, scales], axis=-1)


@pytest.mark.parametrize("b,n,window,start,n_comp,k", [
    (8, 1, 128, 40000, 9000, 1000),         # decode, split index lists
    (16, 1, 128, 131071, 4000, 1024),       # batch 16, top-1024
    (2, 1, 128, 5, 1, 3),                   # a short ring, one compressed row
    (1, 600, 16, 200, 150, 64),             # >= 512 queries: the 64-head plan
])
def test_sparse_mla_fp4_cache_equals_bf16_on_decoded_cache(gpu, b, n, window, start, n_comp, k):
    """Packed fp4 compressed cache decoded in-kernel: bit-identical to the bf16 path on the
    decoded cache (an e2m1 value times an e4m3 scale is exact in bf16), the decode form's ring
    write identical too, and within the bf16 tolerance of the oracle."""
    from dsv41 import _abi
    rng = rng_for(f"mla4{b}{n}{start}")
    h, d, rd = 64, 512, 64
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 2, "bf16")
    win = R.cast(rng.standard_normal((b, window, d)).astype(F32), "bf16")
    chunk = R.cast(rng.standard_normal((b, n, d)).astype(F32), "bf16")
    rows = _fp4_cache(rng, b, n_comp + 5, d)
    comp = R.fp4_e4m3_decode(rows)
    assert np.array_equal(R.cast(comp, "bf16"), comp)
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    lens = R.query_lens(start, n, 4)
    cidx = np.sort(rng.integers(0, n_comp, size=(b, n, k)), axis=-1)
    cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
    cidx[:, :, ::5] = -1
    idx_t = torch.as_tensor(cidx).to(gpu)
    args = (d ** -0.5, window, start, dev(rc), dev(rs), rd)
    rows_t = torch.as_tensor(rows).to(gpu)
    got4 = _abi.sparse_mla_fp4(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), rows_t, n_comp, dev(sink),
                               idx_t, *args)
    got16 = _abi.sparse_mla(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"), dev(comp, "bf16"), n_comp,
                            dev(sink), idx_t, *args)
    assert torch.equal(got4, got16)
    if n == 1:                                     # the decode form: output and ring write
        ring4, ring16 = dev(win, "bf16"), dev(win, "bf16")
        o4 = _abi.sparse_mla_fp4(dev(q, "bf16"), ring4, dev(chunk, "bf16"), rows_t, n_comp, dev(sink), idx_t, *args,
                                 write_ring=True)
        o16 = _abi.sparse_mla(dev(q, "bf16"), ring16, dev(chunk, "bf16"), dev(comp, "bf16"), n_comp, dev(sink),
                              idx_t, *args, write_ring=True)
        assert torch.equal(o4, o16) and torch.equal(o4, got4) and torch.equal(ring4, ring16)
        assert torch.equal(ring4[:, start % window], dev(chunk, "bf16")[:, 0])
    kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
    widx = np.broadcast_to(R.window_idx_matrix(wp, n, window)[None], (b, n, min(window, wp + n)))
    o = R.sparse_attn(q, kv_all, sink, np.concatenate([widx, cidx], axis=-1), d ** -0.5, dtype="bf16")
    pos = start + np.arange(n)
    want = R.rope_tail(o, rd, rc[pos], rs[pos], inverse=True, dtype="bf16")
    assert_attn_close(to_np(got4), want)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n,window,start", [(21, 16, 300), (5, 128, 7), (1, 128, 131071)])
def test_window_write_mxfp8_ring(gpu, dt, n, window, start):
    """The MXFP8 ring write stores the oracle's MXFP8 rows of the last min(n, window) chunk rows
    at slots p % window, byte for byte, and leaves the other slots alone; for window KV carrying
    the fp8 QAT (the GPU's own kv_window_prep output) the rows decode to that KV exactly."""
    from dsv41 import _abi
    rng = rng_for(f"w8ring{dt}{n}{start}")
    rc, rs = R.precompute_freqs_cis(64, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    b, d = 3, 512
    kv = R.cast(rng.standard_normal((b, n, d)).astype(F32) * 3, dt)
    t = dev(kv, dt)
    _abi.kv_window_prep(t, dev(np.ones(d, F32)), dev(rc), dev(rs), 64, start, 1e-20)   # carries the QAT
    for src in (dev(kv, dt), t):
        ring = torch.full((b, window, _abi.mxfp8_row_bytes(d)), 0x5A, dtype=torch.uint8, device=gpu)
        _abi.window_write_mxfp8(ring, src, start)
        torch.cuda.synchronize()
        got, x = ring.cpu().numpy(), to_np(src)
        keep = min(n, window)
        want = np.full_like(got, 0x5A)
        for j in range(n - keep, n):
            want[:, (start + j) % window] = R.mxfp8_encode(x[:, j])
        assert np.array_equal(got, want)
    slots = [(start + j) % window for j in range(n - keep, n)]
    dec = R.mxfp8_decode(got[:, slots])
    assert np.array_equal(dec.view(np.uint32), to_np(t)[:, n - keep:].view(np.uint32))


def _mxfp8_ring(rng, b, window, d):
    """MXFP8 ring rows: e4m3 codes without the NaN patterns, ue8m0 scales 2^-4 .. 2^3."""
    codes = rng.integers(0, 256, size=(b, window, d), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] ^= 0x01
    scales = rng.integers(123, 131, size=(b, window, d // 32), dtype=np.uint8)
    return np.concatenate([codes, scales], axis=-1)


@pytest.mark.parametrize("b,n,window,start,n_comp,k", [
    (8, 1, 128, 40000, 9000, 1000),         # decode, split index lists
    (4, 1, 128, 60, 15, 15),                # ring still filling
    (3, 1, 128, 300, 0, 0),                 # a window-only layer
    (1, 600, 16, 200, 150, 64),             # >= 512 queries: the 64-head plan
])
def test_sparse_mla_packed_equals_bf16_on_decoded_caches(gpu, b, n, window, start, n_comp, k):
    """MXFP8 window ring and packed fp4 compressed rows, both decoded in-kernel: bit-identical to
    the bf16 path on the decoded caches; the decode form's ring store writes the token's MXFP8 row
    and nothing else; within the bf16 tolerance of the oracle."""
    from dsv41 import _abi
    rng = rng_for(f"mlap{b}{n}{start}")
    h, d, rd = 64, 512, 64
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 2, "bf16")
    ring8 = _mxfp8_ring(rng, b, window, d)
    win = R.mxfp8_decode(ring8)
    assert np.array_equal(R.cast(win, "bf16"), win)
    chunk = R.fq_fp8_ue8m0(R.cast(rng.standard_normal((b, n, d)).astype(F32), "bf16"), 32, "bf16")
    rows4 = _fp4_cache(rng, b, n_comp + 5, d)
    comp = R.fp4_e4m3_decode(rows4)
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    cidx = None
    if k:
        lens = R.query_lens(start, n, 4)
        cidx = np.sort(rng.integers(0, n_comp, size=(b, n, k)), axis=-1)
        cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
        cidx[:, :, ::5] = -1
    idx_t = torch.as_tensor(cidx).to(gpu) if k else None
    args = (d ** -0.5, window, start, dev(rc), dev(rs), rd)
    r8 = torch.as_tensor(ring8).to(gpu)
    c4 = torch.as_tensor(rows4).to(gpu) if n_comp else None
    got = _abi.sparse_mla_packed(dev(q, "bf16"), r8, dev(chunk, "bf16"), c4, n_comp, dev(sink), idx_t, *args)
    ref = _abi.sparse_mla(dev(q, "bf16"), dev(win, "bf16"), dev(chunk, "bf16"),
                          dev(comp, "bf16") if n_comp else None, n_comp, dev(sink), idx_t, *args)
    assert torch.equal(got, ref)
    if n == 1:
        r8d = r8.clone()
        o = _abi.sparse_mla_packed(dev(q, "bf16"), r8d, dev(chunk, "bf16"), c4, n_comp, dev(sink), idx_t, *args,
                                   write_ring=True)
        assert torch.equal(o, got)
        want_ring = ring8.copy()
        want_ring[:, start % window] = R.mxfp8_encode(chunk[:, 0])
        assert np.array_equal(r8d.cpu().numpy(), want_ring)
    kv_all = _concat_reference(win, chunk, comp, n_comp, start, window)
    widx = np.broadcast_to(R.window_idx_matrix(wp, n, window)[None], (b, n, min(window, wp + n)))
    full = np.concatenate([widx, cidx], axis=-1) if k else widx
    o = R.sparse_attn(q, kv_all, sink, np.ascontiguousarray(full), d ** -0.5, dtype="bf16")
    pos = start + np.arange(n)
    want = R.rope_tail(o, rd, rc[pos], rs[pos], inverse=True, dtype="bf16")
    assert_attn_close(to_np(got), want)


@pytest.mark.parametrize("form,dt,b,n,h,d,window,start,n_comp,k,rdo", [
    ("dense", "f32", 1, 1, 4, 64, 128, 143, 36, 16, 16),     # C1 decode, the fp32 kernel
    ("dense", "f32", 2, 20, 4, 64, 8, 30, 12, 4, 0),         # a chunk, no inverse rope (the hook)
    ("dense", "bf16", 32, 1, 64, 512, 128, 16383, 4096, 512, 64),   # bs32 decode: split lists
    ("dense", "bf16", 1, 600, 64, 512, 16, 200, 150, 64, 64),       # >= 512 queries: the 64-head plan
    ("dense", "bf16", 2, 1, 64, 512, 128, 5, 0, 0, 0),       # window only, no inverse rope
    ("fp8", "bf16", 8, 1, 64, 512, 128, 40000, 9000, 1000, 64),
    ("fp4", "bf16", 8, 1, 64, 512, 128, 40000, 9000, 1000, 64),
    ("packed", "bf16", 8, 1, 64, 512, 128, 40000, 9000, 1000, 64),
    ("packed", "bf16", 1, 600, 64, 512, 16, 200, 150, 64, 64),
])
def test_sparse_mla_q_rope_in_launch(gpu, form, dt, b, n, h, d, window, start, n_comp, k, rdo):
    """q_rd: the launch applies q's forward rope tail (attention.py:117) as it loads q. Bit-equal
    to dsv41_rope_tail on q followed by the same call without it, on every cache form and plan
    (whatever rd the output's inverse rope uses); q itself is left as given; and the roped q
    equals the oracle's rope_tail."""
    from dsv41 import _abi
    rng = rng_for(f"mlaqr{form}{dt}{b}{n}{start}")
    rd = 16 if d == 64 else 64
    rc, rs = R.precompute_freqs_cis(rd, start + n + 1, 65536, 160000.0, 16.0, 32, 1)
    q = R.cast(rng.standard_normal((b, n, h, d)).astype(F32) * 2, dt)
    chunk = R.cast(rng.standard_normal((b, n, d)).astype(F32), dt)
    sink = rng.standard_normal(h).astype(F32)
    wp = min(start, window)
    cidx = None
    if k:
        lens = R.query_lens(start, n, 4)
        cidx = np.sort(rng.integers(0, n_comp, size=(b, n, k)), axis=-1)
        cidx = np.where(cidx < np.minimum(lens, n_comp)[None, :, None], cidx + wp + n, -1).astype(np.int32)
    idx_t = torch.as_tensor(cidx).to(gpu) if k else None
    cos, sin = dev(rc), dev(rs)
    if form == "dense":
        win = dev(R.cast(rng.standard_normal((b, window, d)).astype(F32), dt), dt)
        comp = dev(R.cast(rng.standard_normal((b, n_comp + 7, d)).astype(F32), dt), dt) if n_comp else None
        call = lambda qq, **kw: _abi.sparse_mla(qq, win, dev(chunk, dt), comp, n_comp, dev(sink), idx_t,  # noqa: E731
                                                d ** -0.5, window, start, cos, sin, rdo, **kw)
    elif form == "fp8":
        codes, scales = _fp8_cache(rng, b, n_comp + 5, d, 32)
        win = dev(R.cast(rng.standard_normal((b, window, d)).astype(F32), dt), dt)
        c8, s8 = torch.as_tensor(codes).to(gpu), torch.as_tensor(scales).to(gpu)
        call = lambda qq, **kw: _abi.sparse_mla_fp8(qq, win, dev(chunk, dt), c8, s8, 32, n_comp,  # noqa: E731
                                                    dev(sink), idx_t, d ** -0.5, window, start, cos, sin, rdo, **kw)
    elif form == "fp4":
        win = dev(R.cast(rng.standard_normal((b, window, d)).astype(F32), dt), dt)
        c4 = torch.as_tensor(_fp4_cache(rng, b, n_comp + 5, d)).to(gpu)
        call = lambda qq, **kw: _abi.sparse_mla_fp4(qq, win, dev(chunk, dt), c4, n_comp, dev(sink), idx_t,  # noqa: E731
                                                    d ** -0.5, window, start, cos, sin, rdo, **kw)
    else:
        r8 = torch.as_tensor(_mxfp8_ring(rng, b, window, d)).to(gpu)
        c4 = torch.as_tensor(_fp4_cache(rng, b, n_comp + 5, d)).to(gpu)
        call = lambda qq, **kw: _abi.sparse_mla_packed(qq, r8, dev(chunk, dt), c4, n_comp, dev(sink),  # noqa: E731
                                                       idx_t, d ** -0.5, window, start, cos, sin, rdo, **kw)
    q_dev = dev(q, dt)
    q_keep = q_dev.clone()
    got = call(q_dev, q_rd=rd)
    roped = _abi.rope_tail(q_dev.clone(), rd, cos, sin, start, 1)
    want = call(roped)
    torch.cuda.synchronize()
    assert torch.equal(q_dev, q_keep), "q must be left as given"
    assert torch.equal(got, want), "in-launch q rope differs from rope_tail + attention"
    pos = start + np.arange(n)
    assert np.array_equal(to_np(roped), R.rope_tail(q, rd, rc[pos], rs[pos], dtype=dt))


def test_reference_kernel_module_seam(gpu):
    """dsv41.kernel stands in for the reference model's native `kernel` module."""
    import dsv41.kernel as K
    rng = rng_for("seam")
    x = rng.standard_normal((64, 128)).astype(F32) * 2
    t = dev(x)
    K.act_quant(t, 32, "ue8m0", None, True)
    assert np.array_equal(to_np(t), R.fq_fp8_ue8m0(x, 32))
    t = dev(x)
    K.fp4_act_quant(t, 32, True)
    assert np.array_equal(to_np(t), R.fq_fp4_ue8m0(x, 32))
    t = dev(x)
    K.fp4_act_quant(t, 16, True, torch.float8_e4m3fn)
    assert np.array_equal(to_np(t), R.fq_fp4_e4m3(x, 16))
    q = rng.standard_normal((1, 3, 4, 64)).astype(F32)
    kv = rng.standard_normal((1, 20, 64)).astype(F32)
    sink = rng.standard_normal(4).astype(F32)
    idx = rng.integers(-1, 20, size=(1, 3, 7)).astype(np.int32)
    got = to_np(K.sparse_attn(dev(q), dev(kv), dev(sink), torch.as_tensor(idx).to(gpu), 0.125))
    assert max_abs(got, R.sparse_attn(q, kv, sink, idx, 0.125)) < 1e-5
    with pytest.raises(NotImplementedError):
        K.act_quant(dev(x), 32)
    with pytest.raises(RuntimeError):
        K.fp8_gemm()


@pytest.mark.parametrize("dt,b,h,d,window,start,n_comp,k", [
    ("bf16", 32, 64, 512, 128, 16383, 4096, 512),   # split lists + combine
    ("bf16", 600, 64, 512, 128, 700, 175, 64),     # one workgroup per 64 heads, no split
    ("bf16", 3, 16, 576, 128, 5, 1, 1),            # ring still filling
    ("f32", 2, 4, 64, 8, 37, 9, 4),                # fp32 kernel, wrapped ring
])
def test_sparse_mla_decode_writes_the_ring(gpu, dt, b, h, d, window, start, n_comp, k):
    """dsv41_sparse_mla_decode: same output as dsv41_sparse_mla, and the ring afterwards equals
    what the separate window write produces."""
    from dsv41 import _abi
    rng = rng_for(f"mlad{dt}{b}{d}")
    rd = 16 if d == 64 else 64
    rc, rs = R.precompute_freqs_cis(rd, start + 2, 65536, 160000.0, 16.0, 32, 1)
    q = dev(R.cast(rng.standard_normal((b, 1, h, d)).astype(F32), dt), dt)
    win = dev(R.cast(rng.standard_normal((b, window, d)).astype(F32), dt), dt)
    chunk = dev(R.cast(rng.standard_normal((b, 1, d)).astype(F32), dt), dt)
    comp = dev(R.cast(rng.standard_normal((b, n_comp, d)).astype(F32), dt), dt)
    sink = dev(rng.standard_normal(h).astype(F32))
    cidx = np.sort(rng.integers(0, n_comp, size=(b, 1, k)), axis=-1)
    cidx[:, :, ::5] = -1
    wp = min(start, window)
    idx = torch.as_tensor(np.where(cidx >= 0, cidx + wp + 1, -1).astype(np.int32)).to(gpu)
    args = (comp, n_comp, sink, idx, d ** -0.5, window, start, dev(rc), dev(rs), rd)
    ring_a, ring_b = win.clone(), win.clone()
    want = _abi.sparse_mla(q, ring_a, chunk, *args)
    _abi.window_write(ring_a, chunk, start)
    got = _abi.sparse_mla(q, ring_b, chunk, *args, write_ring=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(ring_b, ring_a)


def test_wrappers_refuse_bad_buffers_before_launch(gpu):
    """A caller's malformed buffer raises ValueError on the host, before any kernel runs: an
    undersized or mistyped out, a cache with fewer batch rows than the call, a bf16 sink or norm
    weight. The same calls with correct buffers then run."""
    from dsv41 import _abi
    from dsv41.layers import precompute_freqs_cis
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 77)
    rn = lambda *s: torch.randn(*s, generator=g, device=gpu)   # noqa: E731
    b, H, D, W, nb, K, start, rd = 4, 64, 512, 128, 2048, 256, 8191, 64
    q, chunk, win = rn(b, 1, H, D).bfloat16(), rn(b, 1, D).bfloat16(), rn(b, W, D).bfloat16()
    comp, sink = rn(b, nb, D).bfloat16(), rn(H)
    iq, ik, w = rn(b, 1, 64, 128).bfloat16(), rn(b, nb, 128).bfloat16(), rn(b, 1, 64).bfloat16()
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    scores = _abi.indexer_score(iq, w, 0.01, ik, start, 4)
    idx = _abi.topk_select(scores, K, start, 4, W + 1)
    args = (q, win, chunk, comp, nb, sink, idx, D ** -0.5, W, start, cos, sin, rd)
    with pytest.raises(ValueError, match="out must be"):
        _abi.sparse_mla(*args, out=torch.empty(b, 1, H, D // 2, dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="batch rows"):
        _abi.sparse_mla(q, win, chunk, comp[: b - 1], nb, sink, idx, D ** -0.5, W, start, cos, sin, rd)
    with pytest.raises(ValueError, match="attn_sink"):
        _abi.sparse_mla(q, win, chunk, comp, nb, sink.bfloat16(), idx, D ** -0.5, W, start, cos, sin, rd)
    with pytest.raises(ValueError, match="out must be"):
        _abi.indexer_score(iq, w, 0.01, ik, start, 4, out=torch.empty(b, 1, nb - 1, device=gpu))
    with pytest.raises(ValueError, match="out must be"):
        _abi.topk_select(scores, K, start, 4, W + 1, out=torch.empty(b, 1, K, dtype=torch.int64, device=gpu))
    with pytest.raises(ValueError, match="batch rows"):
        _abi.comp_write(rn(b, 1, D).bfloat16(), comp[: b - 1], 0, 4, cos, sin, rd)
    with pytest.raises(ValueError, match="k_norm"):
        _abi.index_key_publish(rn(b, 1, 128).bfloat16(), ik, 0, 4, torch.ones(128, device=gpu).bfloat16(), cos,
                               sin, rd, 1e-6)
    torch.cuda.synchronize()
    o = _abi.sparse_mla(*args, out=torch.empty_like(q))
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()


def test_sparse_mla_rows_on_both_sides_of_a_2gib_address_boundary(gpu):
    """Regression test of a GPU memory fault met while the decode kernel was written: a 64-bit row
    address is carried across lanes as two 32-bit halves (readlane) and rebuilt; the low half must
    be zero-extended (lane_u64, sparse_mla.hip). Sign-extending it turned every row whose low
    address word had bit 31 set into a wild address. Here the compressed cache is placed across a
    multiple of 2 GiB inside one allocation, so its rows' low words have bit 31 both set and clear,
    and the selected rows come from both sides."""
    from dsv41 import _abi
    from dsv41.layers import precompute_freqs_cis
    b, H, D, W, nb, K, start, rd = 1, 64, 512, 128, 8192, 512, 32767, 64
    row = D * 2
    big = torch.empty((1 << 31) + (16 << 20), dtype=torch.uint8, device=gpu)
    base = big.data_ptr()
    off = ((1 << 31) - base % (1 << 31) - nb * row // 2) % (1 << 31)   # the boundary at the cache's midpoint
    comp = big[off:off + nb * row].view(torch.bfloat16).view(b, nb, D)
    cross = ((base + off) // (1 << 31) + 1) * (1 << 31)
    assert comp.data_ptr() < cross < comp.data_ptr() + nb * row and comp.data_ptr() % 16 == 0
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 31)
    rn = lambda *s: torch.randn(*s, generator=g, device=gpu)   # noqa: E731
    sc = 576 ** -0.5
    comp.copy_((rn(b, nb, D) * sc).bfloat16())
    q, chunk, win, sink = (rn(b, 1, H, D) * sc).bfloat16(), (rn(b, 1, D) * sc).bfloat16(), \
        (rn(b, W, D) * sc).bfloat16(), rn(H)
    idx = _abi.topk_select(rn(b, 1, nb), K, start, 4, W + 1)
    pos = idx[0, 0].long() - (W + 1)
    first_after = (cross - comp.data_ptr()) // row
    assert (pos < first_after).any() and (pos >= first_after).any()
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
    out = _abi.sparse_mla(q, win, chunk, comp, nb, sink, idx, D ** -0.5, W, start, cos, sin, rd)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()   # noqa: E731
    slots = (start - W + np.arange(W)) % W
    kv_all = np.concatenate([f(win)[:, slots], f(chunk), f(comp)], axis=1)
    widx = R.window_idx_matrix(W, 1, W)[None]
    o = R.sparse_attn(f(q), kv_all, f(sink), np.concatenate([widx, f(idx).astype(np.int32)], -1), D ** -0.5,
                      dtype="bf16")
    rc, rs = R.precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1)
    want = R.rope_tail(o, rd, rc[[start]], rs[[start]], inverse=True, dtype="bf16")
    assert_attn_close(to_np(out), want)
    del big


# ------------------------------------------------------------------ fp8 caches in 32 x 32 blocks


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fp8_writers_with_32_row_scale_blocks(gpu, dt):
    """The fp8 writers with one scale per 32 channels of every 32 rows: a prefill of 70 rows
    (blocks opened at rows 0, 32, 64: two launches, openers first), then single-row appends that
    continue block 2 and open block 3. Every stored value equals the oracle's block-row store of
    the GPU's own roped (and normed) values: bit-exact codes and scales."""
    from dsv41 import _abi
    rng = rng_for("w8b" + dt)
    rc, rs = R.precompute_freqs_cis(64, 4096, 65536, 160000.0, 16.0, 32, 1)
    b, d, di, r = 2, 512, 128, 4
    cos, sin = dev(rc), dev(rs)
    codes = torch.zeros(b, 128, d, dtype=torch.uint8, device=gpu)
    scales = torch.zeros(b, 4, d // 32, dtype=torch.uint8, device=gpu)
    kc = torch.zeros(b, 128, di, dtype=torch.uint8, device=gpu)
    ks = torch.zeros(b, 4, di // 32, dtype=torch.uint8, device=gpu)
    nw = dev((1 + 0.1 * rng.standard_normal(di)).astype(F32))
    want_v, want_k, sc_v, sc_k = [], [], None, None
    for g0, g in ((0, 70), (70, 1), (71, 1), (95, 1), (96, 1), (97, 1)):
        lat = dev(R.cast(rng.standard_normal((b, g, d)).astype(F32) * (1 + g0 % 7), dt), dt)
        kr = dev(R.cast(rng.standard_normal((b, g, di)).astype(F32), dt), dt)
        _abi.comp_write_fp8(lat, codes, scales, g0, r, cos, sin, 64, scale_rb=32)
        _abi.index_key_publish_fp8(kr, kc, ks, g0, r, nw, cos, sin, 64, 1e-20, scale_rb=32)
        roped = to_np(_abi.rope_tail(lat, 64, cos, sin, g0 * r, r))
        keyed = to_np(_abi.rope_tail(_abi.rmsnorm(kr, nw, 1e-20), 64, cos, sin, g0 * r, r))
        v, sc_v = R.fp8_block_rows(roped, g0, 32, sc_v)
        k, sc_k = R.fp8_block_rows(keyed, g0, 32, sc_k)
        want_v.append(v)
        want_k.append(k)
    torch.cuda.synchronize()
    written = list(range(72)) + [95, 96, 97]
    got_v = R.dequant_fp8_cache(codes.cpu().numpy()[:, :98], scales.cpu().numpy(), 32)[:, written]
    got_k = R.dequant_fp8_cache(kc.cpu().numpy()[:, :98], ks.cpu().numpy(), 32)[:, written]
    assert np.array_equal(got_v, np.concatenate(want_v, 1))
    assert np.array_equal(got_k, np.concatenate(want_k, 1))
    # the stored scale bytes are the oracle's block scales; rows never written stay zero
    assert np.array_equal(np.ldexp(1.0, scales.cpu().numpy().astype(np.int32) - 127).astype(F32), sc_v)
    assert not codes[:, 72:95].any() and not codes[:, 98:].any()


def _fp8_keys(g, b, rows, rb, device, pad=True):
    codes = torch.randint(0, 256, (b, rows, 128), generator=g, device=device, dtype=torch.int32)
    codes = torch.where((codes & 0x7F) == 0x7F, codes ^ 1, codes).to(torch.uint8)     # no NaN codes
    nblk = -(-rows // rb)
    scales = torch.randint(123, 132, (b, (nblk + 3) // 4 * 4 if pad else nblk, 4), generator=g, device=device,
                           dtype=torch.int32).to(torch.uint8)
    return codes, scales


@pytest.mark.parametrize("b,n,h,nb,start,rb,use_cand", [
    (16, 1, 64, 32768, 131071, 32, False),   # the fp8 decode line: bs16, 128K context, 32 x 32 blocks
    (16, 1, 64, 32768, 131071, 1, False),    # per-row scales
    (3, 5, 32, 1000, 3990, 1, True),         # causal rows, candidates
    (2, 40, 16, 700, 2700, 32, False),       # prefill-sized, most rows visible
])
def test_indexer_score_mxq_fp8(gpu, b, n, h, nb, start, rb, use_cand):
    """Block-scaled MFMA with the MXFP4 query (fp4) against fp8 keys: within 1e-4 max|S| of the
    oracle on the decoded query and keys and of the dequantizing fp8 scorer (exact) on the same
    values -- the instruction's sums carry a few 1e-5 of relative error."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 48 + rb + n)
    d, r = 128, 4
    cos, sin = (t.to(gpu) for t in (torch.ones(start + n, 32), torch.zeros(start + n, 32)))   # identity rope
    q_raw = (torch.randn(b, n, h, d, generator=g, device=gpu) * 0.7).bfloat16()
    q_mx = _abi.index_q_prep_mxfp4(q_raw, cos, sin, 64, start)
    q16 = _abi.index_q_prep(q_raw.clone(), cos, sin, 64, start)                             # the same values
    w = torch.randn(b, n, h, generator=g, device=gpu).bfloat16()
    codes, scales = _fp8_keys(g, b, nb + 3, rb, gpu)
    cand = (torch.rand(b, n, nb, generator=g, device=gpu) < 0.7) if use_cand else None
    ws = weight_scale(h, d, torch.bfloat16)
    got = _abi.indexer_score_mxq_fp8(q_mx, w, ws, codes, scales, rb, nb, start, r, cand)
    ref8 = _abi.indexer_score_fp8(q16, w, ws, codes, scales, rb, nb, start, r, cand)
    torch.cuda.synchronize()
    keys = R.dequant_fp8_cache(codes.cpu().numpy(), scales.cpu().numpy(), rb)[:, :nb]
    wv = R.cast(to_np(w) * F32(ws), "bf16")
    want = R.indexer_scores(R.mxfp4_decode(q_mx[0].cpu().numpy(), q_mx[1].cpu().numpy()), keys, wv, start, r,
                            cand.cpu().numpy() if use_cand else None)
    gv, g8 = to_np(got), to_np(ref8)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(gv), fin) and np.array_equal(np.isfinite(g8), fin)
    scale = max(np.abs(want[fin]).max(), 1.0)
    err = np.abs(gv[fin] - want[fin]).max() / scale
    print(f"[mxq_fp8] max |score - exact| / max|S| = {err:.2e}", flush=True)
    assert err <= 1e-4
    assert np.abs(g8[fin] - want[fin]).max() <= 1e-5 * scale           # the exact path
    assert np.abs(gv[fin] - g8[fin]).max() <= 1e-4 * scale


@pytest.mark.parametrize("b,n,h,nb,topk,start,rb,use_cand", [
    (16, 1, 64, 32768, 1024, 131071, 32, False),   # the C5 layer shape: top-1024 of 32K entries
    (16, 1, 64, 32768, 512, 131071, 32, True),     # a candidate-masked consumer
    (8, 4, 16, 16384, 512, 20000, 1, False),       # causal rows, ranges past visibility
])
def test_indexer_topk_mxq_fp8_equals_two_calls(gpu, b, n, h, nb, topk, start, rb, use_cand):
    from dsv41 import _abi
    g = torch.Generator(gpu).manual_seed(SEED_BASE + 49)
    q_mx = (torch.randint(0, 256, (b, n, h, 64), generator=g, device=gpu, dtype=torch.int32).to(torch.uint8),
            torch.randint(120, 130, (b, n, h, 4), generator=g, device=gpu, dtype=torch.int32).to(torch.uint8))
    w = torch.randn(b, n, h, generator=g, device=gpu).bfloat16()
    codes, scales = _fp8_keys(g, b, nb, rb, gpu)
    cand = (torch.rand(b, n, nb, generator=g, device=gpu) < 0.7) if use_cand else None
    fused = _abi.indexer_topk_mxq_fp8(q_mx, w, 0.01, codes, scales, rb, nb, start, 4, topk, 129, cand)
    if fused is None:                                    # k above a quarter of a range: two calls
        assert _abi.indexer_topk_workspace_bytes(b, n, h, 128, nb, topk, use_cand) == 0
        return
    scores = _abi.indexer_score_mxq_fp8(q_mx, w, 0.01, codes, scales, rb, nb, start, 4, cand)
    assert torch.equal(fused, _abi.topk_select(scores, topk, start, 4, 129))


# ------------------------------------------------------------------ grouped output LoRA


@pytest.mark.parametrize("rows,groups,d,r,dt", [
    (1, 8, 4096, 1024, "bf16"),       # the release's output LoRA, one decode row
    (32, 8, 4096, 1024, "bf16"),      # bs32 decode
    (37, 8, 4096, 1024, "bf16"),      # a partial 16-row tile
    (64, 8, 4096, 1024, "bf16"),
    (70, 8, 4096, 1024, "bf16"),      # three 32-row query tiles, a partial one
    (100, 2, 512, 128, "bf16"),       # four 32-row query tiles, a partial one
    (64, 1, 5120, 1280, "bf16"),      # one group: a dense projection's shape
    (32, 1, 1280, 8192, "bf16"),      # the indexer's query projection at decode (d not a multiple of 512)
    (128, 8, 4096, 1024, "bf16"),
    (129, 8, 4096, 1024, "bf16"),     # the tiled kernel, a partial 256-row query tile
    (257, 8, 4096, 1024, "bf16"),     # one row in the second 256-row query tile
    (700, 4, 1024, 256, "bf16"),
    (300, 2, 512, 384, "bf16"),       # r not a multiple of 256: the 128 x 128 tiles
    (2048, 8, 4096, 1024, "bf16"),    # a prefill chunk
    (9, 2, 128, 16, "bf16"),          # a test configuration's shape: the plain kernel
    (9, 2, 128, 16, "f32"),
    (40, 8, 512, 128, "f32"),         # fp32 activations: the plain kernel
])
def test_wo_a_grouped(gpu, rows, groups, d, r, dt):
    """dsv41_wo_a_grouped = the reference's einsum("bsgd,grd->bsgr") on fp32 copies, cast back
    (attention.py:176-179). Against a float64 product of the same values: every fp32 output
    within 2e-5 of sum_k |o_k w_k| (fp32 sums; bf16 products are exact); the bf16 output is the
    fp32 output rounded once, bit for bit; repeated calls are bit-identical."""
    from dsv41 import _abi
    g = torch.Generator(device=gpu).manual_seed(SEED_BASE + rows + d)
    tdt = DT[dt]
    o = torch.randn(rows, groups * d, generator=g, device=gpu).to(tdt)
    w = (torch.randn(groups * r, d, generator=g, device=gpu) * 0.02).to(tdt)
    got32 = _abi.wo_a_grouped(o, w, groups, out_dtype=torch.float32)
    got = _abi.wo_a_grouped(o, w, groups)
    again = _abi.wo_a_grouped(o, w, groups)
    torch.cuda.synchronize()
    assert got.dtype == tdt and got.shape == (rows, groups * r)
    o64 = o.double().view(rows, groups, d).transpose(0, 1).contiguous()    # [G, rows, d]
    w64 = w.double().view(groups, r, d).transpose(1, 2).contiguous()       # [G, d, r]
    ref = torch.bmm(o64, w64).transpose(0, 1).reshape(rows, groups * r)
    mag = torch.bmm(o64.abs(), w64.abs()).transpose(0, 1).reshape(rows, groups * r)
    err = ((got32.double() - ref).abs() / mag.clamp_min(1e-30)).max().item()
    assert err < 2e-5, f"fp32 sums off by {err:.2e} of sum |o w|"
    assert torch.equal(got, got32.to(tdt)), "the output is the fp32 result rounded once"
    assert torch.equal(got, again), "repeated calls differ"
    if dt == "bf16":                   # and so mostly equal to the float64 result rounded once
        assert (got != ref.to(tdt)).float().mean().item() < 2e-3


@pytest.mark.parametrize("rows,k,n,splits", [
    (64, 5120, 1280, None),       # wq_a at the C4 batch (8 contraction ranges)
    (32, 5120, 512, None),        # wkv at bs32 (16 ranges)
    (1, 5120, 1792, None),        # one decode row, wq_a + wkv's width
    (100, 1280, 8192, None),      # the indexer's wq_b, a partial 32-row query tile (one range)
    (64, 5120, 1280, 1),          # no split: the kernel stores bf16 itself
    (37, 640, 96, 5),             # odd row count, n a multiple of 32 only
    (64, 8192, 5120, None),       # wo_b at the C4 batch: 160-row tiles, 8 ranges (256 workgroups)
    (40, 8192, 5120, 4),          # the same on 128-row tiles (4 ranges: 160 workgroups), 40 rows
    (48, 1280, 32768, None),      # wq_b at 48 rows: 128-row tiles, one range, partial query tile
    (64, 2048, 16384, 2),         # 128-row tiles over 2 ranges
    (64, 5120, 64, None),         # the indexer's weights_proj: 2 tiles x 40 ranges
])
def test_linear_rows(gpu, rows, k, n, splits):
    """dsv41_linear_rows = nn.Linear (x @ w^T) at decode rows: against a float64 product of the
    same values every output within one bf16 step of the exact sum (bf16 products are exact,
    fp32 sums per contraction range, then the ranges in order, rounded once), most outputs equal
    to the float64 result rounded once; repeat calls bit-identical."""
    from dsv41 import _abi
    g = torch.Generator(device=gpu).manual_seed(SEED_BASE + rows + k + n)
    x = torch.randn(rows, k, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    got = _abi.linear_rows(x, w, splits)
    again = _abi.linear_rows(x, w, splits)
    torch.cuda.synchronize()
    assert got.shape == (rows, n) and got.dtype == torch.bfloat16
    assert torch.equal(got, again), "repeated calls differ"
    ref = x.double() @ w.double().t()
    mag = x.double().abs() @ w.double().abs().t()
    err = ((got.double() - ref).abs() - ref.abs() * 2.0 ** -8).clamp_min(0) / mag.clamp_min(1e-30)
    assert err.max().item() < 2e-5, f"beyond one bf16 rounding: {err.max().item():.2e} of sum |x w|"
    assert (got != ref.to(torch.bfloat16)).float().mean().item() < 2e-3


@pytest.mark.parametrize("rows,k,n0,n1,splits", [
    (64, 5120, 1280, 512, None),  # wq_a + wkv at the C4 batch (4 ranges)
    (1, 5120, 1280, 512, None),   # one decode row
    (37, 640, 96, 64, 5),         # odd row count, widths multiples of 32 only
    (64, 2048, 8192, 8192, 2),    # 128-row tiles, the boundary between the weights on a tile edge
    (64, 2048, 8160, 8224, 2),    # a boundary inside a 128-row tile: 32-row tiles instead
])
def test_linear_rows_pair(gpu, rows, k, n0, n1, splits):
    """dsv41_linear_rows_pair (wq_a(x), wkv(x) in one launch): each output bit-identical to
    dsv41_linear_rows on its own weight with the same ranges, and within one bf16 step of a float64
    product of the same values."""
    from dsv41 import _abi
    g = torch.Generator(device=gpu).manual_seed(SEED_BASE + 11 * rows + k + n0 + 3 * n1)
    x = torch.randn(rows, k, generator=g, device=gpu).to(torch.bfloat16)
    w0 = (torch.randn(n0, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    w1 = (torch.randn(n1, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    if splits is None:
        splits = max(_abi.linear_rows_splits(k, n0 + n1, rows), 2)
    y0, y1 = _abi.linear_rows_pair(x, w0, w1, splits)
    torch.cuda.synchronize()
    assert y0.shape == (rows, n0) and y1.shape == (rows, n1)
    assert torch.equal(y0, _abi.linear_rows(x, w0, splits)), "first output differs from the single call"
    assert torch.equal(y1, _abi.linear_rows(x, w1, splits)), "second output differs from the single call"
    for got, w in ((y0, w0), (y1, w1)):
        ref = x.double() @ w.double().t()
        mag = x.double().abs() @ w.double().abs().t()
        err = ((got.double() - ref).abs() - ref.abs() * 2.0 ** -8).clamp_min(0) / mag.clamp_min(1e-30)
        assert err.max().item() < 2e-5


@pytest.mark.parametrize("rows", [1, 4, 300])
def test_attention_wo_a_fp32_at_release_shape(gpu, rows):
    """An fp32 layer at the release's output-LoRA shape (8 groups x (4096 -> 1024)) takes one fp32
    GEMM per group from two rows on and the grouped kernel below that; either way the result is
    the reference's fp32 einsum (attention.py:176-179) within 2e-5 of sum_k |o_k w_k| of a float64
    product of the same values."""
    from dsv41.attention import Attention
    from dsv41.config import ModelArgs
    a = ModelArgs(n_layers=1, compress_ratios=(0,))
    attn = Attention(0, a, torch.float32, gpu)
    g = torch.Generator(device=gpu).manual_seed(SEED_BASE + 70 + rows)
    attn.wo_a.weight.copy_(torch.randn(attn.wo_a.weight.shape, generator=g, device=gpu) * 0.02)
    o = torch.randn(1, rows, a.n_heads * a.head_dim, generator=g, device=gpu)
    got = attn._wo_a(o, torch.float32)
    torch.cuda.synchronize()
    G, r, d = a.o_groups, a.o_lora_rank, a.n_heads * a.head_dim // a.o_groups
    o64 = o.double().view(rows, G, d).transpose(0, 1).contiguous()
    w64 = attn.wo_a.weight.double().view(G, r, d).transpose(1, 2).contiguous()
    ref = torch.bmm(o64, w64).transpose(0, 1).reshape(1, rows, G * r)
    mag = torch.bmm(o64.abs(), w64.abs()).transpose(0, 1).reshape(1, rows, G * r)
    assert got.shape == ref.shape and got.dtype == torch.float32
    assert ((got.double() - ref).abs() / mag.clamp_min(1e-30)).max().item() < 2e-5
