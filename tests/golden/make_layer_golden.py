"""Layer-composition fixtures from DeepSeek's torch attention (docs/reference/model.py).

Writes tests/golden/layer_golden.npz. CPU only; it runs where the reference tree exists (it is
read from REFERENCE below) and never on a GPU machine. The fixture holds data only: the
configs, the hidden-state inputs, and the reference's outputs.

What runs is the reference's own ``Attention`` / ``Compressor`` / ``Indexer`` classes
(model.py:429-789) over float32 weights, with:

* a ``kernel`` module written here for model.py's imports: ``act_quant`` and ``fp4_act_quant``
  as fake-quant round trips (the in-place semantics of kernel.py:40-204: block amax, power-of-two
  or e4m3 scale, e4m3 / e2m1 round to nearest even), ``sparse_attn`` as float64 softmax
  attention with the sink in the denominator (kernel.py:310-403). The fake-quant rounding here is
  a brute-force nearest-grid search and frexp scale, not the oracle's bit arithmetic;
* PIL stubbed (model.py imports image_processor, which attention never calls);
* the one adaptation the reference's own parity test declares for the indexer
  (tests/test_parity.py:116-129): a key owner's indexer reads its own key cache, instead of the
  process-wide pointer that an incomplete ratio-2 group leaves at the last owner.

The stack is attention only, as the oracle's ``AttentionStack``: h <- h + attn_l(norm_l(h)) with
the reference's RMSNorm. Weights are the oracle's seeded ``make_params`` arrays (data; the tests
regenerate them from the stored seed). Per config and per fake-quant setting (off / on) the
fixture stores: all-position outputs of prefills of several lengths from position 0, the
outputs of single-token decode steps after a prefill, and from the longest prefill the owners'
compressed-KV and index-key caches, and every index source's scores (as its top-k ranks them)
and selected compressed positions.

Configs carry 8 index heads (the reference test's count, tests/test_parity.py:73-76) so that
exact zero scores (ReLU) rarely tie at the top-k boundary, where torch.topk and the
lowest-index rule may choose different sets; the script checks that no selection it records
has a tie at its boundary.

    python tests/golden/make_layer_golden.py
"""

from __future__ import annotations

import json
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE = "/root/reference"
OUT = os.path.join(HERE, "layer_golden.npz")

sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from common import C1, RELEASE_TOY, TOPO  # noqa: E402
from oracle import cpu_ref as R            # noqa: E402  (only for the seeded weight arrays)

torch.set_default_dtype(torch.float32)

# ------------------------------------------------------------------ the kernel stand-in

QAT = {"on": True}
_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float64)


def _pow2_ceil(r: torch.Tensor) -> torch.Tensor:
    """2 ** ceil(log2 r) for r > 0, from frexp: r = m * 2^e with m in [0.5, 1)."""
    m, e = torch.frexp(r.double())
    e = torch.where(m == 0.5, e - 1, e)
    return torch.ldexp(torch.ones_like(r, dtype=torch.float64), e).float()


def _e2m1(v: torch.Tensor) -> torch.Tensor:
    """Nearest e2m1 value by exhaustive search over the grid; a tie takes the even code."""
    mag = v.double().abs()
    d = (mag.unsqueeze(-1) - _E2M1).abs()
    best = d.min(-1, keepdim=True).values
    cand = d == best
    even = (torch.arange(8) % 2 == 0)
    pick = (cand.double() * 2 + (cand & even).double()).argmax(-1)
    return (torch.sign(v.double()) * _E2M1[pick]).float()


def act_quant(x, block_size=128, scale_fmt=None, scale_dtype=None, inplace=False):
    assert inplace, "only the in-place fake-quant form runs in fp32 attention"
    if not QAT["on"]:
        return x
    xb = x.float().unflatten(-1, (-1, block_size))
    amax = xb.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    s = _pow2_ceil(amax * torch.tensor(1.0 / 448.0, dtype=torch.float32))
    q = (xb / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).float() * s
    x.copy_(q.flatten(-2).to(x.dtype))
    return x


def fp4_act_quant(x, block_size=32, inplace=False, scale_dtype=torch.float8_e8m0fnu):
    assert inplace
    if not QAT["on"]:
        return x
    xb = x.float().unflatten(-1, (-1, block_size))
    amax = xb.abs().amax(-1, keepdim=True)
    if scale_dtype == torch.float8_e4m3fn:
        s = (amax.clamp_min(6.0 * 2.0 ** -9) / 6.0).to(torch.float8_e4m3fn).float()
    else:
        s = _pow2_ceil(amax.clamp_min(6.0 * 2.0 ** -126) * torch.tensor(1.0 / 6.0, dtype=torch.float32))
    q = _e2m1((xb / s).clamp(-6.0, 6.0)) * s
    x.copy_(q.flatten(-2).to(x.dtype))
    return x


def sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale):
    b, m, h, d = q.shape
    idx = topk_idxs.long()
    valid = idx >= 0
    rows = torch.gather(kv.double().unsqueeze(1).expand(b, m, kv.size(1), d), 2,
                        idx.clamp(min=0).unsqueeze(-1).expand(b, m, idx.size(-1), d))
    logits = torch.einsum("bmhd,bmkd->bmhk", q.double(), rows) * softmax_scale
    logits = logits.masked_fill(~valid.unsqueeze(2), float("-inf"))
    mx = torch.maximum(logits.amax(-1, keepdim=True), attn_sink.double().view(1, 1, h, 1)).clamp_min(-1e30)
    w = torch.exp(logits - mx).masked_fill(~valid.unsqueeze(2), 0.0)
    den = w.sum(-1, keepdim=True) + torch.exp(attn_sink.double().view(1, 1, h, 1) - mx)
    return (torch.einsum("bmhk,bmkd->bmhd", w, rows) / den).to(q.dtype)


def _unused(*a, **k):
    raise NotImplementedError("not on the fp32 attention path")


kernel = types.ModuleType("kernel")
kernel.act_quant, kernel.fp4_act_quant, kernel.sparse_attn = act_quant, fp4_act_quant, sparse_attn
kernel.fp8_gemm = kernel.fp4_gemm = kernel.hc_split_sinkhorn = _unused

# ------------------------------------------------------------------ import the reference


def import_reference():
    sys.path.insert(0, os.path.join(REFERENCE, "docs", "reference"))
    pil = types.ModuleType("PIL")
    pil.Image = types.SimpleNamespace()
    pil.ImageOps = types.SimpleNamespace()
    sys.modules.setdefault("PIL", pil)
    sys.modules["kernel"] = kernel
    import model as REF
    REF.default_dtype = torch.float32
    orig = REF.Indexer.forward

    def own_keys(self, x, qr, latent, start_pos, offset):
        if self.owns_k:
            REF.shared_attn.index_k = self.k_cache
        return orig(self, x, qr, latent, start_pos, offset)

    REF.Indexer.forward = own_keys
    return REF


# ------------------------------------------------------------------ the attention-only stack

FIXTURES = {
    # C1 with the reference test's 8 index heads; 128-token prefill then 16 decode steps
    "c1": dict(cfg=dict(C1, index_n_heads=8), seed=101, B=1, prefill=(7, 33, 144), start=128, decode=16),
    "topo": dict(cfg=dict(TOPO, index_n_heads=8), seed=102, B=2, prefill=(7, 33, 48, 56), start=48, decode=8),
    "release": dict(cfg=dict(RELEASE_TOY), seed=104, B=2, prefill=(7, 33, 48, 56), start=48, decode=8),
}
_REF_ARGS = ("dim", "n_layers", "n_heads", "head_dim", "rope_head_dim", "q_lora_rank", "o_lora_rank", "o_groups",
             "window_size", "compress_ratios", "kv_source_layers", "index_source_layers",
             "candidate_source_layer", "candidate_topk_blocks", "candidate_block_size", "index_n_heads",
             "index_head_dim", "index_topk", "rope_theta", "compress_rope_theta", "original_seq_len", "rope_factor")


class RefStack:
    def __init__(self, REF, cfg, params, B):
        self.REF = REF
        kw = {k: cfg[k] for k in _REF_ARGS if k in cfg}
        rargs = REF.ModelArgs(max_batch_size=B, max_seq_len=cfg["max_seq_len"], dtype="bf16", expert_dtype=None,
                              n_mtp_layers=0, vision_n_layers=0, **kw)
        self.layers, self.norms = [], []
        with torch.no_grad():
            for i, p in enumerate(params):
                a = REF.Attention(i, rargs).float()
                self._load(a, p)
                n = REF.RMSNorm(cfg["dim"], rargs.norm_eps)
                n.weight.copy_(torch.from_numpy(p["attn_norm"]))
                self.layers.append(a)
                self.norms.append(n)
        REF.shared_attn = REF.SharedAttentionRuntime()
        self.picks = []

    @staticmethod
    def _load(a, p):
        def put(mod, arr):
            mod.weight.copy_(torch.from_numpy(np.asarray(arr, np.float32)))
        for name in ("wq_a", "wq_b", "wkv", "wo_a", "wo_b"):
            put(getattr(a, name), p[name])
        put(a.q_norm, p["q_norm"])
        put(a.kv_norm, p["kv_norm"])
        a.attn_sink.copy_(torch.from_numpy(p["attn_sink"]))
        if "compressor" in p:
            c = p["compressor"]
            put(a.compressor.wkv, c["wkv"])
            put(a.compressor.norm, c["norm"])
            if "wgate" in c:
                put(a.compressor.wgate, c["wgate"])
        if "indexer" in p:
            ix = p["indexer"]
            put(a.indexer.wq_b, ix["wq_b"])
            put(a.indexer.weights_proj, ix["weights_proj"])
            if "wk" in ix:
                put(a.indexer.wk, ix["wk"])
                put(a.indexer.k_norm, ix["k_norm"])

    def reset(self):
        """A fresh sequence: zero every cache the layers keep (the state a new model has)."""
        for a in self.layers:
            a.window_kv_cache.zero_()
            if a.compressor is not None and a.compress_ratio > 1:
                a.compressor.kv_state.zero_()
                a.compressor.score_state.fill_(float("-inf"))
            if a.is_kv_source:
                a.compress_kv_cache.zero_()
            if a.indexer is not None and a.indexer.owns_k:
                a.indexer.k_cache.zero_()

    def __call__(self, h, start_pos):
        x = torch.from_numpy(np.ascontiguousarray(h))
        with torch.no_grad():
            for a, n in zip(self.layers, self.norms):
                x = x + a(n(x), start_pos)
        return x.numpy()


def _boundary_ties(scores: torch.Tensor, k: int) -> int:
    """Rows whose k-th and (k+1)-th best finite scores are equal (a tie at the top-k boundary)."""
    if k >= scores.size(-1):
        return 0
    top = torch.sort(scores, dim=-1, descending=True).values[..., :k + 1]
    kth, nxt = top[..., k - 1], top[..., k]
    return int(((kth == nxt) & torch.isfinite(kth)).sum())


def run_fixture(REF, name, spec, out):
    cfg = spec["cfg"]
    a = R.Args(**cfg)
    params = R.make_params(a, spec["seed"])
    B = spec["B"]
    T = max(spec["prefill"])
    rng = np.random.default_rng(spec["seed"])
    h = rng.standard_normal((B, T, a.dim)).astype(np.float32)
    st = RefStack(REF, cfg, params, B)

    # the index sources' selections, as compressed positions (-1 kept); and a check that none of
    # the recorded selections has a tie at its boundary
    picks, scores, ties = [], [], [0]
    orig_topk = torch.Tensor.topk
    index_layers = [l for l in st.layers if l.indexer is not None]

    def forward_recording(self, x, qr, latent, start_pos, offset):
        def topk(t, k, *args, **kw):
            if t.dim() == 3 and t.dtype == torch.float32 and t.size(-1) == (start_pos + x.size(1)) // self.compress_ratio:
                ties[0] += _boundary_ties(t, k)
                scores.append(t.detach().clone().numpy())
            return orig_topk(t, k, *args, **kw)
        torch.Tensor.topk = topk
        try:
            idx = own(self, x, qr, latent, start_pos, offset)
        finally:
            torch.Tensor.topk = orig_topk
        picks.append(torch.where(idx >= 0, idx - offset, -1).numpy().astype(np.int32))
        return idx

    own = REF.Indexer.forward
    REF.Indexer.forward = forward_recording
    try:
        for qat in ("off", "on"):
            QAT["on"] = qat == "on"
            pre = f"{name}/{qat}/"
            for n in spec["prefill"]:
                st.reset()
                picks.clear()
                scores.clear()
                out[pre + f"prefill_{n}"] = st(h[:, :n], 0)
            # from the longest prefill: caches and selections
            for i, layer in enumerate(st.layers):
                r = layer.compress_ratio
                if layer.is_kv_source:
                    out[pre + f"comp_kv_{i}"] = layer.compress_kv_cache[:B, :T // r].numpy().copy()
                if layer.indexer is not None and layer.indexer.owns_k:
                    out[pre + f"index_k_{i}"] = layer.indexer.k_cache[:B, :T // r].numpy().copy()
            # the scores each index source ranks (after its candidate mask), and its selection
            for layer, sel, sc in zip(index_layers, picks, scores):
                out[pre + f"picks_{st.layers.index(layer)}"] = sel
                out[pre + f"scores_{st.layers.index(layer)}"] = sc
            # single-token decode steps after a prefill of `start` tokens
            s0 = spec["start"]
            st.reset()
            st(h[:, :s0], 0)
            dec = [st(h[:, t:t + 1], t) for t in range(s0, s0 + spec["decode"])]
            out[pre + "decode"] = np.concatenate(dec, axis=1)
    finally:
        REF.Indexer.forward = own
    assert ties[0] == 0, f"{name}: {ties[0]} top-k selections tie at their boundary; choose another seed"
    out[f"{name}/h"] = h
    out[f"{name}/spec"] = np.frombuffer(json.dumps(
        {"cfg": {k: list(v) if isinstance(v, tuple) else v for k, v in cfg.items()}, "seed": spec["seed"],
         "B": B, "prefill": list(spec["prefill"]), "start": spec["start"], "decode": spec["decode"]}).encode(),
        dtype=np.uint8)


def main():
    REF = import_reference()
    out = {}
    for name, spec in FIXTURES.items():
        run_fixture(REF, name, spec, out)
        print(f"{name}: {sum(v.nbytes for k, v in out.items() if k.startswith(name + '/'))} bytes")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
