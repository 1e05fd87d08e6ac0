"""The decode hot path of one compressing attention layer as a fixed-shape step.

One step = indexer scoring of every visible compressed entry (MFMA) -> top-k selection ->
sparse MLA over the window ring, this token's KV and the selected compressed entries, with
q's rope tail applied as the attention loads q and the inverse rope on the output -- i.e.
attention.py:117 and 143-175 minus the projections, the cache writes and the fake-quant
prologues, which are per-token elementwise work.

All outputs and scratch are allocated once, so a step issues exactly three kernels (four
when the attention splits its index list) and can be captured in a HIP graph. Where the fused
indexer form serves the shape (bf16 keys, 16/32/64 index heads of 128 channels, 2048 or 4096
scored entries per workgroup), scoring and selection are dsv41_indexer_topk: the scoring kernel
keeps each row range's best top-k and a merge kernel selects from those lists, so the
[b, 1, nb] scores are never written; the selection is bit-equal to the two-call form.
"""

from __future__ import annotations

import torch

from . import _abi


class SparseDecodeStep:
    def __init__(self, bsz: int, heads: int, head_dim: int, rd: int, index_heads: int,
                 index_dim: int, nb: int, index_topk: int, window: int, start_pos: int,
                 ratio: int, dtype=torch.bfloat16, device="cuda", fused: bool = True):
        self.bsz, self.heads, self.head_dim, self.rd = bsz, heads, head_dim, rd
        self.index_heads, self.index_dim = index_heads, index_dim
        self.nb, self.topk, self.window = nb, index_topk, window
        self.start_pos, self.ratio = start_pos, ratio
        self.dtype = dtype
        self.wp = min(start_pos, window)
        self.offset = self.wp + 1
        self.k = min(index_topk, nb)
        fws = (_abi.indexer_topk_workspace_bytes(bsz, 1, index_heads, index_dim, nb, index_topk)
               if fused and dtype == torch.bfloat16 else 0)
        self.fused = fws > 0
        # the scores are written only by the two-call form (fused False or a shape it does not serve)
        self.scores = torch.empty(bsz, 1, nb, dtype=torch.float32, device=device)
        self.idx = torch.empty(bsz, 1, self.k, dtype=torch.int32, device=device)
        self.fused_ws = torch.empty(max(fws, 1), dtype=torch.uint8, device=device)
        tws = 0 if self.fused else _abi.topk_workspace_bytes(bsz, nb, index_topk)
        self.topk_ws = torch.empty(max(tws, 1), dtype=torch.uint8, device=device)
        self.out = torch.empty(bsz, 1, heads, head_dim, dtype=dtype, device=device)
        rows = min(window, self.wp + 1) + self.k
        ws = _abi.mla_workspace_bytes(bsz, 1, heads, head_dim, rows, dtype)
        self.workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=device)

    def __call__(self, q, index_q, w_raw, w_scale, index_k, comp_kv, win_kv, chunk_kv, sink,
                 cos, sin):
        """q [b,1,H,D] as wq_b gives it (the attention launch applies its rope tail);
        index_q [b,1,Hi,Di] (already roped + fake-quantized); w_raw [b,1,Hi];
        index_k / comp_kv: the owner's caches ([b, >=nb, *] views, read in place);
        win_kv [b, window, D] ring of the previous tokens; chunk_kv [b,1,D] this token's KV."""
        keys = index_k[:, :self.nb]
        if self.fused:
            idx = _abi.indexer_topk(index_q, w_raw, w_scale, keys, self.start_pos, self.ratio, self.topk,
                                    self.offset, None, out=self.idx, workspace=self.fused_ws)
        else:
            _abi.indexer_score(index_q, w_raw, w_scale, keys, self.start_pos, self.ratio, None, out=self.scores)
            idx = _abi.topk_select(self.scores, self.topk, self.start_pos, self.ratio, self.offset,
                                   workspace=self.topk_ws, out=self.idx)
        _abi.sparse_mla(q, win_kv, chunk_kv, comp_kv, self.nb, sink, idx, self.head_dim ** -0.5,
                        self.window, self.start_pos, cos, sin, self.rd, out=self.out,
                        workspace=self.workspace, q_rd=self.rd)
        return self.out, idx


class _LayerPlan:
    __slots__ = ("layer_id", "ratio", "kv_source", "index_source", "owns_k", "candidate_source",
                 "uses_candidates", "cos", "sin", "out", "idx", "fused_idx")


class StackDecodeStep:
    """One decode token through every layer of an attention-only stack, kernels only.

    Per layer this is the kernel sequence of attention.py:106-175 with the projections left
    out (as in ``SparseDecodeStep``): the owners store the token's completed group (latent ->
    rope -> fp4/e4m3 fake-quant into comp_kv; key -> k_norm -> rope -> fp4/ue8m0 into
    index_k), index sources score their queries against the most recent key owner's cache
    (layers after the candidate source with its block mask applied) and select the top-k, and
    every layer attends over its window ring, this token's KV and the most recent owner's
    comp_kv in place and, in the same launch, writes the token into its ring. The sharing
    follows the layer loop of model.py:141-154: the most recent kv source, key owner, top-k
    selection and candidate mask are handed down the stack.

    ``inputs[l]`` holds layer l's per-token tensors: ``q`` [b,1,H,D] (wq_b's output: the
    attention launch applies its rope tail), ``kv`` [b,1,D]
    (the window KV after its prologue), ``sink`` [H]; index sources add ``index_q``
    [b,1,Hi,Di] (roped, fake-quantized) -- or, when the key owners' caches are MXFP4,
    ``index_q_mx`` (its codes and scales from dsv41_index_q_prep_mxfp4) --, ``w_raw`` [b,1,Hi]
    and ``w_scale``; kv sources add ``latent`` [b,1,D] (pre-rope); key owners add ``k_raw``
    [b,1,Di] and ``k_norm`` [Di]. Caches may be dense, carry MXFP4 index keys, hold the
    compressed KV packed (cache_format "fp4": e2m1 codes + e4m3 scales per 16 channels) and the
    window ring too ("packed": MXFP8 rows), or be the fp8 variant (cache_format "fp8": fp8
    compressed KV and index keys, with ue8m0 scales per 32 channels of each row or of 32-row
    blocks); each layer takes the kernels that read and
    write its owners' format. Over fp8 keys an index source given ``index_q_mx`` scores on the
    block-scaled fp4 x fp8 MFMA (dsv41_indexer_*_mxq_fp8), else it dequantizes the keys for the
    bf16 MFMA. On every key format, index sources other than the candidate source score and
    select in the fused form (dsv41_indexer_topk(_fp8, _mxfp4, _mxq_fp8)) where it serves the
    shape; the candidate source writes its scores for the block mask (kept in ``candidates``).
    Outputs (``out`` per layer) and scratch are allocated once, so a step can be captured in
    a HIP graph.
    """

    def __init__(self, args, bsz: int, start_pos: int, dtype=torch.bfloat16, device="cuda"):
        from .layers import yarn_inv_freqs

        self.args, self.bsz, self.start_pos, self.dtype = args, bsz, start_pos, dtype
        dev = torch.device(device)
        self.end_pos = start_pos + 1
        self.window = args.window_size
        self.wp = min(start_pos, self.window)
        self.offset = self.wp + 1
        self.scale = args.head_dim ** -0.5
        tables = {}

        def table(ratio):
            key = bool(ratio)
            if key not in tables:
                orig, theta = (args.original_seq_len, args.compress_rope_theta) if ratio else (0, args.rope_theta)
                f = torch.from_numpy(yarn_inv_freqs(args.rope_head_dim, orig, theta, args.rope_factor,
                                                    args.beta_fast, args.beta_slow)).to(dev)
                tables[key] = _abi.rope_table(f, self.end_pos)
            return tables[key]

        self.plan = []
        max_rows, max_nb, max_fws = 1, 1, 1
        for l in range(args.n_layers):
            p = _LayerPlan()
            p.layer_id = l
            p.ratio = args.compress_ratio(l)
            p.kv_source = l in args.kv_source_layers
            p.index_source = p.ratio > 0 and l in args.index_source_layers
            p.owns_k = p.index_source and p.kv_source
            p.candidate_source = p.index_source and l == args.candidate_source_layer
            p.uses_candidates = p.index_source and 0 <= args.candidate_source_layer < l
            p.cos, p.sin = table(p.ratio)
            p.out = torch.empty(bsz, 1, args.n_heads, args.head_dim, dtype=dtype, device=dev)
            p.idx = None                                   # an index source's last selection
            p.fused_idx = None
            if p.ratio:
                nb = self.end_pos // p.ratio
                max_nb = max(max_nb, nb)
                max_rows = max(max_rows, min(self.window, self.wp + 1) + min(args.index_topk, nb))
                if p.index_source and not p.candidate_source and dtype == torch.bfloat16:
                    fws = _abi.indexer_topk_workspace_bytes(bsz, 1, args.index_n_heads, args.index_head_dim, nb,
                                                            args.index_topk, p.uses_candidates)
                    if fws > 0:                    # bf16 keys take the fused indexer + top-k form
                        max_fws = max(max_fws, fws)
                        p.fused_idx = torch.empty(bsz, 1, min(args.index_topk, nb), dtype=torch.int32, device=dev)
            self.plan.append(p)
        self.scores = torch.empty(bsz * max_nb, dtype=torch.float32, device=dev)   # [b, 1, nb] per layer
        self.fused_ws = torch.empty(max_fws, dtype=torch.uint8, device=dev)
        self.candidates = None                             # the candidate source's last block mask
        ws = _abi.mla_workspace_bytes(bsz, 1, args.n_heads, args.head_dim, max_rows, dtype)
        self.workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=dev)

    def __call__(self, cache, inputs):
        """cache: a ``ModelCache`` for ``bsz`` rows; returns the per-layer outputs."""
        a, sp, b = self.args, self.start_pos, self.bsz
        kv_src = key_src = topk = cand = None
        for p in self.plan:
            x = inputs[p.layer_id]
            lc = cache.layers[p.layer_id]
            comp, n_comp, idx, comp_kind = None, 0, None, "dense"
            if p.ratio:
                nb = self.end_pos // p.ratio
                emits = self.end_pos % p.ratio == 0       # this token completes group nb - 1
                if p.kv_source:
                    kv_src = lc
                if p.index_source:
                    if p.owns_k:
                        if emits and lc.index_k8 is not None:
                            _abi.index_key_publish_fp8(x["k_raw"], lc.index_k8, lc.index_k8s, nb - 1, p.ratio,
                                                       x["k_norm"], p.cos, p.sin, a.rope_head_dim, a.norm_eps,
                                                       lc.fp8_rb)
                        elif emits and lc.index_k4 is not None:
                            _abi.index_key_publish_mxfp4(x["k_raw"], lc.index_k4, lc.index_ks, nb - 1, p.ratio,
                                                         x["k_norm"], p.cos, p.sin, a.rope_head_dim, a.norm_eps)
                        elif emits:
                            _abi.index_key_publish(x["k_raw"], lc.index_k, nb - 1, p.ratio, x["k_norm"],
                                                   p.cos, p.sin, a.rope_head_dim, a.norm_eps)
                        key_src = lc
                    scores = self.scores[:b * nb].view(b, 1, nb)
                    keys = key_src.index_keys(b, nb)
                    c = cand if p.uses_candidates else None
                    kind = getattr(keys, "kind", None)
                    sel = None                     # the fused form's selection, where it serves the layer
                    if p.fused_idx is not None and kind is None:
                        sel = _abi.indexer_topk(x["index_q"], x["w_raw"], x["w_scale"], keys, sp, p.ratio,
                                                a.index_topk, self.offset, c, out=p.fused_idx, workspace=self.fused_ws)
                    elif p.fused_idx is not None and kind == "mxfp4":
                        sel = _abi.indexer_topk_mxfp4(x["index_q_mx"], x["w_raw"], x["w_scale"], keys.codes,
                                                      keys.scales, nb, sp, p.ratio, a.index_topk, self.offset, c,
                                                      out=p.fused_idx, workspace=self.fused_ws)
                    elif p.fused_idx is not None and kind == "fp8" and "index_q_mx" in x:
                        sel = _abi.indexer_topk_mxq_fp8(x["index_q_mx"], x["w_raw"], x["w_scale"], keys.codes,
                                                        keys.scales, keys.rb, nb, sp, p.ratio, a.index_topk,
                                                        self.offset, c, out=p.fused_idx, workspace=self.fused_ws)
                    elif p.fused_idx is not None and kind == "fp8":
                        sel = _abi.indexer_topk_fp8(x["index_q"], x["w_raw"], x["w_scale"], keys.codes, keys.scales,
                                                    keys.rb, nb, sp, p.ratio, a.index_topk, self.offset, c,
                                                    out=p.fused_idx, workspace=self.fused_ws)
                    if sel is not None:
                        topk = p.idx = sel
                    else:
                        if kind == "mxfp4":
                            _abi.indexer_score_mxfp4(x["index_q_mx"], x["w_raw"], x["w_scale"], keys.codes,
                                                     keys.scales, nb, sp, p.ratio, c, out=scores)
                        elif kind == "fp8" and "index_q_mx" in x:
                            _abi.indexer_score_mxq_fp8(x["index_q_mx"], x["w_raw"], x["w_scale"], keys.codes,
                                                       keys.scales, keys.rb, nb, sp, p.ratio, c, out=scores)
                        elif kind == "fp8":
                            _abi.indexer_score_fp8(x["index_q"], x["w_raw"], x["w_scale"], keys.codes, keys.scales,
                                                   keys.rb, nb, sp, p.ratio, c, out=scores)
                        else:
                            _abi.indexer_score(x["index_q"], x["w_raw"], x["w_scale"], keys, sp, p.ratio, c,
                                               out=scores)
                        if p.candidate_source:
                            cand = self.candidates = _abi.candidate_blocks(scores, a.candidate_topk_blocks,
                                                                           a.candidate_block_size, None, sp, p.ratio)
                        topk = p.idx = _abi.topk_select(scores, a.index_topk, sp, p.ratio, self.offset)
                if p.kv_source and emits and lc.comp_kv8 is not None:
                    _abi.comp_write_fp8(x["latent"], lc.comp_kv8, lc.comp_ks, nb - 1, p.ratio, p.cos, p.sin,
                                        a.rope_head_dim, lc.fp8_rb)
                elif p.kv_source and emits and lc.comp_kv4 is not None:
                    _abi.comp_write_fp4(x["latent"], lc.comp_kv4, nb - 1, p.ratio, p.cos, p.sin, a.rope_head_dim)
                elif p.kv_source and emits:
                    _abi.comp_write(x["latent"], lc.comp_kv, nb - 1, p.ratio, p.cos, p.sin, a.rope_head_dim)
                (comp_kind, comp), n_comp, idx = kv_src.comp_source(b), nb, topk
            # attention + this token's ring write in one launch
            if lc.win_kv8 is not None:
                _abi.sparse_mla_packed(x["q"], lc.win_kv8, x["kv"], comp if comp_kind == "fp4" else None, n_comp,
                                       x["sink"], idx, self.scale, self.window, sp, p.cos, p.sin, a.rope_head_dim,
                                       out=p.out, workspace=self.workspace, write_ring=True, q_rd=a.rope_head_dim)
            elif comp_kind == "fp8":
                _abi.sparse_mla_fp8(x["q"], lc.win_kv, x["kv"], comp, kv_src.comp_ks[:b], kv_src.fp8_rb, n_comp,
                                    x["sink"], idx, self.scale, self.window, sp, p.cos, p.sin, a.rope_head_dim,
                                    out=p.out, workspace=self.workspace, write_ring=True, q_rd=a.rope_head_dim)
            elif comp_kind == "fp4":
                _abi.sparse_mla_fp4(x["q"], lc.win_kv, x["kv"], comp, n_comp, x["sink"], idx, self.scale, self.window,
                                    sp, p.cos, p.sin, a.rope_head_dim, out=p.out, workspace=self.workspace,
                                    write_ring=True, q_rd=a.rope_head_dim)
            else:
                _abi.sparse_mla(x["q"], lc.win_kv, x["kv"], comp, n_comp, x["sink"], idx, self.scale, self.window,
                                sp, p.cos, p.sin, a.rope_head_dim, out=p.out, workspace=self.workspace,
                                write_ring=True, q_rd=a.rope_head_dim)
        return [p.out for p in self.plan]
