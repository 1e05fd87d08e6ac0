"""Benchmark of the DeepSeek-V4.1 sparse-attention hot path on one MI355X.

Workload (the headline metric, "sparse-MLA decode tokens/s + HBM GB/s (% peak), bs32 64K ctx;
prefill TFLOP/s"): one decode step of one compressing attention layer at batch 32 and
65,536 tokens of context, i.e. 16,384 compressed entries per sequence (ratio 4), top-512,
64 heads x 512 (64-channel rope tail), indexer 64 heads x 128, window 128, bf16. A step is
indexer scoring of all 16,384 entries (MFMA) -> top-k -> sparse MLA over the 128 window
rows + 512 selected rows (+ inverse rope). Inputs are seeded synthetic tensors resident in
HBM; NSETS independent input sets (> 512 MB in total) rotate so the 256 MB Infinity Cache
cannot serve the streamed caches. Steps are replayed from HIP graphs (one graph holds one
step per input set), bracketed by events on the launch stream.

Secondary: C3 prefill (8,192-token chunk after 32,768 tokens, top-2,048) indexer and sparse
MLA TFLOP/s; the fp8-cache decode step (batch 16, 131,072 tokens, top-1,024, e4m3 caches with
ue8m0 block scales dequantized in-kernel); the 40-layer decode step of the C4 sharing topology
(batch 64, 65,536 tokens, kernels only); and the CPU oracle (numpy) timed on a bounded sample
of the decode workload.

    python bench.py [--steps K] [--warmup W] [--no-prefill] [--no-fp8] [--no-c4] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseek-v41-mlx_amd"))
sys.path.insert(0, ROOT)

METRIC = "sparse-MLA decode tokens/s + HBM GB/s (% peak), bs32 64K ctx; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
SEED = 20261201


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--ctx", type=int, default=65536)
    p.add_argument("--sets", type=int, default=4)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-fp8", action="store_true", help="skip the fp8-cache decode line")
    p.add_argument("--no-c4", action="store_true", help="skip the 40-layer decode line")
    p.add_argument("--no-mx", action="store_true", help="skip the MXFP4-index decode line")
    p.add_argument("--no-wo-a", action="store_true", help="skip the grouped output-LoRA line")
    p.add_argument("--no-token", action="store_true", help="skip the caller-path decode token line")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--eager", action="store_true",
                   help="launch the decode kernels without HIP graphs (for counter-collecting profilers)")
    p.add_argument("--calib-mb", type=int, default=0,
                   help="eager mode: also run a plain streaming copy of this many MB (read and write), "
                        "the reference kernel for scaling HBM byte counters")
    return p.parse_args()


# HBM bytes per indexer launch, from two rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE)
# scaled by the same counters over a copy of known size; the summary names its commands.
TRAFFIC_FILE = "profiles/indexer_topk_bs32_ctx64k_hbm_traffic.md"


def measured_traffic():
    path = os.path.join(ROOT, TRAFFIC_FILE)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Shape:
    def __init__(self, batch, ctx):
        self.B, self.H, self.D, self.rd = batch, 64, 512, 64
        self.Hi, self.Di, self.W, self.K, self.r = 64, 128, 128, 512, 4
        self.start = ctx                      # decoding the token at position ctx
        self.nb = (ctx + 1) // self.r         # visible compressed entries
        self.wp = min(self.start, self.W)
        self.rows = min(self.W, self.wp + 1) + min(self.K, self.nb)

    def bytes_indexer(self):
        return self.B * (self.nb * self.Di * 2 + self.Hi * self.Di * 2 + self.Hi * 2 + self.nb * 4)

    def bytes_indexer_topk(self):
        # the fused form: keys, q, w in, the top-k indices out (no scores)
        return self.B * (self.nb * self.Di * 2 + self.Hi * self.Di * 2 + self.Hi * 2 + self.K * 4)

    def bytes_topk(self):
        return self.B * (self.nb * 4 + self.K * 4)

    def bytes_sparse(self):
        return self.B * (self.rows * self.D * 2 + 2 * self.H * self.D * 2 + self.K * 4)

    def flops_indexer(self):
        return 2 * self.B * self.Hi * self.Di * self.nb

    def flops_sparse(self):
        return 4 * self.B * self.H * self.rows * self.D


def make_set(s: Shape, seed, device):
    """One input set: caches and queries N(0,1)/sqrt(576), fp4-grid index keys/queries, bf16."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16
    sc = 576 ** -0.5

    def fp4ish(*shape):
        # values on the fp4 e2m1 grid times a power of two: what the index caches hold
        grid = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], device=device)
        return (grid[torch.randint(0, 16, shape, generator=g, device=device)] * 0.25).to(bf)

    return dict(
        q=(torch.randn(s.B, 1, s.H, s.D, generator=g, device=device) * sc).to(bf),
        win=(torch.randn(s.B, s.W, s.D, generator=g, device=device) * sc).to(bf),
        chunk=(torch.randn(s.B, 1, s.D, generator=g, device=device) * sc).to(bf),
        comp=(torch.randn(s.B, s.nb, s.D, generator=g, device=device) * sc).to(bf),
        iq=fp4ish(s.B, 1, s.Hi, s.Di),
        ik=fp4ish(s.B, s.nb, s.Di),
        w=torch.randn(s.B, 1, s.Hi, generator=g, device=device).to(bf),
        sink=torch.randn(s.H, generator=g, device=device),
    )


def graph_of(fn, reps_sets, torch):
    """Capture fn(set) for every set in order into one graph (after one eager warm call of each
    distinct set)."""
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        seen = set()
        for d in reps_sets:
            if id(d) not in seen:
                seen.add(id(d))
                fn(d)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for d in reps_sets:
            fn(d)
    torch.cuda.synchronize()
    return gr


def upload_graph(gr, torch) -> int:
    """hipGraphUpload of a captured graph's executable on the current stream: the device-side
    set-up that a graph's first launch would otherwise pay for, with no step run. Returns the HIP
    status (0 = uploaded)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")   # the runtime torch has already loaded (same soname)
    fn = hip.hipGraphUpload
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    rc = fn(ctypes.c_void_p(gr.raw_cuda_graph_exec()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return int(rc)


def time_graph(gr, reps, torch):
    """Average ms per replay over `reps` replays, events on the current stream."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def run_decode(args, torch, device):
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis
    from dsv41.step import SparseDecodeStep

    s = Shape(args.batch, args.ctx)
    log(f"[bench] decode B={s.B} ctx={args.ctx} nb={s.nb} K={s.K} sets={args.sets}")
    sets = [make_set(s, SEED + i, device) for i in range(args.sets)]
    cos, sin = precompute_freqs_cis(s.rd, s.start + 1, 65536, 160000.0, 16.0, 32, 1, device=device)
    steps = [SparseDecodeStep(s.B, s.H, s.D, s.rd, s.Hi, s.Di, s.nb, s.K, s.W, s.start, s.r,
                              torch.bfloat16, device) for _ in sets]
    ws = weight_scale(s.Hi, s.Di, torch.bfloat16)
    for d, st in zip(sets, steps):
        d["step"] = st
    assert all(st.fused for st in steps), "the bs32 decode shape is served by the fused indexer + top-k form"

    def full(d):
        d["step"](d["q"], d["iq"], d["w"], ws, d["ik"], d["comp"], d["win"], d["chunk"], d["sink"], cos, sin)

    def only_fused(d):
        _abi.indexer_topk(d["iq"], d["w"], ws, d["ik"], s.start, s.r, s.K, s.wp + 1, None, out=d["step"].idx,
                          workspace=d["step"].fused_ws)

    def only_indexer(d):
        _abi.indexer_score(d["iq"], d["w"], ws, d["ik"], s.start, s.r, None, out=d["step"].scores)

    def only_topk(d):
        d["idx"] = _abi.topk_select(d["step"].scores, s.K, s.start, s.r, s.wp + 1)

    def only_sparse(d):
        _abi.sparse_mla(d["q"], d["win"], d["chunk"], d["comp"], s.nb, d["sink"], d["idx"], s.D ** -0.5, s.W,
                        s.start, cos, sin, s.rd, out=d["step"].out, workspace=d["step"].workspace)

    per_replay = len(sets)
    if args.eager:
        # plain launches: each step's three kernels issued from Python (host overhead included)
        for i in range(args.warmup):
            full(sets[i % per_replay])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            full(sets[i % per_replay])
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        log(f"[bench] eager decode step {ms * 1e3:.2f} us (host-bound timing)")
        if args.calib_mb:
            # the unfused entries too, so that counter passes over this run see every decode kernel
            for d in sets:
                only_indexer(d)
                only_topk(d)
            torch.cuda.synchronize()
            # plain streaming copy (elementwise kernel: N MB read, N MB written) for counter scaling
            n = args.calib_mb << 20
            src = torch.ones(n // 2, dtype=torch.bfloat16, device=device)
            dst = torch.empty_like(src)
            for _ in range(4):
                torch.neg(src, out=dst)
            torch.cuda.synchronize()
            log(f"[bench] calibration copy of {args.calib_mb} MB x4 done")
        kern = {k: float("nan") for k in ("indexer_topk", "indexer_score", "topk_select", "sparse_mla")}
        return s, ms, kern, sets, cos, sin, ws, [], []
    # exactly `warmup` untimed steps, then exactly `steps` timed steps, each graph cycling through
    # the input sets in order. Both graphs are captured first (the timed one uploaded, no step
    # run), so the warm-up steps run right before the timed ones: a capture between them leaves
    # the GPU idle for tens of milliseconds, and the timed replay would start at a lower engine
    # clock. Later replays of the same graph, beside it, show what first-launch cost is left.
    g_warm = graph_of(full, [sets[i % per_replay] for i in range(args.warmup)], torch) if args.warmup > 0 else None
    g_full = graph_of(full, [sets[i % per_replay] for i in range(args.steps)], torch)
    up = upload_graph(g_full, torch)
    if g_warm is not None:
        g_warm.replay()
    ms = time_graph(g_full, 1, torch) / args.steps
    del g_warm
    later = [time_graph(g_full, 1, torch) / args.steps for _ in range(4)]
    log(f"[bench] decode step {ms * 1e3:.2f} us ({args.steps} steps, {args.warmup} warm-up, graph upload "
        f"{'ok' if up == 0 else f'status {up}'}); later replays "
        + " ".join(f"{x * 1e3:.2f}" for x in later) + " us")
    reps = max(1, args.steps // per_replay)

    # per-kernel averages (each kernel alone, same rotation, graph-replayed)
    for d in sets:
        only_indexer(d)
        only_topk(d)
    kern, graphs = {}, [g_full]
    for name, fn in (("indexer_topk", only_fused), ("indexer_score", only_indexer), ("topk_select", only_topk),
                     ("sparse_mla", only_sparse)):
        gr = graph_of(fn, sets, torch)
        graphs.append(gr)        # keeps graph-pool outputs (d["idx"]) alive
        gr.replay()
        kern[name] = time_graph(gr, reps, torch) / per_replay
        log(f"[bench] {name} {kern[name] * 1e3:.2f} us")
    torch.cuda.synchronize()
    return s, ms, kern, sets, cos, sin, ws, graphs, later


def run_mx_decode(args, torch, device):
    """The bs32 / 64K decode step with the index cache in MXFP4 (e2m1 codes + ue8m0 scales per
    32 channels, 68 bytes per key instead of 256): the packed form of the fp4 fake-quantized
    keys the indexer stores; the index query arrives in the same form from its prologue (as the
    bf16 line's query arrives roped and quantized); scored with block-scaled fp4 MFMA, the top-k
    fused into the scoring as in the bf16 line.
    Everything else as the bf16 line (same shapes, 4 rotating input sets)."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis

    s = Shape(args.batch, args.ctx)
    log(f"[bench] MXFP4-index decode B={s.B} ctx={args.ctx} nb={s.nb} K={s.K}")
    sets = []
    for i in range(args.sets):
        d = make_set(s, SEED + 400 + i, device)
        g = torch.Generator(device=device).manual_seed(SEED + 450 + i)
        del d["ik"], d["iq"]
        d["qc"] = torch.randint(0, 256, (s.B, 1, s.Hi, s.Di // 2), generator=g, device=device,
                                dtype=torch.int32).to(torch.uint8)
        d["qs"] = torch.randint(123, 132, (s.B, 1, s.Hi, s.Di // 32), generator=g, device=device,
                                dtype=torch.int32).to(torch.uint8)
        d["kc"] = torch.randint(0, 256, (s.B, s.nb, s.Di // 2), generator=g, device=device,
                                dtype=torch.int32).to(torch.uint8)
        d["ks"] = torch.randint(123, 132, (s.B, s.nb, s.Di // 32), generator=g, device=device,
                                dtype=torch.int32).to(torch.uint8)
        d["scores"] = torch.empty(s.B, 1, s.nb, dtype=torch.float32, device=device)
        d["out"] = torch.empty(s.B, 1, s.H, s.D, dtype=torch.bfloat16, device=device)
        d["ws"] = torch.empty(max(_abi.mla_workspace_bytes(s.B, 1, s.H, s.D, s.rows, torch.bfloat16), 1),
                              dtype=torch.uint8, device=device)
        d["fidx"] = torch.empty(s.B, 1, s.K, dtype=torch.int32, device=device)
        d["fws"] = torch.empty(max(_abi.indexer_topk_workspace_bytes(s.B, 1, s.Hi, s.Di, s.nb, s.K), 1),
                               dtype=torch.uint8, device=device)
        sets.append(d)
    cos, sin = precompute_freqs_cis(s.rd, s.start + 1, 65536, 160000.0, 16.0, 32, 1, device=device)
    ws = weight_scale(s.Hi, s.Di, torch.bfloat16)

    def f_idx(d):
        _abi.indexer_score_mxfp4((d["qc"], d["qs"]), d["w"], ws, d["kc"], d["ks"], s.nb, s.start, s.r, out=d["scores"])

    def f_topk(d):
        d["idx"] = _abi.topk_select(d["scores"], s.K, s.start, s.r, s.wp + 1)

    def f_fused(d):
        # the step's scoring + selection: the fused form over the MXFP4 query and keys
        sel = _abi.indexer_topk_mxfp4((d["qc"], d["qs"]), d["w"], ws, d["kc"], d["ks"], s.nb, s.start, s.r, s.K,
                                      s.wp + 1, out=d["fidx"], workspace=d["fws"])
        assert sel is not None, "the bs32 decode shape is served by the fused form"

    def f_sparse(d, key="idx"):
        _abi.sparse_mla(d["q"], d["win"], d["chunk"], d["comp"], s.nb, d["sink"], d[key], s.D ** -0.5, s.W,
                        s.start, cos, sin, s.rd, out=d["out"], workspace=d["ws"])

    def full(d):
        f_fused(d)
        f_sparse(d, "fidx")

    per = len(sets)
    reps = max(1, args.steps // per)
    g_full = graph_of(full, sets, torch)
    for _ in range(max(1, args.warmup // per)):
        g_full.replay()
    step_ms = time_graph(g_full, reps, torch) / per
    kern, graphs = {}, [g_full]
    for name, fn in (("indexer_topk", f_fused), ("indexer_score", f_idx), ("topk_select", f_topk),
                     ("sparse_mla", f_sparse)):
        gr = graph_of(fn, sets, torch)
        graphs.append(gr)
        gr.replay()
        kern[name] = time_graph(gr, reps, torch) / per
        log(f"[bench] mxfp4 {name} {kern[name] * 1e3:.2f} us")
    torch.cuda.synchronize()
    b_idx = s.B * (s.nb * (s.Di // 2 + s.Di // 32) + s.Hi * (s.Di // 2 + s.Di // 32) + s.Hi * 2 + s.nb * 4)
    b_fused = b_idx - s.B * s.nb * 4 + s.B * s.K * 4     # codes, scales, q, w in; indices out
    step_bytes = b_fused + s.bytes_sparse()
    log(f"[bench] MXFP4-index decode step {step_ms * 1e3:.2f} us")
    return {
        "workload": "bs32 / 64K decode step with an MXFP4 index cache (e2m1 codes + ue8m0 block scales, 68 B per "
                    "128-channel key) scored by block-scaled fp4 MFMA; KV caches bf16 as in the main line",
        "step_us": step_ms * 1e3, "tokens_per_s": s.B / (step_ms * 1e-3),
        "kernels_us": {k: v * 1e3 for k, v in kern.items()},
        "step_algorithmic_bytes": step_bytes,
        "hbm_GBps_step": step_bytes / (step_ms * 1e-3) / 1e9,
        "indexer_topk_GBps": b_fused / (kern["indexer_topk"] * 1e-3) / 1e9,
        "indexer_bytes_per_launch": b_idx,
        "indexer_GBps": b_idx / (kern["indexer_score"] * 1e-3) / 1e9,
        "indexer_hbm_frac": b_idx / (kern["indexer_score"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }


def run_prefill(torch, device):
    """C3: B=1, 8,192-token chunk after 32,768 prior tokens, top-2,048, 64 heads x 512."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis

    B, n, prior, H, D, rd, Hi, Di, W, K, r = 1, 8192, 32768, 64, 512, 64, 64, 128, 128, 2048, 4
    end = prior + n
    nb = end // r
    log(f"[bench] prefill n={n} prior={prior} nb={nb} K={K}")
    g = torch.Generator(device=device).manual_seed(SEED + 100)
    bf = torch.bfloat16
    q = torch.randn(B, n, H, D, generator=g, device=device).to(bf)
    chunk = torch.randn(B, n, D, generator=g, device=device).to(bf)
    win = torch.randn(B, W, D, generator=g, device=device).to(bf)
    comp = torch.randn(B, nb, D, generator=g, device=device).to(bf)
    iq = torch.randn(B, n, Hi, Di, generator=g, device=device).to(bf)
    ik = torch.randn(B, nb, Di, generator=g, device=device).to(bf)
    w = torch.randn(B, n, Hi, generator=g, device=device).to(bf)
    sink = torch.randn(H, generator=g, device=device)
    cos, sin = precompute_freqs_cis(rd, end, 65536, 160000.0, 16.0, 32, 1, device=device)
    ws = weight_scale(Hi, Di, bf)
    scores = torch.empty(B, n, nb, dtype=torch.float32, device=device)
    out = torch.empty_like(q)
    lens = (prior + torch.arange(n) + 1) // r
    vis = int(lens.sum())
    idx_holder = {}

    def f_idx():
        _abi.indexer_score(iq, w, ws, ik, prior, r, None, out=scores)

    def f_topk():
        idx_holder["idx"] = _abi.topk_select(scores, K, prior, r, W + n)

    def f_sparse():
        _abi.sparse_mla(q, win, chunk, comp, nb, sink, idx_holder["idx"], D ** -0.5, W, prior, cos, sin, rd,
                        out=out)

    def timed(fn, reps=3):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    # the engine clock ramps up under the first heavy launches: warm every form (in the pipeline's
    # order, each reading the previous one's output), then time each twice, alternating, and keep
    # the faster pass of each
    fns = (("indexer_score", f_idx), ("topk_select", f_topk), ("sparse_mla", f_sparse))
    for _, fn in fns:
        fn()
    res = {name: timed(fn) for name, fn in fns}
    for name, fn in fns:
        res[name] = min(res[name], timed(fn))
    for name, _ in fns:
        log(f"[bench] prefill {name} {res[name]:.3f} ms")
    rows_sparse = min(W, W + n) + K   # window rows listed per query (<= W valid) + top-k
    fl_idx = 2.0 * Hi * Di * vis
    fl_sparse = 4.0 * n * H * (W + K) * D
    return {
        "workload": "C3 chunked prefill: B=1, 8192-token chunk after 32768 tokens, nb=10240, top-2048",
        "indexer_ms": res["indexer_score"], "topk_ms": res["topk_select"], "sparse_ms": res["sparse_mla"],
        "indexer_TFLOPs": fl_idx / res["indexer_score"] / 1e9,
        "sparse_TFLOPs": fl_sparse / res["sparse_mla"] / 1e9,
        "indexer_mfma_frac": fl_idx / res["indexer_score"] / 1e9 / BF16_PEAK_TFLOPS,
        "sparse_mfma_frac": fl_sparse / res["sparse_mla"] / 1e9 / BF16_PEAK_TFLOPS,
        "flops_note": f"indexer 2*Hi*Di*sum(lens)={fl_idx:.3e} (causal), sparse 4*n*H*(W+K)*D={fl_sparse:.3e}",
        "rows_per_query": rows_sparse,
    }


def run_wo_a(torch, device):
    """The grouped block-diagonal output LoRA (attention.py:176-179) at the release's shape:
    8 groups, d = 64 * 512 / 8 = 4096 channels per group, rank 1024 (wo_a 64 MiB of bf16). Rows =
    the decode batch (32, 64) or a prefill chunk (8192). dsv41_wo_a_grouped reads the attention
    output and the weight in place; beside it, in the same run, torch.bmm (hipBLASLt) on operands
    copied once into its layout ([G, rows, d] x [G, d, r], contiguous) -- the copy not timed. Then
    wo_b (8192 -> 5120) as torch's linear and, where the attention takes it (33-64 rows), on
    dsv41_linear_rows. Every form rotates over 4 weight sets (592 MB of wo_a and wo_b weights,
    beyond the 256 MB Infinity Cache), so the decode rows' weights stream from HBM."""
    from dsv41 import _abi
    G, R, d = 8, 1024, 4096
    NSET = 4
    g = torch.Generator(device=device).manual_seed(SEED + 300)
    bf = torch.bfloat16
    dim = 5120
    w = [(torch.randn(G * R, d, generator=g, device=device) * 0.02).to(bf) for _ in range(NSET)]
    wT = [x.view(G, R, d).transpose(1, 2).contiguous() for x in w]
    wb = [(torch.randn(dim, G * R, generator=g, device=device) * 0.02).to(bf) for _ in range(NSET)]

    def rot():
        i = [0]

        def nxt():
            i[0] = (i[0] + 1) % NSET
            return i[0]
        return nxt

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3     # us

    out = {"workload": "grouped wo_a: 8 groups x (4096 -> 1024), bf16 in, fp32 sums, bf16 out; then wo_b "
                       "(8192 -> 5120) as torch linear (hipBLASLt) and, at 33-64 rows, on dsv41_linear_rows as the "
                       "attention runs it; 4 rotating weight sets (592 MB)", "lines": {}}
    for rows in (32, 64, 8192):
        o = torch.randn(rows, G * d, generator=g, device=device).to(bf)
        y = torch.empty(rows, G * R, dtype=bf, device=device)
        reps = 48 if rows <= 64 else 8
        ob = o.view(rows, G, d).transpose(0, 1).contiguous()
        splits = _abi.linear_rows_splits(G * R, dim, rows)
        decode_b = _abi.linear_rows_wide(rows, G * R, dim, splits)
        ra, rl, rb, rd, rab = rot(), rot(), rot(), rot(), rot()
        ours = lambda: _abi.wo_a_grouped(o, w[ra()], G, out=y)   # noqa: E731
        lib = lambda: torch.bmm(ob, wT[rl()])                     # noqa: E731
        lin_b = lambda: torch.nn.functional.linear(y, wb[rb()])   # noqa: E731
        dec_b = lambda: _abi.linear_rows(y, wb[rd()], splits)     # noqa: E731

        def both():
            i = rab()
            ya = _abi.wo_a_grouped(o, w[i], G, out=y)
            return _abi.linear_rows(ya, wb[i], splits) if decode_b else torch.nn.functional.linear(ya, wb[i])
        # the engine clock ramps up under the first heavy launches: warm every form, then time
        # each twice, alternating, and keep the faster pass of each
        fns = (ours, lib, lin_b, dec_b, both) if decode_b else (ours, lib, lin_b, both)
        for fn in fns:
            timed(fn, reps)
        t = [timed(fn, reps) for fn in fns]
        t = [min(x, timed(fn, reps)) for x, fn in zip(t, fns)]
        if decode_b:
            us, us_bmm, us_b, us_db, us_ab = t
        else:
            us, us_bmm, us_b, us_ab = t
            us_db = None
        b_bytes = (dim * G * R + rows * G * R + rows * dim) * 2
        b_flops = 2.0 * rows * dim * G * R
        nbytes = (G * R * d + rows * G * d + rows * G * R) * 2
        flops = 2.0 * rows * G * R * d
        line = {"us": us, "GBps": nbytes / us / 1e3, "hbm_frac": nbytes / us / 1e3 / HBM_PEAK_GBS,
                "TFLOPs": flops / us / 1e6, "mfma_frac": flops / us / 1e6 / BF16_PEAK_TFLOPS,
                "algorithmic_bytes": nbytes, "flops": flops, "hipblaslt_bmm_pre_transposed_us": us_bmm,
                # wo_b alone (torch linear, and dsv41_linear_rows where the attention takes it) and
                # after wo_a as the attention runs the pair; a fused pair would save at most the
                # intermediate's write and read
                "wo_b_torch_us": us_b, "wo_b_decode_us": us_db,
                "wo_b_us": us_db if decode_b else us_b,
                "wo_b_algorithmic_bytes": b_bytes, "wo_a_then_wo_b_us": us_ab,
                "intermediate_bytes_frac": 2 * rows * G * R * 2 / (nbytes + b_bytes)}
        ub = line["wo_b_us"]
        line.update({"wo_b_GBps": b_bytes / ub / 1e3, "wo_b_hbm_frac": b_bytes / ub / 1e3 / HBM_PEAK_GBS,
                     "wo_b_TFLOPs": b_flops / ub / 1e6, "wo_b_mfma_frac": b_flops / ub / 1e6 / BF16_PEAK_TFLOPS})
        out["lines"][str(rows)] = line
        dec = f", on dsv41_linear_rows {us_db:.1f} us" if decode_b else ""
        log(f"[bench] wo_a rows={rows}: {us:.1f} us ({line['GBps']:.0f} GB/s, {line['TFLOPs']:.0f} TFLOP/s), "
            f"hipBLASLt bmm on transposed copies {us_bmm:.1f} us; wo_b torch {us_b:.1f} us{dec}; "
            f"wo_a then wo_b {us_ab:.1f} us")
        del o, y, ob
    return out


def run_fp8_decode(args, torch, device):
    """fp8-cache decode (batch 16, 131,072-token context -> 32,768 compressed entries, top-1,024):
    compressed KV and index keys stored as e4m3 with ue8m0 scales per 32 x 32 block (2^-4..2^4),
    dequantized in-kernel; the 128-row window ring and this token's KV stay bf16. Same step as
    the bf16 decode line (indexer -> top-k -> sparse MLA), 4 rotating input sets."""
    from dsv41 import _abi
    from dsv41.indexer import weight_scale
    from dsv41.layers import precompute_freqs_cis

    B, ctx, H, D, rd, Hi, Di, W, K, r = 16, 131072, 64, 512, 64, 64, 128, 128, 1024, 4
    start, nb = ctx, (ctx + 1) // 4
    wp, rb = min(ctx, W), 32
    rows = min(W, wp + 1) + K
    log(f"[bench] fp8-cache decode B={B} ctx={ctx} nb={nb} K={K}")
    bf = torch.bfloat16

    def codes(g, *shape):
        c = torch.randint(0, 256, shape, generator=g, device=device, dtype=torch.int32)
        c = torch.where((c & 0x7F) == 0x7F, c ^ 1, c)          # no NaN codes
        return c.to(torch.uint8)

    def scales(g, *shape):
        return torch.randint(123, 132, shape, generator=g, device=device, dtype=torch.int32).to(torch.uint8)

    sets = []
    for i in range(args.sets):
        g = torch.Generator(device=device).manual_seed(SEED + 200 + i)
        sc = 576 ** -0.5
        sets.append(dict(
            q=(torch.randn(B, 1, H, D, generator=g, device=device) * sc).to(bf),
            win=(torch.randn(B, W, D, generator=g, device=device) * sc).to(bf),
            chunk=(torch.randn(B, 1, D, generator=g, device=device) * sc).to(bf),
            comp8=codes(g, B, nb, D), comp_sc=scales(g, B, nb // rb, D // 32),
            iq=_abi.fq_fp4_ue8m0(torch.randn(B, 1, Hi, Di, generator=g, device=device).to(bf)),
            iq_mx=(codes(g, B, 1, Hi, Di // 2), scales(g, B, 1, Hi, Di // 32)),
            ik8=codes(g, B, nb, Di), ik_sc=scales(g, B, nb // rb, Di // 32),
            w=torch.randn(B, 1, Hi, generator=g, device=device).to(bf),
            sink=torch.randn(H, generator=g, device=device),
            scores=torch.empty(B, 1, nb, dtype=torch.float32, device=device),
            out=torch.empty(B, 1, H, D, dtype=bf, device=device),
            ws=torch.empty(max(_abi.mla_workspace_bytes(B, 1, H, D, rows, bf), 1), dtype=torch.uint8,
                           device=device),
            fidx=torch.empty(B, 1, K, dtype=torch.int32, device=device),
            fws=torch.empty(max(_abi.indexer_topk_workspace_bytes(B, 1, Hi, Di, nb, K), 1), dtype=torch.uint8,
                            device=device)))
    # the fused indexer + top-k form serves ranges of at least 4k rows; top-1,024 over 32,768
    # entries at B=16 takes the two calls, as the decode steps do
    fused_ok = _abi.indexer_topk_workspace_bytes(B, 1, Hi, Di, nb, K) > 0
    cos, sin = precompute_freqs_cis(rd, start + 1, 65536, 160000.0, 16.0, 32, 1, device=device)
    wsc = weight_scale(Hi, Di, bf)

    def f_fused(d):
        # the step's scoring + selection: the fused form over the fp8 keys (exact scores)
        sel = _abi.indexer_topk_fp8(d["iq"], d["w"], wsc, d["ik8"], d["ik_sc"], rb, nb, start, r, K, wp + 1,
                                    out=d["fidx"], workspace=d["fws"])
        assert sel is not None

    def f_idx(d):
        # the step's scores: keys dequantized in-kernel for the bf16 MFMA, exact products, fp32 sums
        _abi.indexer_score_fp8(d["iq"], d["w"], wsc, d["ik8"], d["ik_sc"], rb, nb, start, r, out=d["scores"])

    def f_idx_mxq(d):
        # opt-in: the index query in MXFP4 form against the fp8 keys on the block-scaled fp4 x fp8
        # MFMA (its sums carry a few 1e-5 of max |S|, so its selection may swap near-ties)
        _abi.indexer_score_mxq_fp8(d["iq_mx"], d["w"], wsc, d["ik8"], d["ik_sc"], rb, nb, start, r, out=d["scores"])

    def f_topk(d):
        d["idx"] = _abi.topk_select(d["scores"], K, start, r, wp + 1)

    def f_sparse(d, key="idx"):
        _abi.sparse_mla_fp8(d["q"], d["win"], d["chunk"], d["comp8"], d["comp_sc"], rb, nb, d["sink"], d[key],
                            D ** -0.5, W, start, cos, sin, rd, out=d["out"], workspace=d["ws"])

    def full(d):
        if fused_ok:
            f_fused(d)
            f_sparse(d, "fidx")
        else:
            f_idx(d)
            f_topk(d)
            f_sparse(d)

    per = len(sets)
    reps = max(1, args.steps // per)
    g_full = graph_of(full, sets, torch)
    for _ in range(max(1, args.warmup // per)):
        g_full.replay()
    step_ms = time_graph(g_full, reps, torch) / per
    kern, graphs = {}, [g_full]
    parts = (("indexer_topk", f_fused),) if fused_ok else ()
    for name, fn in parts + (("indexer_score", f_idx), ("indexer_score_mxq_opt_in", f_idx_mxq),
                             ("topk_select", f_topk), ("sparse_mla", f_sparse)):
        gr = graph_of(fn, sets, torch)
        graphs.append(gr)
        gr.replay()
        kern[name] = time_graph(gr, reps, torch) / per
        log(f"[bench] fp8 {name} {kern[name] * 1e3:.2f} us")
    torch.cuda.synchronize()
    b_idx = B * (nb * Di + (nb // rb) * (Di // 32) + Hi * Di * 2 + Hi * 2 + nb * 4)
    b_fused = b_idx - B * nb * 4 + B * K * 4           # keys, scales, q, w in; indices out
    b_topk = B * (nb * 4 + K * 4)
    b_sparse = B * (K * (D + D // 32) + (rows - K) * D * 2 + 2 * H * D * 2 + K * 4)
    step_bytes = (b_fused if fused_ok else b_idx + b_topk) + b_sparse
    log(f"[bench] fp8-cache decode step {step_ms * 1e3:.2f} us")
    return {
        "workload": "fp8-cache decode step: B=16, 131072-token context (nb=32768), top-1024; compressed KV and "
                    "index keys e4m3 with ue8m0 32x32-block scales, dequantized in-kernel (exact index scores: bf16 "
                    "query on the fp4 grid, bf16 MFMA, fp32 sums); window ring bf16. indexer_score_mxq_opt_in: the "
                    "MXFP4 query on the block-scaled fp4 x fp8 MFMA, timed alone",
        "step_us": step_ms * 1e3, "tokens_per_s": B / (step_ms * 1e-3),
        "kernels_us": {k: v * 1e3 for k, v in kern.items()},
        "step_algorithmic_bytes": step_bytes,
        "hbm_GBps_step": step_bytes / (step_ms * 1e-3) / 1e9,
        "fused_indexer_topk": fused_ok,
        "indexer_GBps": b_idx / (kern["indexer_score"] * 1e-3) / 1e9,
        "sparse_GBps": b_sparse / (kern["sparse_mla"] * 1e-3) / 1e9,
    }


def c4_model_args(**over):
    """The 40-layer attention-only stack: layers 0-1 window only, ratio 4 elsewhere; owners
    2/8/14/20; index sources 2/8/14/20/24/28/32/36 (24-36 score against layer 20's keys under
    its candidate mask: blocks of 8, top 2,048 blocks); 64 heads x 512, indexer 64 x 128, top-512."""
    from dsv41.config import ModelArgs
    cfg = dict(n_layers=40, compress_ratios=(0, 0) + (4,) * 38, kv_source_layers=(2, 8, 14, 20),
               index_source_layers=(2, 8, 14, 20, 24, 28, 32, 36), candidate_source_layer=20,
               candidate_topk_blocks=2048, candidate_block_size=8, index_n_heads=64, index_head_dim=128,
               index_topk=512, window_size=128, n_heads=64, head_dim=512, rope_head_dim=64,
               compress_rope_theta=160000.0, original_seq_len=65536, rope_factor=16.0, max_seq_len=65536)
    cfg.update(over)
    return ModelArgs(**cfg)


def c4_step_bytes(a, B, start_pos, index_format="dense", mx_query=None):
    """Algorithmic HBM bytes of one 40-layer decode step: per layer the sparse MLA gather
    (window + top-k rows), q and o; per index source the key stream, its queries and the score
    write; top-k score reads and index writes; the candidate mask write and reads; the window /
    latent / key writes of this token. index_format: "dense" (bf16 caches), "mxfp4" (packed
    index keys), "packed" (MXFP4 index keys, fp4 compressed rows -- e2m1 + e4m3 per 16
    channels -- and an MXFP8 window ring) or "fp8" (the fp8 cache variant: e4m3 + ue8m0 per
    32 x 32 block for the compressed rows and the index keys)."""
    H, D, Hi, Di, W, K = a.n_heads, a.head_dim, a.index_n_heads, a.index_head_dim, a.window_size, a.index_topk
    # per index key, per index-query head, per compressed KV row; the fp8 variant's scale bytes cover
    # 32 x 32 blocks, i.e. 1/32 byte per 32 channels of a row
    kb = {"mxfp4": Di // 2 + Di // 32, "packed": Di // 2 + Di // 32, "fp8": Di + Di / 1024}.get(index_format, Di * 2)
    if mx_query is None:
        mx_query = index_format in ("mxfp4", "packed")
    qb = Di // 2 + Di // 32 if mx_query else Di * 2
    cb = {"fp8": D + D / 1024, "packed": D // 2 + D // 16}.get(index_format, D * 2)
    wb = D + D // 32 if index_format == "packed" else D * 2  # per window-ring row
    wp = min(start_pos, W)
    total = 0
    for l in range(a.n_layers):
        r = a.compress_ratio(l)
        rows = min(W, wp + 1)                                # ring rows + this token's row
        total += B * wb                                      # window write
        if r:
            nb = (start_pos + 1) // r
            k = min(K, nb)
            rows += k
            total += B * k * 4                               # index list read
            if l in a.index_source_layers:
                total += B * (nb * kb + Hi * qb + Hi * 2 + nb * 4)          # indexer
                total += B * (nb * 4 + k * 4)                               # top-k
                if l == a.candidate_source_layer:
                    total += B * (nb * 4 + nb)                              # block max + mask write
                elif 0 <= a.candidate_source_layer < l:
                    total += B * nb                                         # mask read
            if l in a.kv_source_layers:
                total += B * (D * 2 + cb) + (B * (Di * 2 + kb) if l in a.index_source_layers else 0)
            total += B * ((rows - k - 1) * wb + D * 2) + B * k * cb   # gather: ring, token, selected rows
        else:
            total += B * ((rows - 1) * wb + D * 2)
        total += B * 2 * H * D * 2                           # q, o
    return int(total)


def c4_fill(cache, g, device, torch):
    """Random rows in every buffer of a stack cache, whatever its format: dense rows N(0, 1/576),
    index keys on the fp4 grid, packed codes without the NaN patterns and scales in the ranges
    the kernels meet in use."""
    from dsv41 import _abi
    sc = 576 ** -0.5

    def rbytes(lo, hi, *shape):
        return torch.randint(lo, hi, shape, generator=g, device=device, dtype=torch.int32).to(torch.uint8)

    for lc in cache.layers:
        for t in (lc.win_kv, lc.comp_kv):
            if t is not None:
                t.copy_(torch.randn(t.shape, generator=g, device=device) * sc)
        if lc.index_k is not None:
            lc.index_k.copy_(torch.randn(lc.index_k.shape, generator=g, device=device))
            _abi.fq_fp4_ue8m0(lc.index_k, out=lc.index_k)
        if lc.index_k4 is not None:
            lc.index_k4.copy_(rbytes(0, 256, *lc.index_k4.shape))
            lc.index_ks.copy_(rbytes(123, 132, *lc.index_ks.shape))
        if lc.win_kv8 is not None:                 # e4m3 codes without the NaN patterns, ue8m0 2^-9 .. 2^-6
            B, W, R = lc.win_kv8.shape             # rows of D codes then D / 32 scale bytes
            D = R * 32 // 33
            c = rbytes(0, 256, B, W, D)
            lc.win_kv8[..., :D].copy_(torch.where((c & 0x7F) == 0x7F, c ^ 1, c))
            lc.win_kv8[..., D:].copy_(rbytes(118, 122, B, W, D // 32))
        if lc.comp_kv4 is not None:                # e2m1 codes, e4m3 scales 2^-6 .. 2^-2
            B, n, R = lc.comp_kv4.shape            # rows of D / 2 code bytes then D / 16 scale bytes
            D = R * 16 // 9
            lc.comp_kv4[..., :D // 2].copy_(rbytes(0, 256, B, n, D // 2))
            lc.comp_kv4[..., D // 2:].copy_(rbytes(0x08, 0x28, B, n, D // 16))
        for codes, scales in ((lc.comp_kv8, lc.comp_ks), (lc.index_k8, lc.index_k8s)):
            if codes is not None:                  # e4m3 codes without the two NaN patterns
                c = rbytes(0, 256, *codes.shape)
                codes.copy_(torch.where((c & 0x7F) == 0x7F, c ^ 1, c))
                scales.copy_(rbytes(123, 132, *scales.shape))


def run_c4(args, torch, device, index_format="dense", B=64, start=65535, topk=512, mxq=False):
    """C4: one decode token through the 40-layer stack at batch 64 and 65,536 tokens of context
    (16,384 compressed entries per sequence), kernels only: window writes, owner latent / key
    writes (the token completes a group), indexer + top-k at the 8 index sources (candidate
    blocks at layer 20, applied at 24-36), sparse MLA at every layer. Caches (about 5.7 GB)
    exceed the Infinity Cache, so one input set suffices. index_format "mxfp4": the index
    caches and index queries in packed fp4 form (codes + ue8m0 scales, random valid bytes);
    "packed": those and the compressed KV as packed fp4 rows (e2m1 + e4m3 per 16 channels);
    "fp8": the fp8 cache variant in 32 x 32 blocks, scored exactly (bf16 index queries on the fp4
    grid against keys dequantized in-kernel), or with mxq on the block-scaled fp4 x fp8 MFMA
    (MXFP4 queries; opt-in, its sums are not the exact scores)."""
    from dsv41 import _abi
    from dsv41.cache import ModelCache
    from dsv41.indexer import weight_scale
    from dsv41.step import StackDecodeStep

    a = c4_model_args(index_topk=topk, max_seq_len=start + 1)
    bf = torch.bfloat16
    log(f"[bench] 40-layer decode B={B} start_pos={start} top-{topk} index={index_format}")
    g = torch.Generator(device=device).manual_seed(SEED + 300)
    sc = 576 ** -0.5
    H, D, Hi, Di, W = a.n_heads, a.head_dim, a.index_n_heads, a.index_head_dim, a.window_size
    packed = index_format == "packed"
    mx = index_format == "mxfp4" or packed
    fp8 = index_format == "fp8"
    if fp8:
        cache = ModelCache(a, B, start + 1, bf, device, cache_format="fp8", fp8_block_rows=32)
    elif packed:
        cache = ModelCache(a, B, start + 1, bf, device, "mxfp4", cache_format="packed")
    else:
        cache = ModelCache(a, B, start + 1, bf, device, index_format)

    def rbytes(lo, hi, *shape):
        return torch.randint(lo, hi, shape, generator=g, device=device, dtype=torch.int32).to(torch.uint8)

    c4_fill(cache, g, device, torch)
    rn = lambda *shape: torch.randn(*shape, generator=g, device=device)   # noqa: E731
    ins = []
    for l in range(a.n_layers):
        x = dict(q=(rn(B, 1, H, D) * sc).to(bf), kv=(rn(B, 1, D) * sc).to(bf), sink=rn(H))
        if a.compress_ratio(l) and l in a.index_source_layers:
            x.update(w_raw=rn(B, 1, Hi).to(bf), w_scale=weight_scale(Hi, Di, bf))
            if mx or (fp8 and mxq):          # the query in MXFP4 form (fp8 keys: the fp4 x fp8 MFMA)
                x["index_q_mx"] = (rbytes(0, 256, B, 1, Hi, Di // 2), rbytes(123, 132, B, 1, Hi, Di // 32))
            else:
                x["index_q"] = _abi.fq_fp4_ue8m0(rn(B, 1, Hi, Di).to(bf))
        if l in a.kv_source_layers:
            x["latent"] = rn(B, 1, D).to(bf)
            if l in a.index_source_layers:
                x.update(k_raw=rn(B, 1, Di).to(bf), k_norm=torch.ones(Di, device=device))
        ins.append(x)
    step = StackDecodeStep(a, B, start, bf, device)
    reps = max(4, args.steps // 8)
    if getattr(args, "eager", False):       # plain launches (counter passes cannot see into a graph)
        for _ in range(max(1, args.warmup // 4)):
            step(cache, ins)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            step(cache, ins)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
    else:
        gr = graph_of(lambda _: step(cache, ins), [None], torch)
        for _ in range(max(1, args.warmup // 4)):
            gr.replay()
        ms = time_graph(gr, reps, torch)
    nbytes = c4_step_bytes(a, B, start, index_format, mx_query=mx or (fp8 and mxq))
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] C4 step {ms:.3f} ms, {B / (ms * 1e-3):.0f} tokens/s, {gbs:.0f} GB/s")
    name = "C5" if fp8 else "C4"
    return {
        "workload": f"{name}: 40-layer attention-only decode step (kernels only), B={B}, {start + 1}-token context "
                    f"(nb={(start + 1) // 4}), ratio 4, top-{topk}; owners 2/8/14/20, index sources 2..36, candidate "
                    f"source 20; " + ("fp8 caches (e4m3 + ue8m0 per 32x32 block) for compressed KV and index keys, "
                                      + ("index queries MXFP4 (fp4 x fp8 MFMA scoring, opt-in)" if mxq else
                                         "exact index scores (keys dequantized in-kernel)") + ", window ring bf16"
                                      if fp8
                                      else "packed caches: compressed KV e2m1 + e4m3 per 16 channels (288 B/row), "
                                      "window ring MXFP8 (528 B/row), index keys and queries MXFP4" if packed
                                      else f"index caches {index_format}"),
        "step_ms": ms, "tokens_per_s": B / (ms * 1e-3), "steps": reps,
        "step_algorithmic_bytes": nbytes, "hbm_GBps_step": gbs, "hbm_frac_step": gbs / HBM_PEAK_GBS,
    }


def run_token(args, torch, device, B=64, start=65535):
    """One decode token as callers run it: AttentionStack.forward, i.e. model.py:141-154's layer
    loop with attention.py:106-179 in every layer (q and kv projections with their norms, the
    window-KV prologue, compressor and indexer at their layers, top-k, sparse MLA, grouped wo_a,
    wo_b, the residual add), MoE and hyper-connections as identity. 40 layers with C4's sharing
    layout at the release's widths (dim 5120, q LoRA 1280, 64 x 512 heads, indexer 64 x 128,
    8 x 1024 output LoRA), bf16 weights (torch's default init) and bf16 caches of random rows,
    B=64 at 65,536 tokens of context. The token is timed eagerly (Python issuing every launch, as
    the reference's generate loop runs it) and replayed from one HIP graph captured at position
    65,535; every call rewrites that position's ring slot, latent and key."""
    from dsv41.model import AttentionStack

    a = c4_model_args(max_seq_len=start + 1)
    bf = torch.bfloat16
    log(f"[bench] decode token through AttentionStack: B={B} start_pos={start}, release widths")
    torch.manual_seed(SEED + 400)
    stack = AttentionStack(a, bf, device)
    g = torch.Generator(device=device).manual_seed(SEED + 401)
    for attn in stack.layers:
        attn.attn_sink.copy_(torch.randn(a.n_heads, generator=g, device=device))
    cache = stack.make_cache(B, start + 1)
    c4_fill(cache, g, device, torch)
    h = torch.randn(B, 1, a.dim, generator=g, device=device).to(bf)

    def token(_):
        cache.offset = start
        return stack(h, cache)

    reps = max(4, args.steps // 20)
    for _ in range(2):
        token(None)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        token(None)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / reps
    gr = graph_of(token, [None], torch)
    for _ in range(2):
        gr.replay()
    ms = time_graph(gr, reps, torch)
    weight_bytes = sum(p.numel() * p.element_size() for p in stack.parameters())
    cache_bytes = c4_step_bytes(a, B, start)
    nbytes = weight_bytes + cache_bytes
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] decode token {ms:.3f} ms graph-replayed, {eager_ms:.3f} ms eager, {gbs:.0f} GB/s")
    del gr, stack, cache
    return {
        "workload": f"one decode token through AttentionStack (40 layers, C4 sharing layout, release widths: "
                    f"dim {a.dim}, q LoRA {a.q_lora_rank}, {a.n_heads} x {a.head_dim} heads, indexer "
                    f"{a.index_n_heads} x {a.index_head_dim}, wo_a {a.o_groups} x {a.o_lora_rank}), B={B}, "
                    f"{start + 1}-token context, bf16 weights and caches; wq_a + wkv, wq_b, wo_b and the "
                    f"indexer's wq_b and weights_proj on dsv41_linear_rows(_pair), the compressor's fp32 "
                    f"projections torch GEMMs",
        "token_ms": ms, "token_ms_eager": eager_ms, "tokens_per_s": B / (ms * 1e-3), "steps": reps,
        "weight_bytes": weight_bytes, "cache_algorithmic_bytes": cache_bytes,
        "token_algorithmic_bytes": nbytes, "hbm_GBps_token": gbs, "hbm_frac_token": gbs / HBM_PEAK_GBS,
    }


def achievable_peaks(torch, device):
    """What this box reaches, measured in the same run: a device-to-device copy (torch's copy
    kernel) over 4 rotating 256 MiB bf16 buffers, read + write bytes per second; and a 8192^3
    bf16 torch.matmul (hipBLASLt), flops per second. The fractions against these sit beside the
    ones against the published peaks."""
    n = 256 << 20
    srcs = [torch.ones(n // 2, dtype=torch.bfloat16, device=device) for _ in range(4)]
    dsts = [torch.empty_like(x) for x in srcs]
    for x, y in zip(srcs, dsts):
        y.copy_(x)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 40
    torch.cuda.synchronize()
    e0.record()
    for i in range(reps):
        dsts[i % 4].copy_(srcs[i % 4])
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * n * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del srcs, dsts
    m = 8192
    a = torch.randn(m, m, dtype=torch.bfloat16, device=device)
    b = torch.randn(m, m, dtype=torch.bfloat16, device=device)
    c = torch.empty(m, m, dtype=torch.bfloat16, device=device)
    for _ in range(3):
        torch.matmul(a, b, out=c)
    reps = 20
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    gemm_tf = 2 * m ** 3 * reps / (e0.elapsed_time(e1) * 1e-3) / 1e12
    del a, b, c
    torch.cuda.empty_cache()
    log(f"[bench] achievable: copy {copy_gbs:.0f} GB/s, bf16 GEMM {gemm_tf:.0f} TFLOP/s")
    return {"hbm_copy_GBps": copy_gbs, "bf16_gemm_TFLOPs": gemm_tf,
            "how": "torch copy over 4 rotating 256 MiB bf16 buffers (read + write bytes); 8192^3 bf16 "
                   "torch.matmul (hipBLASLt), same run"}


def cpu_baseline(s: Shape, sets, cos, sin, ws, seconds, torch):
    """The numpy oracle on whole batch rows of the same decode workload, until `seconds` pass."""
    import numpy as np
    from threadpoolctl import threadpool_info

    from oracle import cpu_ref as R

    d = sets[0]
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    lens = R.query_lens(s.start, 1, s.r)
    wslots = (s.start - s.wp + np.arange(s.wp)) % s.W
    widx = R.window_idx_matrix(s.wp, 1, s.W)[None]
    rc = f(cos[s.start:s.start + 1])
    rsn = f(sin[s.start:s.start + 1])
    sink = f(d["sink"])
    rows, el = 0, 0.0
    while el < seconds:
        b = rows % s.B            # device->host copy of the row is outside the timed part
        iq, ik, w = f(d["iq"][b:b + 1]), f(d["ik"][b:b + 1]), f(d["w"][b:b + 1])
        q, win, chunk, comp = f(d["q"][b:b + 1]), f(d["win"][b:b + 1]), f(d["chunk"][b:b + 1]), f(d["comp"][b:b + 1])
        t0 = time.perf_counter()
        sc = R.indexer_scores(iq, ik, R.cast(w * np.float32(ws), "bf16"), s.start, s.r)
        idx = R.topk_indices(sc, s.K, lens, s.wp + 1)
        kv_all = np.concatenate([win[:, wslots], chunk, comp], axis=1)
        q = R.rope_tail(q, s.rd, rc, rsn, dtype="bf16")
        o = R.sparse_attn(q, kv_all, sink, np.concatenate([widx, idx], -1), s.D ** -0.5, dtype="bf16")
        R.rope_tail(o, s.rd, rc, rsn, inverse=True, dtype="bf16")
        el += time.perf_counter() - t0
        rows += 1
    threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    return {"value": rows / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{rows} batch rows of the bs32/64K decode step (indexer + top-k + q rope + sparse MLA + "
                      f"inverse rope), "
                      f"numpy float32 oracle, BLAS threads {threads}, host cpu_count {os.cpu_count()}, "
                      f"{el:.1f} s of compute (row copies to the host untimed)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the hot path is "
              "batch-sharded with zero exchange, so N GPUs run N independent copies)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda:0")
    from dsv41 import _abi
    _abi.lib()

    s, ms, kern, sets, cos, sin, ws, _graphs, later = run_decode(args, torch, device)
    # the step runs the fused indexer + top-k form and the sparse MLA (with its split combine)
    step_bytes = s.bytes_indexer_topk() + s.bytes_sparse()
    step_gbs = step_bytes / (ms * 1e-3) / 1e9
    fused_gbs = s.bytes_indexer_topk() / (kern["indexer_topk"] * 1e-3) / 1e9
    idx_gbs = s.bytes_indexer() / (kern["indexer_score"] * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": s.B / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_later_replays": later,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "sparse-MLA decode step of one compressing layer: indexer scoring + top-k + "
                               "sparse MLA (+inverse rope), bs32, 64K context",
                   "batch": s.B, "context": args.ctx, "compressed_entries": s.nb, "index_topk": s.K,
                   "heads": s.H, "head_dim": s.D, "rope_dim": s.rd, "index_heads": s.Hi, "index_dim": s.Di,
                   "window": s.W, "input_sets": len(sets)},
        "hbm_GBps_step": step_gbs,
        "hbm_frac_step": step_gbs / HBM_PEAK_GBS,
        "step_algorithmic_bytes": step_bytes,
        "kernels_us": {k: v * 1e3 for k, v in kern.items()},
        "roofline": {"bound": "hbm",
                     "kernel": "indexer_topk (dsv41_indexer_topk -> indexer_decode_kernel<4, 8, false, 4> "
                               "scoring + per-range top-k, then topk_merge_kernel<4>; one call, timed as a unit)",
                     "achieved": fused_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": fused_gbs / HBM_PEAK_GBS,
                     "traffic": measured_traffic(),
                     "traffic_source": TRAFFIC_FILE,
                     "bytes_per_launch": s.bytes_indexer_topk(), "avg_launch_us": kern["indexer_topk"] * 1e3},
        # the scoring kernel alone as the two-call form runs it (scores written to HBM)
        "indexer_score_unfused": {"kernel": "indexer_decode_kernel<4, 8, false, 0>", "achieved_GBps": idx_gbs,
                                  "frac": idx_gbs / HBM_PEAK_GBS, "bytes_per_launch": s.bytes_indexer(),
                                  "avg_launch_us": kern["indexer_score"] * 1e3},
    }
    try:
        peaks = achievable_peaks(torch, device)
        result["achievable"] = peaks
        result["roofline"]["frac_of_achievable"] = fused_gbs / peaks["hbm_copy_GBps"]
    except Exception as e:
        peaks = None
        result["achievable"] = {"error": repr(e)}
    # the single-layer MXFP4 and fp8 lines are graph-timed only: counter passes (--eager) reach
    # their kernels through the 40-layer lines
    if not args.no_mx and not args.eager:
        try:
            result["mxfp4_index_decode"] = run_mx_decode(args, torch, device)
        except Exception as e:
            result["mxfp4_index_decode"] = {"error": repr(e)}
    if not args.no_prefill:
        try:
            result["prefill"] = run_prefill(torch, device)
            if peaks:
                for key in ("indexer", "sparse"):
                    result["prefill"][f"{key}_frac_of_gemm"] = (result["prefill"][f"{key}_TFLOPs"] /
                                                                peaks["bf16_gemm_TFLOPs"])
        except Exception as e:  # report, do not hide: the decode line still prints
            result["prefill"] = {"error": repr(e)}
    if not args.no_wo_a:                  # event-timed, so it also runs in the eager counter passes
        try:
            result["output_lora"] = run_wo_a(torch, device)
        except Exception as e:
            result["output_lora"] = {"error": repr(e)}
        torch.cuda.empty_cache()
    if not args.no_fp8 and not args.eager:
        try:
            result["fp8_cache_decode"] = run_fp8_decode(args, torch, device)
        except Exception as e:
            result["fp8_cache_decode"] = {"error": repr(e)}
    if not args.no_c4:
        try:
            result["c4_stack_decode"] = run_c4(args, torch, device)
        except Exception as e:
            result["c4_stack_decode"] = {"error": repr(e)}
        torch.cuda.empty_cache()
        if not args.no_mx:
            try:
                result["c4_stack_decode_mxfp4_index"] = run_c4(args, torch, device, "mxfp4")
            except Exception as e:
                result["c4_stack_decode_mxfp4_index"] = {"error": repr(e)}
            torch.cuda.empty_cache()
            try:
                result["c4_stack_decode_packed"] = run_c4(args, torch, device, "packed")
            except Exception as e:
                result["c4_stack_decode_packed"] = {"error": repr(e)}
            torch.cuda.empty_cache()
        if not args.no_fp8:
            try:
                result["c5_stack_decode_fp8"] = run_c4(args, torch, device, "fp8", B=16, start=131071, topk=1024)
            except Exception as e:
                result["c5_stack_decode_fp8"] = {"error": repr(e)}
            torch.cuda.empty_cache()
            if not args.no_mx:
                try:
                    result["c5_stack_decode_fp8_mxq_opt_in"] = run_c4(args, torch, device, "fp8", B=16, start=131071,
                                                                      topk=1024, mxq=True)
                except Exception as e:
                    result["c5_stack_decode_fp8_mxq_opt_in"] = {"error": repr(e)}
                torch.cuda.empty_cache()
    if not args.no_token and not args.eager:
        try:
            result["decode_token_stack"] = run_token(args, torch, device)
        except Exception as e:
            result["decode_token_stack"] = {"error": repr(e)}
        torch.cuda.empty_cache()
    if not args.no_cpu:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(s, sets, cos, sin, ws, args.cpu_seconds, torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
