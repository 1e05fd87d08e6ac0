"""CPU checks of the boundary: libdsv41.so loads and exports exactly the C ABI that
include/dsv41.h declares, the ctypes table matches the header, the host-side config mirrors
the reference's topology rules, and wrappers refuse non-GPU tensors instead of falling back."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsv41.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsv41_\w+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    for must in ("dsv41_sparse_attn", "dsv41_sparse_mla", "dsv41_indexer_score", "dsv41_topk_select",
                 "dsv41_candidate_blocks", "dsv41_compress_pool", "dsv41_comp_write",
                 "dsv41_index_key_publish", "dsv41_fq_fp8_ue8m0", "dsv41_fq_fp4_ue8m0",
                 "dsv41_fq_fp4_e4m3", "dsv41_rope_tail", "dsv41_last_error_string"):
        assert must in names


def test_library_loads_and_exports_every_declared_symbol():
    from dsv41 import _abi
    lib = _abi.lib()
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in dsv41.h but not exported"
    assert set(_abi._SIGNATURES) == set(header_functions())
    assert "gfx950" in _abi.version()


def test_ctypes_arity_matches_header():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    from dsv41 import _abi
    for name, args in _abi._SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name


def test_workspace_query_is_host_only():
    from dsv41 import _abi
    # decode-sized work splits its index list across workgroups and needs scratch
    assert _abi.mla_workspace_bytes(32, 1, 64, 512, 640, torch.bfloat16) > 0
    # prefill-sized work does not
    assert _abi.mla_workspace_bytes(1, 8192, 64, 512, 2176, torch.bfloat16) == 0
    assert _abi.mla_workspace_bytes(1, 1, 4, 64, 16, torch.float32) == 0


def test_wrappers_refuse_cpu_tensors():
    from dsv41 import _abi
    from dsv41.sparse_attention import sparse_attn
    q = torch.zeros(1, 1, 4, 64)
    with pytest.raises(ValueError, match="GPU"):
        sparse_attn(q, torch.zeros(1, 8, 64), torch.zeros(4), torch.zeros(1, 1, 4, dtype=torch.int32), 0.1)
    with pytest.raises(ValueError, match="GPU"):
        _abi.fq_fp8_ue8m0(torch.zeros(4, 32))
    with pytest.raises(ValueError, match="GPU"):
        _abi.topk_select(torch.zeros(1, 1, 8), 4, 0, 1, 0)


def test_contract_violations_are_reported_by_the_library():
    """Host-side validation in the C ABI runs before any launch (null pointers, shapes)."""
    from dsv41 import _abi
    lib = _abi.lib()
    rc = lib.dsv41_sparse_attn(None, None, None, None, None, 1, 1, 4, 64, 8, 4, ctypes.c_float(0.1), 1,
                               None, 0, None)
    assert rc == -1 and b"null" in lib.dsv41_last_error_string()
    fake = ctypes.c_void_p(256)    # never dereferenced: rejected before launch
    rc = lib.dsv41_fq_fp8_ue8m0(fake, fake, 4, 48, 32, 1, None)
    assert rc == -3
    rc = lib.dsv41_fq_fp8_ue8m0(fake, fake, 4, 64, 8, 1, None)
    assert rc == -3 and b"block" in lib.dsv41_last_error_string()
    rc = lib.dsv41_rmsnorm(fake, fake, fake, 4, 64, ctypes.c_float(1e-6), 7, None)
    assert rc == -2
    rc = lib.dsv41_topk_select(fake, fake, 1, 1, 1 << 23, 4, 0, 1, 0, None)
    assert rc == -3
    rc = lib.dsv41_compress_pool(fake, fake, fake, fake, fake, fake, 1, 1, 64, 1, 0, ctypes.c_float(0),
                                 1, None)
    assert rc == -1 and b"ratio" in lib.dsv41_last_error_string()
    # two-stage top-k: the workspace is checked before any launch (the shape must take that form,
    # or the call below would launch on the fake pointers)
    need = _abi.topk_workspace_bytes(16, 32768, 512)
    assert need > 0
    rc = lib.dsv41_topk_select_ws(fake, fake, 16, 1, 32768, 512, 131071, 4, 129, None, 0, None)
    assert rc == -4 and b"workspace" in lib.dsv41_last_error_string()
    rc = lib.dsv41_topk_select_ws(fake, fake, 16, 1, 32768, 512, 131071, 4, 129, fake, need - 1, None)
    assert rc == -4
    # fused indexer + top-k: unserved shapes and a missing or short workspace, before any launch
    need = _abi.indexer_topk_workspace_bytes(32, 1, 64, 128, 16384, 512)
    args = (fake, fake, ctypes.c_float(0.01), fake, 16384 * 128, None, fake, 32, 1)
    rc = lib.dsv41_indexer_topk(*args, 64, 128, 16384, 65535, 4, 512, 129, None, 0, None)
    assert rc == -4 and b"workspace" in lib.dsv41_last_error_string()
    rc = lib.dsv41_indexer_topk(*args, 64, 128, 16384, 65535, 4, 512, 129, fake, need - 1, None)
    assert rc == -4
    rc = lib.dsv41_indexer_topk(*args, 48, 128, 16384, 65535, 4, 512, 129, fake, need, None)
    assert rc == -3 and b"fused" in lib.dsv41_last_error_string()
    # the fp8 and MXFP4 fused entries check the same way (fp8: byte strides of codes and scales)
    a8 = (fake, fake, ctypes.c_float(0.01), fake, 16384 * 128, fake, 16384 * 4, 1, None, fake, 32, 1)
    rc = lib.dsv41_indexer_topk_fp8(*a8, 64, 128, 16384, 65535, 4, 512, 129, None, 0, None)
    assert rc == -4 and b"workspace" in lib.dsv41_last_error_string()
    rc = lib.dsv41_indexer_topk_fp8(*a8, 48, 128, 16384, 65535, 4, 512, 129, fake, need, None)
    assert rc == -3
    rc = lib.dsv41_indexer_topk_fp8(*a8[:7], 2, *a8[8:], 64, 128, 16384, 65535, 4, 512, 129, fake, need, None)
    assert rc == -1 and b"row block" in lib.dsv41_last_error_string()
    amx = (fake, fake, fake, ctypes.c_float(0.01), fake, 16384 * 64, fake, 16384 * 4, None, fake, 32, 1)
    rc = lib.dsv41_indexer_topk_mxfp4(*amx, 64, 128, 16384, 65535, 4, 512, 129, fake, need - 1, None)
    assert rc == -4
    rc = lib.dsv41_indexer_topk_mxfp4(*amx, 64, 64, 16384, 65535, 4, 512, 129, fake, need, None)
    assert rc == -3 and b"dim 128" in lib.dsv41_last_error_string()


def test_topk_workspace_sizes():
    """Two stages (a workspace) only for rows over 16384 scores with k <= 2048 whose chunk lists
    fit one register workgroup: keys and positions of each 4096-score chunk's best k."""
    from dsv41 import _abi
    assert _abi.topk_workspace_bytes(32, 16384, 512) == 0            # one workgroup per row
    assert _abi.topk_workspace_bytes(16, 20000, 5000) == 0           # k above half a chunk
    assert _abi.topk_workspace_bytes(1, 4 << 20, 2048) == 0          # lists too long for one stage-2 group
    # k above an eighth of a 4,096-entry chunk: 8,192-entry chunks (4 lists of 1,024 per 32K row)
    assert _abi.topk_workspace_bytes(16, 32768, 1024) == 2 * 16 * 4 * 1024 * 4
    assert _abi.topk_workspace_bytes(1, 40000, 1024) == 2 * ((5 * 1024 * 4 + 255) // 256 * 256)   # row > 32K
    assert _abi.topk_workspace_bytes(16, 32768, 512) == 2 * 16 * 8 * 512 * 4
    assert _abi.topk_workspace_bytes(3, 16390, 512) == 2 * (((3 * 5 * 512 * 4) + 255) // 256 * 256)
    assert _abi.topk_workspace_bytes(0, 32768, 1024) == 0


def test_indexer_topk_workspace_sizes():
    """The fused decode form serves bf16 keys of 128 channels, 16/32/64 heads, fewer than 8
    queries per row (or a candidate mask) and row ranges of at least 4k rows: two lists (keys,
    positions) of k entries per (query, range)."""
    from dsv41 import _abi
    lists = lambda rows, ranges, k: 2 * ((rows * ranges * k * 4 + 255) // 256 * 256)   # noqa: E731
    assert _abi.indexer_topk_workspace_bytes(32, 1, 64, 128, 16384, 512) == lists(32, 8, 512)
    assert _abi.indexer_topk_workspace_bytes(16, 1, 64, 128, 32768, 512) == lists(16, 16, 512)
    assert _abi.indexer_topk_workspace_bytes(16, 1, 64, 128, 32768, 1024) == 0   # k above a quarter of a range
    assert _abi.indexer_topk_workspace_bytes(2, 1, 64, 128, 256, 64) == lists(2, 1, 64)
    assert _abi.indexer_topk_workspace_bytes(8, 8, 64, 128, 16384, 512, True) == lists(64, 4, 512)
    assert _abi.indexer_topk_workspace_bytes(8, 8, 64, 128, 16384, 512) == 0     # prefill-sized, no mask
    assert _abi.indexer_topk_workspace_bytes(8, 1, 64, 128, 16384, 512) == 0     # 512-row ranges < 4k
    assert _abi.indexer_topk_workspace_bytes(32, 1, 48, 128, 16384, 512) == 0    # head count
    assert _abi.indexer_topk_workspace_bytes(32, 1, 64, 64, 16384, 512) == 0     # key width
    assert _abi.indexer_topk_workspace_bytes(0, 1, 64, 128, 16384, 512) == 0


# ------------------------------------------------------------------ host logic


def test_model_args_topology_and_both_config_layouts():
    from dsv41.config import ModelArgs
    flat = {"dim": 256, "n_layers": 8, "compress_ratios": [0, 0, 2, 2, 2, 1, 1, 1],
            "kv_source_layers": [2, 5], "index_source_layers": [2, 5, 7],
            "candidate_source_layer": 5, "candidate_topk_blocks": 3, "candidate_block_size": 2,
            "index_n_heads": 8, "rope_scaling": {"factor": 4.0, "original_max_position_embeddings": 64}}
    hub = {"model_type": "x", "text_config": {"hidden_size": 256, "num_hidden_layers": 8,
                                              "compress_ratios": [0, 0, 2, 2, 2, 1, 1, 1],
                                              "kv_source_layer_ids": [2, 5],
                                              "index_source_layer_ids": [2, 5, 7],
                                              "candidate_source_layer_id": 5,
                                              "candidate_topk_blocks": 3, "candidate_block_size": 2,
                                              "index_n_heads": 8,
                                              "rope_scaling": {"factor": 4.0,
                                                               "original_max_position_embeddings": 64}}}
    for a in (ModelArgs.from_dict(flat), ModelArgs.from_dict(hub)):
        assert a.dim == 256 and a.n_layers == 8 and a.index_n_heads == 8
        assert a.rope_factor == 4.0 and a.original_seq_len == 64
        assert [a.compress_ratio(i) for i in range(10)] == [0, 0, 2, 2, 2, 1, 1, 1, 0, 0]
        assert a.kv_source_for(4) == 2 and a.kv_source_for(7) == 5
        assert a.index_source_for(6) == 5 and a.index_source_for(7) == 7
        with pytest.raises(ValueError):
            a.kv_source_for(1)
    bad = ModelArgs(compress_ratios=(2, 1), kv_source_layers=(0,))
    with pytest.raises(ValueError, match="ratio"):
        bad.kv_source_for(1)
    # fields outside the attention path are read by their reference names, never interpreted;
    # keys outside the reference's table are kept verbatim
    a = ModelArgs.from_dict({**flat, "hc_mult": 3, "moe_inter_dim": 32, "vision_dim": 9})
    assert a.hc_mult == 3 and a.moe_inter_dim == 32 and a.extra == {"vision_dim": 9} and a.vision_dim == 9
    assert ModelArgs(n_routed_experts=8).n_routed_experts == 8
    with pytest.raises(AttributeError):
        ModelArgs().no_such_field
    # defaults are the release's attention shape
    d = ModelArgs()
    assert (d.dim, d.n_heads, d.head_dim, d.rope_head_dim, d.window_size, d.index_topk) == \
        (5120, 64, 512, 64, 128, 512)
    # the topology is re-resolved when the sharing fields change
    d.compress_ratios, d.kv_source_layers = (0, 4, 4), (1,)
    assert d.kv_source_for(2) == 1
    d.kv_source_layers = (2,)
    with pytest.raises(ValueError):
        d.kv_source_for(1)


# every attribute of the reference's ModelArgs (deepseek_v41_mlx/config.py:30-102) with the value
# its from_dict gives for the two release files (config.py:136-193, read by hand): both layouts
# describe the same model, so one table serves both
_RELEASE_ATTRS = {
    "vocab_size": 129280, "dim": 5120, "n_layers": 40, "moe_inter_dim": 2304, "n_heads": 64, "head_dim": 512,
    "rope_head_dim": 64, "q_lora_rank": 1280, "o_lora_rank": 1024, "o_groups": 8, "window_size": 128,
    "norm_eps": 1e-20, "n_routed_experts": 384, "n_shared_experts": 1, "n_activated_experts": 6,
    "score_func": "sqrtsoftplus", "gate_temp": 1.0, "norm_topk_prob": True, "route_scale": 1.5,
    "swiglu_limit": 10.0, "kv_source_layers": (2, 8, 14, 20),
    "index_source_layers": (2, 8, 14, 20, 24, 28, 32, 36), "compress_rope_theta": 160000,
    "candidate_source_layer": 20, "candidate_topk_blocks": 2048, "candidate_block_size": 8,
    "original_seq_len": 65536, "rope_theta": 10000, "rope_factor": 16, "beta_fast": 32, "beta_slow": 1,
    "max_seq_len": 1048576, "index_n_heads": 32, "index_head_dim": 128, "index_topk": 512, "hc_mult": 4,
    "hc_sinkhorn_iters": 20, "hc_eps": 1e-6, "engram_layer_ids": (1, 14),
    "engram_num_embeddings": (384006168, 384016682), "engram_max_ngram_size": 4, "engram_vocab_size": 16000000,
    "engram_n_heads": 8, "engram_head_dim": 256, "engram_pad_id": 2, "engram_compressed_vocab_size": 99092,
    "n_mtp_layers": 3, "dspark_target_layer_ids": (37, 38, 39), "vision_n_layers": 0,
}

# keyword construction: the dataclass defaults of config.py:30-102
_DEFAULT_ATTRS = {
    "vocab_size": 129280, "dim": 5120, "n_layers": 40, "moe_inter_dim": 2304, "n_heads": 64, "head_dim": 512,
    "rope_head_dim": 64, "q_lora_rank": 1280, "o_lora_rank": 1024, "o_groups": 8, "window_size": 128,
    "norm_eps": 1e-20, "n_routed_experts": 384, "n_shared_experts": 1, "n_activated_experts": 6,
    "score_func": "sqrtsoftplus", "gate_temp": 1.0, "norm_topk_prob": True, "route_scale": 1.5,
    "swiglu_limit": 10.0, "compress_ratios": (), "kv_source_layers": (), "index_source_layers": (),
    "compress_rope_theta": 160000.0, "candidate_source_layer": -1, "candidate_topk_blocks": 0,
    "candidate_block_size": 0, "original_seq_len": 65536, "rope_theta": 10000.0, "rope_factor": 16.0,
    "beta_fast": 32, "beta_slow": 1, "max_seq_len": 1048576, "index_n_heads": 32, "index_head_dim": 128,
    "index_topk": 512, "hc_mult": 4, "hc_sinkhorn_iters": 20, "hc_eps": 1e-6, "engram_layer_ids": (),
    "engram_num_embeddings": (), "engram_max_ngram_size": 4, "engram_vocab_size": 0, "engram_n_heads": 0,
    "engram_head_dim": 0, "engram_pad_id": 2, "engram_compressed_vocab_size": 0, "n_mtp_layers": 0,
    "dspark_target_layer_ids": (), "vision_n_layers": 0,
}


def test_model_args_release_files_expose_every_reference_attribute():
    """Both release layouts (the flat inference config.json and the hub file, stored verbatim in
    tests/golden/release_configs.json) give every attribute the reference's ModelArgs defines, with
    the values its from_dict gives, and keyword construction gives the dataclass defaults."""
    import json
    from dsv41.config import ModelArgs
    with open(os.path.join(os.path.dirname(__file__), "golden", "release_configs.json")) as f:
        files = json.load(f)
    assert set(_RELEASE_ATTRS) | {"compress_ratios"} == set(_DEFAULT_ATTRS)
    for layout in ("flat", "hub"):
        a = ModelArgs.from_dict(files[layout])
        for name, want in _RELEASE_ATTRS.items():
            got = getattr(a, name)
            assert got == want and type(got) is type(want), (layout, name, got, want)
        assert len(a.compress_ratios) == 43 and a.compress_ratios[:4] == (0, 0, 2, 2)
        assert [a.kv_source_for(i) for i in (2, 7, 21, 39)] == [2, 2, 20, 20]
        assert a.raw == {"model_type": "deepseek_v41"}
    d = ModelArgs()
    for name, want in _DEFAULT_ATTRS.items():
        assert getattr(d, name) == want, (name, getattr(d, name), want)
    # the two routes differ where the reference's differ (config.py:162, 193)
    assert ModelArgs.from_dict({}).swiglu_limit == 0.0 and ModelArgs().swiglu_limit == 10.0
    assert ModelArgs.from_dict({"vision_n_layers": 32}).vision_n_layers == 0
    # every hub alias is read (values away from the defaults, so a dropped alias cannot pass)
    hub = {"text_config": {"moe_intermediate_size": 7, "num_experts_per_tok": 9, "scoring_func": "softmax",
                           "routed_scaling_factor": 2.5, "engram_pad_token_id": 5, "num_nextn_predict_layers": 1,
                           "hidden_size": 64, "num_hidden_layers": 3, "num_attention_heads": 4,
                           "qk_rope_head_dim": 16, "sliding_window": 32, "rms_norm_eps": 1e-6,
                           "kv_source_layer_ids": [1], "index_source_layer_ids": [1],
                           "candidate_source_layer_id": 2, "max_position_embeddings": 4096}}
    a = ModelArgs.from_dict(hub)
    assert (a.moe_inter_dim, a.n_activated_experts, a.score_func, a.route_scale, a.engram_pad_id,
            a.n_mtp_layers) == (7, 9, "softmax", 2.5, 5, 1)
    assert (a.dim, a.n_layers, a.n_heads, a.rope_head_dim, a.window_size, a.norm_eps, a.kv_source_layers,
            a.index_source_layers, a.candidate_source_layer, a.max_seq_len) == \
        (64, 3, 4, 16, 32, 1e-6, (1,), (1,), 2, 4096)


def test_rope_frequencies_match_oracle_restatement():
    from dsv41.layers import yarn_inv_freqs
    from oracle import cpu_ref as R
    for args in [(64, 65536, 160000.0, 16.0, 32, 1), (16, 0, 10000.0, 4.0, 32, 1), (16, 64, 40000.0, 4.0, 32, 1)]:
        assert np.array_equal(yarn_inv_freqs(*args), R.yarn_freqs(*args))


@pytest.mark.parametrize("index_format,cache_format", [("dense", "dense"), ("mxfp4", "dense"), ("dense", "fp8"),
                                                       ("mxfp4", "fp4"), ("mxfp4", "packed")])
def test_cache_snapshot_restore(index_format, cache_format):
    """snapshot() copies every buffer of every cache format (a torch slice would alias the
    buffers the kernels update in place); restore() writes the copies back into the same tensors
    and resets the offset, as generate.py:18-44 does for the reference."""
    from common import C4_TOY, model_args
    from dsv41.cache import _BUFFERS, ModelCache, restore, snapshot
    a = model_args(C4_TOY)
    cache = ModelCache(a, 2, 64, torch.float32, "cpu", index_format, cache_format)
    g = torch.Generator().manual_seed(11)

    def tensors():
        out = []
        for lc in cache.layers:
            for name in _BUFFERS:
                if getattr(lc, name) is not None:
                    out.append(getattr(lc, name))
            if lc.comp_state is not None:
                out += [lc.comp_state.kv_state, lc.comp_state.score_state]
        return out

    def scramble():
        for t in tensors():
            if t.dtype == torch.uint8:
                t.copy_(torch.randint(0, 256, t.shape, generator=g, dtype=torch.uint8))
            else:
                t.copy_(torch.randn(t.shape, generator=g))

    scramble()
    cache.offset = 7
    want = [t.clone() for t in tensors()]
    ptrs = [t.data_ptr() for t in tensors()]
    snap = snapshot(cache)
    scramble()
    cache.offset = 9
    assert not all(torch.equal(t, w) for t, w in zip(tensors(), want))
    restore(cache, snap)
    assert cache.offset == 7
    assert [t.data_ptr() for t in tensors()] == ptrs
    assert all(torch.equal(t, w) for t, w in zip(tensors(), want))
    kinds = {t.dtype for t in tensors()}
    assert (torch.uint8 in kinds) == (index_format != "dense" or cache_format != "dense")


# ------------------------------------------------------------------ wrapper validation
#
# The wrappers validate every caller buffer on the host before the launch. These tests run the
# wrappers over CPU tensors with the device check and the launch replaced by stand-ins: a valid
# call must reach the launch, and each malformed buffer must raise ValueError before it.


class _Launched(Exception):
    pass


@pytest.fixture
def host_abi(monkeypatch):
    from dsv41 import _abi
    calls = []

    def fake_call(name, *args):
        calls.append(name)
        # the wrapper passes exactly the arguments the C declaration takes
        assert len(args) == len(_abi._SIGNATURES[name]), (name, len(args), len(_abi._SIGNATURES[name]))
        raise _Launched(name)

    monkeypatch.setattr(_abi, "_gpu", lambda name, *t: None)
    monkeypatch.setattr(_abi, "_stream", lambda t: None)
    monkeypatch.setattr(_abi, "_call", fake_call)
    return _abi


def _reaches_launch(fn):
    with pytest.raises(_Launched):
        fn()


def _refused(fn, match=None):
    with pytest.raises(ValueError, match=match):
        fn()


def test_validation_helpers():
    from dsv41 import _abi
    ok = torch.zeros(2, 3)
    assert _abi._out("f", ok, (2, 3), torch.float32, "cpu") is ok
    assert _abi._out("f", None, (2, 3), torch.int32, "cpu").dtype == torch.int32
    _refused(lambda: _abi._out("f", torch.zeros(2, 2), (2, 3), torch.float32, "cpu"), "out must be")
    _refused(lambda: _abi._out("f", torch.zeros(2, 3, dtype=torch.bfloat16), (2, 3), torch.float32, "cpu"))
    _refused(lambda: _abi._out("f", torch.zeros(3, 2).t(), (2, 3), torch.float32, "cpu"))
    _refused(lambda: _abi._vec("f", "sink", torch.zeros(4, dtype=torch.bfloat16), 4), "sink")
    _refused(lambda: _abi._vec("f", "sink", torch.zeros(3), 4), "sink")
    _refused(lambda: _abi._tables("f", torch.zeros(8, 4), torch.zeros(8, 4), 16), "rope tables")
    _refused(lambda: _abi._batch("f", "cache", torch.zeros(1, 4, 4), 2), "batch rows")
    assert _abi._ws("f", None, 0, "cpu") is None
    big = torch.zeros(64, dtype=torch.uint8)
    assert _abi._ws("f", big, 32, "cpu") is big
    assert _abi._ws("f", big, 128, "cpu").numel() == 128       # too small: a fresh one
    _refused(lambda: _abi._ws("f", torch.zeros(64), 32, "cpu"), "workspace")


def test_fake_quant_rope_norm_wrappers_check_out(host_abi):
    A = host_abi
    x = torch.zeros(4, 64)
    _reaches_launch(lambda: A.fq_fp8_ue8m0(x, out=torch.zeros(4, 64)))
    _refused(lambda: A.fq_fp8_ue8m0(x, out=torch.zeros(2, 64)))
    _refused(lambda: A.fq_fp4_e4m3(x, out=torch.zeros(4, 64, dtype=torch.bfloat16)))
    cos = sin = torch.zeros(16, 8)
    xr = torch.zeros(1, 4, 2, 64)
    _reaches_launch(lambda: A.rope_tail(xr, 16, cos, sin))
    _refused(lambda: A.rope_tail(xr, 16, cos, sin, out=torch.zeros(1, 4, 2, 32)))
    _refused(lambda: A.rope_tail(xr, 16, cos.double(), sin.double()), "rope tables")
    _reaches_launch(lambda: A.rmsnorm(x, torch.ones(64), 1e-6))
    _refused(lambda: A.rmsnorm(x, torch.ones(64), 1e-6, out=torch.zeros(4, 63)))
    _refused(lambda: A.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6), "weight")
    _reaches_launch(lambda: A.add_rmsnorm(x, torch.zeros(4, 64), torch.ones(64), 1e-6))
    _refused(lambda: A.add_rmsnorm(x, torch.zeros(4, 32), torch.ones(64), 1e-6), "delta")
    _refused(lambda: A.add_rmsnorm(x, torch.zeros(4, 64, dtype=torch.bfloat16), torch.ones(64), 1e-6), "delta")
    _refused(lambda: A.add_rmsnorm(x, torch.zeros(4, 64), torch.ones(64), 1e-6, out=torch.zeros(4, 63)))
    xb = torch.zeros(4, 128, dtype=torch.bfloat16)
    _reaches_launch(lambda: A.linear_rows(xb, torch.zeros(64, 128, dtype=torch.bfloat16)))
    _refused(lambda: A.linear_rows(xb, torch.zeros(64, 96, dtype=torch.bfloat16)), "contract")
    _refused(lambda: A.linear_rows(xb.float(), torch.zeros(64, 128)), "bfloat16")
    wa, wb = torch.zeros(64, 128, dtype=torch.bfloat16), torch.zeros(32, 128, dtype=torch.bfloat16)
    _reaches_launch(lambda: A.linear_rows_pair(xb, wa, wb))
    _refused(lambda: A.linear_rows_pair(xb, wa, torch.zeros(32, 96, dtype=torch.bfloat16)), "contract")
    _refused(lambda: A.linear_rows_pair(xb, wa, wb.float()), "bfloat16")


def test_cache_writers_check_batch_rows_and_parameters(host_abi):
    A = host_abi
    cos = sin = torch.zeros(64, 8)
    lat = torch.zeros(2, 3, 64)
    _reaches_launch(lambda: A.comp_write(lat, torch.zeros(2, 8, 64), 0, 4, cos, sin, 16))
    _refused(lambda: A.comp_write(lat, torch.zeros(1, 8, 64), 0, 4, cos, sin, 16), "batch rows")
    k = torch.zeros(2, 3, 32)
    _reaches_launch(lambda: A.index_key_publish(k, torch.zeros(2, 8, 32), 0, 4, torch.ones(32), cos, sin, 16,
                                                1e-6))
    _refused(lambda: A.index_key_publish(k, torch.zeros(1, 8, 32), 0, 4, torch.ones(32), cos, sin, 16, 1e-6),
             "batch rows")
    _refused(lambda: A.index_key_publish(k, torch.zeros(2, 8, 32), 0, 4, torch.ones(16), cos, sin, 16, 1e-6),
             "k_norm")
    kv = torch.zeros(2, 1, 64)
    _reaches_launch(lambda: A.kv_window_prep(kv, torch.ones(64), cos, sin, 16, 0, 1e-6))
    _refused(lambda: A.kv_window_prep(kv, torch.ones(64, dtype=torch.bfloat16), cos, sin, 16, 0, 1e-6),
             "norm weight")
    st = torch.zeros(2, 4, 64)
    _reaches_launch(lambda: A.compress_pool(kv, kv.clone(), st, st.clone(), torch.ones(64), 4, 3, 1e-6,
                                            torch.float32))
    _refused(lambda: A.compress_pool(kv, kv.clone(), st, torch.zeros(2, 4, 32), torch.ones(64), 4, 3, 1e-6,
                                     torch.float32), "state")
    _refused(lambda: A.compress_pool(kv, kv.clone(), st, st.clone(), torch.ones(32), 4, 3, 1e-6,
                                     torch.float32), "norm weight")
    lat512 = torch.zeros(2, 3, 512)
    _reaches_launch(lambda: A.comp_write_fp4(lat512, torch.zeros(2, 8, 288, dtype=torch.uint8), 5, 4, cos, sin, 16))
    _refused(lambda: A.comp_write_fp4(lat512, torch.zeros(2, 7, 288, dtype=torch.uint8), 5, 4, cos, sin, 16),
             "cannot take")
    _refused(lambda: A.comp_write_fp4(lat512, torch.zeros(2, 8, 256, dtype=torch.uint8), 5, 4, cos, sin, 16),
             "cannot take")
    _refused(lambda: A.comp_write_fp4(lat512, torch.zeros(1, 8, 288, dtype=torch.uint8), 5, 4, cos, sin, 16),
             "batch rows")


def test_indexer_and_topk_wrappers_check_out(host_abi):
    A = host_abi
    q = torch.zeros(2, 1, 4, 32)
    w = torch.zeros(2, 1, 4)
    ik = torch.zeros(2, 16, 32)
    _reaches_launch(lambda: A.indexer_score(q, w, 0.1, ik, 64, 4))
    _refused(lambda: A.indexer_score(q, w, 0.1, ik, 64, 4, out=torch.zeros(2, 1, 8)))
    _refused(lambda: A.indexer_score(q, w, 0.1, ik, 64, 4, out=torch.zeros(2, 1, 16, dtype=torch.bfloat16)))
    s = torch.zeros(2, 1, 16)
    _reaches_launch(lambda: A.topk_select(s, 4, 64, 4, 0))
    _refused(lambda: A.topk_select(s, 4, 64, 4, 0, out=torch.zeros(2, 1, 3, dtype=torch.int32)))
    _refused(lambda: A.topk_select(s, 4, 64, 4, 0, out=torch.zeros(2, 1, 4)))


def test_sparse_mla_wrappers_check_buffers(host_abi):
    A = host_abi
    b, h, d, W = 2, 16, 512, 8
    q = torch.zeros(b, 1, h, d, dtype=torch.bfloat16)
    ring = torch.zeros(b, W, d, dtype=torch.bfloat16)
    chunk = torch.zeros(b, 1, d, dtype=torch.bfloat16)
    comp = torch.zeros(b, 1024, d, dtype=torch.bfloat16)
    sink = torch.zeros(h)
    idx = torch.zeros(b, 1, 512, dtype=torch.int32)    # long enough that the list is split
    cos = sin = torch.zeros(128, 32)
    assert A.mla_workspace_bytes(b, 1, h, d, W + 512, torch.bfloat16) > 0

    def call(**kw):
        args = dict(q=q, win_kv=ring, chunk_kv=chunk, comp_kv=comp, n_comp=1000, attn_sink=sink, idx=idx,
                    softmax_scale=0.1, window=W, start_pos=64, cos=cos, sin=sin, rd=64)
        args.update(kw)
        return lambda: A.sparse_mla(**args)

    _reaches_launch(call())
    _reaches_launch(call(write_ring=True))
    _refused(call(out=torch.zeros(b, 1, h, d // 2, dtype=torch.bfloat16)), "out must be")
    _refused(call(out=torch.zeros(b, 1, h, d)), "out must be")
    _refused(call(comp_kv=comp[:1]), "batch rows")
    _refused(call(attn_sink=sink.to(torch.bfloat16)), "attn_sink")
    _refused(call(attn_sink=torch.zeros(h - 1)), "attn_sink")
    _refused(call(cos=cos[:, :16], sin=sin[:, :16]), "rope tables")
    _reaches_launch(call(q_rd=64))                # q's rope tail in the launch, one table for both
    _reaches_launch(call(rd=0, q_rd=64))
    _refused(call(q_rd=32), "one shared rope width")
    _refused(call(rd=0, q_rd=64, cos=None, sin=None), "rope tables")
    _refused(call(q_rd=64, start_pos=200), "rope table too short")
    _refused(call(workspace=torch.zeros(1 << 20)), "workspace")
    codes = torch.zeros(b, 1024, d, dtype=torch.uint8)
    scales = torch.zeros(b, 32, d // 32, dtype=torch.uint8)

    def call8(**kw):
        args = dict(q=q, win_kv=ring, chunk_kv=chunk, comp8=codes, comp_scale=scales, scale_rb=32, n_comp=1000,
                    attn_sink=sink, idx=idx, softmax_scale=0.1, window=W, start_pos=64, cos=cos, sin=sin, rd=64)
        args.update(kw)
        return lambda: A.sparse_mla_fp8(**args)

    _reaches_launch(call8())
    _reaches_launch(call8(q_rd=64, write_ring=True))
    _refused(call8(out=torch.zeros(b, 1, h, d - 32, dtype=torch.bfloat16)), "out must be")
    _refused(call8(comp8=codes[:1], comp_scale=scales[:1]), "does not match")
    _refused(call8(attn_sink=sink.double()), "attn_sink")
    packed = torch.zeros(b, 1024, 288, dtype=torch.uint8)

    def call4(**kw):
        args = dict(q=q, win_kv=ring, chunk_kv=chunk, comp_kv4=packed, n_comp=1000, attn_sink=sink, idx=idx,
                    softmax_scale=0.1, window=W, start_pos=64, cos=cos, sin=sin, rd=64)
        args.update(kw)
        return lambda: A.sparse_mla_fp4(**args)

    _reaches_launch(call4())
    _reaches_launch(call4(write_ring=True))
    _reaches_launch(call4(write_ring=True, q_rd=64))
    _refused(call4(q_rd=-2), "one shared rope width")
    _refused(call4(comp_kv4=packed[:1]), "batch rows")
    _refused(call4(comp_kv4=torch.zeros(b, 1024, 256, dtype=torch.uint8)), "does not match")
    _refused(call4(comp_kv4=packed[:, :999]), "does not match")
    _refused(call4(q=q.float()), "bf16")
    _refused(call4(chunk_kv=torch.zeros(b, 2, d, dtype=torch.bfloat16), write_ring=True), "chunk kv")
    _refused(call4(win_kv=None, write_ring=True), "window ring")
    ring8 = torch.zeros(b, W, 528, dtype=torch.uint8)

    def callp(**kw):
        args = dict(q=q, win_kv8=ring8, chunk_kv=chunk, comp_kv4=packed, n_comp=1000, attn_sink=sink, idx=idx,
                    softmax_scale=0.1, window=W, start_pos=64, cos=cos, sin=sin, rd=64)
        args.update(kw)
        return lambda: A.sparse_mla_packed(**args)

    _reaches_launch(callp())
    _reaches_launch(callp(write_ring=True))
    _reaches_launch(callp(write_ring=True, q_rd=64))
    o = torch.zeros(3, 1, 8 * 512, dtype=torch.bfloat16)
    wa = torch.zeros(8 * 128, 512, dtype=torch.bfloat16)
    _reaches_launch(lambda: A.wo_a_grouped(o, wa, 8))
    _reaches_launch(lambda: A.wo_a_grouped(o, wa, 8, out=torch.zeros(3, 1, 1024), out_dtype=torch.float32))
    _refused(lambda: A.wo_a_grouped(o, wa, 8, out=torch.zeros(3, 1, 1024)), "out must be")   # bf16 by default
    _refused(lambda: A.wo_a_grouped(o, wa.float(), 8), "share a dtype")
    _refused(lambda: A.wo_a_grouped(o, wa, 3), "groups")
    _refused(lambda: A.wo_a_grouped(o[..., :-8].contiguous(), wa, 8), "last dim")
    _refused(lambda: A.wo_a_grouped(o, wa, 8, out=torch.zeros(3, 1, 1000, dtype=torch.bfloat16)), "out must be")
    _reaches_launch(callp(comp_kv4=None, n_comp=0, idx=None))
    _refused(callp(win_kv8=ring), "window ring")                      # a bf16 ring is not MXFP8
    _refused(callp(win_kv8=ring8[:, :, :512]), "window ring")
    _refused(callp(win_kv8=None), "window ring")
    _reaches_launch(lambda: A.window_write_mxfp8(ring8, torch.zeros(b, 3, d, dtype=torch.bfloat16), 5))
    _refused(lambda: A.window_write_mxfp8(ring8[:1], torch.zeros(b, 3, d, dtype=torch.bfloat16), 5), "batch rows")
    _refused(lambda: A.window_write_mxfp8(ring, torch.zeros(b, 3, d, dtype=torch.bfloat16), 5), "MXFP8")
