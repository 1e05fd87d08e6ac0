"""ctypes binding of libdsv41.so, the C ABI declared in include/dsv41.h.

Every wrapper takes torch tensors that must already live on the GPU, checks dtype, shape
and contiguity the way the reference's TileLang wrappers assert them
(docs/reference/kernel.py:108, 193-194, 286-298), passes raw device pointers and torch's
current stream, and turns a non-zero status into an exception: ``ValueError`` for a
contract violation (negative dsv41_status), ``RuntimeError`` for a HIP launch error.

There is no fallback: if the library is missing, or a tensor is not on a GPU, the call
raises. The kernels run on the HIP path or not at all.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_NAME = "libdsv41.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, BF16, FP8_E4M3 = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16}

_c_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> argtypes, mirroring include/dsv41.h
_SIGNATURES = {
    "dsv41_fq_fp8_ue8m0": [_c_p, _c_p, _i64, _i32, _i32, _i32, _c_p],
    "dsv41_fq_fp4_ue8m0": [_c_p, _c_p, _i64, _i32, _i32, _i32, _c_p],
    "dsv41_fq_fp4_e4m3": [_c_p, _c_p, _i64, _i32, _i32, _i32, _c_p],
    "dsv41_rope_table": [_c_p, _c_p, _c_p, _i32, _i32, _c_p],
    "dsv41_rope_tail": [_c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _c_p, _c_p, _i32, _i32, _i32,
                        _i32, _c_p],
    "dsv41_rmsnorm": [_c_p, _c_p, _c_p, _i64, _i32, _f32, _i32, _c_p],
    "dsv41_add_rmsnorm": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _f32, _i32, _c_p],
    "dsv41_kv_window_prep": [_c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
                             _c_p],
    "dsv41_window_write": [_c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_window_idx": [_c_p, _i32, _i32, _i32, _c_p],
    "dsv41_compress_pool": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32,
                            _f32, _i32, _c_p],
    "dsv41_comp_write": [_c_p, _c_p, _i64, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                         _c_p],
    "dsv41_index_key_publish": [_c_p, _c_p, _i64, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32,
                                _i32, _f32, _i32, _c_p],
    "dsv41_index_key_publish_mxfp4": [_c_p, _c_p, _i64, _c_p, _i64, _c_p, _c_p, _c_p, _i32, _i32, _i32,
                                      _i32, _i32, _i32, _f32, _i32, _c_p],
    "dsv41_index_q_prep": [_c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_indexer_score": [_c_p, _c_p, _f32, _c_p, _i64, _c_p, _c_p, _i32, _i32, _i32, _i32,
                            _i32, _i32, _i32, _i32, _c_p],
    "dsv41_indexer_score_fp8": [_c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _i32,
                                _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_index_q_prep_mxfp4": [_c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                 _c_p],
    "dsv41_indexer_score_mxfp4": [_c_p, _c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _c_p, _c_p, _i32, _i32,
                                  _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_topk_select": [_c_p, _c_p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_topk_workspace_bytes": [_i64, _i32, _i32],
    "dsv41_indexer_topk_workspace_bytes": [_i32, _i32, _i32, _i32, _i32, _i32, _i32],
    "dsv41_indexer_topk": [_c_p, _c_p, _f32, _c_p, _i64, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                           _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_indexer_topk_fp8": [_c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _i32, _i32, _i32, _i32,
                               _i32, _i32, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_indexer_topk_mxfp4": [_c_p, _c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _c_p, _c_p, _i32, _i32, _i32,
                                 _i32, _i32, _i32, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_topk_select_ws": [_c_p, _c_p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_candidate_blocks": [_c_p, _c_p, _i64, _i32, _i32, _i32, _i32, _c_p, _i32, _i32, _c_p],
    "dsv41_sparse_mla_workspace_bytes": [_i32, _i32, _i32, _i32, _i32, _i32],
    "dsv41_sparse_attn": [_c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                          _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32,
                         _i32, _f32, _c_p, _c_p, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_decode": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32,
                                _i32, _f32, _c_p, _c_p, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_decode_noalloc": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32,
                                        _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _i32, _c_p],
    "dsv41_sparse_mla_fp8": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32,
                             _i32, _i32, _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_fp8_decode": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p,
                                    _i32, _i32, _i32, _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_comp_write_fp4": [_c_p, _c_p, _i64, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_sparse_mla_fp4": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32, _i32,
                             _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_fp4_decode": [_c_p, _c_p, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32,
                                    _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_packed": [_c_p, _c_p, _i64, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32,
                                _i32, _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_sparse_mla_packed_decode": [_c_p, _c_p, _i64, _c_p, _c_p, _i64, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32,
                                       _i32, _i32, _i32, _f32, _c_p, _c_p, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_window_write_mxfp8": [_c_p, _i64, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_wo_a_grouped": [_c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_linear_rows_workspace_bytes": [_i32, _i32, _i32],
    "dsv41_linear_rows": [_c_p, _c_p, _c_p, _c_p, _sz, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_linear_rows_pair": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _sz, _i32, _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_comp_write_fp8": [_c_p, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32,
                             _i32, _c_p],
    "dsv41_index_key_publish_fp8": [_c_p, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32,
                                    _i32, _i32, _f32, _i32, _c_p],
    "dsv41_indexer_score_mxq_fp8": [_c_p, _c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _i32, _i32,
                                    _i32, _i32, _i32, _i32, _i32, _c_p],
    "dsv41_indexer_topk_mxq_fp8": [_c_p, _c_p, _c_p, _f32, _c_p, _i64, _c_p, _i64, _i32, _c_p, _c_p, _i32, _i32,
                                   _i32, _i32, _i32, _i32, _i32, _i32, _i32, _c_p, _sz, _c_p],
    "dsv41_version": [],
    "dsv41_last_error_string": [],
}
_RESTYPES = {
    "dsv41_sparse_mla_workspace_bytes": _sz,
    "dsv41_linear_rows_workspace_bytes": _sz,
    "dsv41_topk_workspace_bytes": _sz,
    "dsv41_indexer_topk_workspace_bytes": _sz,
    "dsv41_version": ctypes.c_char_p,
    "dsv41_last_error_string": ctypes.c_char_p,
}

_LIB = None


def lib() -> ctypes.CDLL:
    """Load libdsv41.so (once). Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python deepseek-v41-mlx_amd/build.py` "
                "(or __graft_entry__.build()); the dsv41 kernels have no fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _LIB = handle
    return _LIB


def version() -> str:
    return lib().dsv41_version().decode()


def _check(rc: int, name: str) -> None:
    if rc == 0:
        return
    msg = (lib().dsv41_last_error_string() or b"").decode()
    if rc < 0:
        raise ValueError(f"{name}: {msg} (status {rc})")
    raise RuntimeError(f"{name}: {msg} (hipError {rc})")


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _gpu(name: str, *tensors):
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
        if not t.is_cuda:
            raise ValueError(f"{name}: tensor on {t.device}; the dsv41 kernels run on the GPU only")


def _contig(name: str, *tensors):
    for t in tensors:
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name}: tensor of shape {tuple(t.shape)} must be contiguous")


def _out(name: str, out, shape, dtype, device) -> torch.Tensor:
    """The output tensor: allocated when the caller passes none, else checked for device, dtype,
    exact shape and contiguity, so a wrong buffer raises here instead of reaching a kernel."""
    shape = tuple(int(x) for x in shape)
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if not isinstance(out, torch.Tensor) or out.device != torch.device(device):
        raise ValueError(f"{name}: out must be a tensor on {device}")
    if out.dtype != dtype or tuple(out.shape) != shape or not out.is_contiguous():
        raise ValueError(f"{name}: out must be contiguous {dtype} {list(shape)}, "
                         f"got {out.dtype} {list(out.shape)}")
    return out


def _vec(name: str, what: str, t: torch.Tensor, n: int, dtype=torch.float32) -> None:
    """A per-channel or per-head parameter vector (norm weight, attention sink)."""
    if t is None or t.dtype != dtype or t.numel() != n or not t.is_contiguous():
        got = "None" if t is None else f"{t.dtype} {list(t.shape)}"
        raise ValueError(f"{name}: {what} must be contiguous {dtype} [{n}], got {got}")


def _tables(name: str, cos, sin, rd: int) -> None:
    """Rope tables: fp32 [positions, rd/2], contiguous, the same shape."""
    if (cos is None or sin is None or cos.dtype != torch.float32 or sin.dtype != torch.float32
            or cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] * 2 != rd):
        raise ValueError(f"{name}: rope tables must be fp32 [positions, {rd // 2}]")
    _contig(name, cos, sin)


def _attn_tables(name: str, cos, sin, rd: int, q_rd: int, start_pos: int, n: int) -> None:
    """The rope tables of a sparse_mla form: rd (the output's inverse rope) and q_rd (q's forward
    rope, applied as q loads) share one table, so nonzero widths must agree; positions
    start_pos .. start_pos + n - 1 must be in it."""
    if rd < 0 or q_rd < 0 or (rd and q_rd and rd != q_rd):
        raise ValueError(f"{name}: rd {rd} and q_rd {q_rd} must be 0 or one shared rope width")
    w = rd or q_rd
    if w:
        _tables(name, cos, sin, w)
        if n and start_pos + n - 1 >= cos.shape[0]:
            raise ValueError(f"{name}: rope table too short")


def _batch(name: str, what: str, t: torch.Tensor, b: int) -> None:
    if t.shape[0] < b:
        raise ValueError(f"{name}: {what} holds {t.shape[0]} batch rows, the call needs {b}")


def _ws(name: str, workspace, nbytes: int, device):
    """A caller's uint8 workspace when it is large enough, else a fresh one (None when the
    call needs none)."""
    if not nbytes:
        return None
    if workspace is not None:
        if (not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8
                or workspace.device != torch.device(device) or not workspace.is_contiguous()):
            raise ValueError(f"{name}: workspace must be a contiguous uint8 tensor on {device}")
        if workspace.numel() >= nbytes:
            return workspace
    return _workspace(nbytes, device)


def dtype_code(t: torch.Tensor, name: str) -> int:
    if t.dtype not in _DTYPES:
        raise ValueError(f"{name}: dtype {t.dtype} not supported (float32 or bfloat16)")
    return _DTYPES[t.dtype]


def _call(name: str, *args) -> None:
    _check(getattr(lib(), name)(*args), name)


def row_stride(t: torch.Tensor, name: str) -> int:
    """Batch stride (elements) of a [b, rows, dim] view whose rows are dense."""
    if t.dim() != 3 or t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        raise ValueError(f"{name}: cache view must be [b, rows, dim] with dense rows")
    return t.stride(0)


# ---------------------------------------------------------------------------- fake-quant


def _fq(name: str, x: torch.Tensor, block: int, out: torch.Tensor | None) -> torch.Tensor:
    _gpu(name, x, out)
    _contig(name, x)
    out = _out(name, out, x.shape, x.dtype, x.device)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    _call(name, _ptr(x), _ptr(out), rows, cols, block, dtype_code(x, name), _stream(x))
    return out


def fq_fp8_ue8m0(x, block=32, out=None):
    return _fq("dsv41_fq_fp8_ue8m0", x, block, out)


def fq_fp4_ue8m0(x, block=32, out=None):
    return _fq("dsv41_fq_fp4_ue8m0", x, block, out)


def fq_fp4_e4m3(x, block=16, out=None):
    return _fq("dsv41_fq_fp4_e4m3", x, block, out)


# ---------------------------------------------------------------------------- rope / norm


def rope_table(freqs: torch.Tensor, seqlen: int):
    """cos, sin [seqlen, half] fp32 on freqs' device."""
    name = "dsv41_rope_table"
    _gpu(name, freqs)
    freqs = freqs.to(torch.float32).contiguous()
    half = freqs.numel()
    cos = torch.empty(seqlen, half, dtype=torch.float32, device=freqs.device)
    sin = torch.empty_like(cos)
    _call(name, _ptr(cos), _ptr(sin), _ptr(freqs), seqlen, half, _stream(freqs))
    return cos, sin


def rope_tail(x, rd, cos, sin, pos_base=0, pos_step=1, inverse=False, out=None):
    """x [b, s, d] or [b, s, h, d]; rows of the tables at pos_base + s*pos_step."""
    name = "dsv41_rope_tail"
    _gpu(name, x, cos, sin, out)
    _contig(name, x)
    if x.dim() not in (3, 4):
        raise ValueError(f"{name}: x must be [b, s, d] or [b, s, h, d], got {tuple(x.shape)}")
    b, s = x.shape[0], x.shape[1]
    h = x.shape[2] if x.dim() == 4 else 1
    d = x.shape[-1]
    if rd > d or rd % 2:
        raise ValueError(f"{name}: rd={rd} must be even and at most {d}")
    _tables(name, cos, sin, rd)
    last = pos_base + (s - 1) * pos_step if s else 0
    if s and last >= cos.shape[0]:
        raise ValueError(f"{name}: position {last} beyond the rope table ({cos.shape[0]} rows)")
    out = _out(name, out, x.shape, x.dtype, x.device)
    _call(name, _ptr(x), _ptr(out), b, s, h, d, rd, _ptr(cos), _ptr(sin), pos_base, pos_step,
          1 if inverse else 0, dtype_code(x, name), _stream(x))
    return out


def rmsnorm(x, weight, eps, out=None):
    name = "dsv41_rmsnorm"
    _gpu(name, x, weight, out)
    _contig(name, x)
    _vec(name, "weight", weight, x.shape[-1])
    out = _out(name, out, x.shape, x.dtype, x.device)
    d = x.shape[-1]
    _call(name, _ptr(x), _ptr(out), _ptr(weight), x.numel() // d, d, float(eps),
          dtype_code(x, name), _stream(x))
    return out


def add_rmsnorm(h, delta, weight, eps, out=None):
    """h <- cast(h + delta) in place, then rmsnorm(h): the residual add of one block and the next
    block's attn_norm (model.py:141-154 with layers.py:20-33) in one pass over the rows."""
    name = "dsv41_add_rmsnorm"
    _gpu(name, h, delta, weight, out)
    _contig(name, h, delta)
    if delta.shape != h.shape or delta.dtype != h.dtype:
        raise ValueError(f"{name}: delta {tuple(delta.shape)} {delta.dtype} must match h {tuple(h.shape)} {h.dtype}")
    _vec(name, "weight", weight, h.shape[-1])
    out = _out(name, out, h.shape, h.dtype, h.device)
    d = h.shape[-1]
    _call(name, _ptr(h), _ptr(delta), _ptr(out), _ptr(weight), h.numel() // d, d, float(eps),
          dtype_code(h, name), _stream(h))
    return out


# ---------------------------------------------------------------------------- window


def kv_window_prep(kv, norm_w, cos, sin, rd, start_pos, eps):
    name = "dsv41_kv_window_prep"
    _gpu(name, kv, norm_w, cos, sin)
    _contig(name, kv)
    b, n, d = kv.shape
    _vec(name, "norm weight", norm_w, d)
    _tables(name, cos, sin, rd)
    if n and start_pos + n - 1 >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(kv), _ptr(norm_w), _ptr(cos), _ptr(sin), b, n, d, rd, start_pos, float(eps),
          dtype_code(kv, name), _stream(kv))
    return kv


def window_write(win_kv, kv, start_pos):
    name = "dsv41_window_write"
    _gpu(name, win_kv, kv)
    _contig(name, win_kv, kv)
    if win_kv.dtype != kv.dtype:
        raise ValueError(f"{name}: ring dtype {win_kv.dtype} != kv dtype {kv.dtype}")
    b, n, d = kv.shape
    if win_kv.shape[0] < b or win_kv.shape[2] != d:
        raise ValueError(f"{name}: ring {tuple(win_kv.shape)} does not hold kv {tuple(kv.shape)}")
    # rows past b in the ring are untouched: the kernel indexes [b, window, d]
    ring = win_kv[:b]
    _call(name, _ptr(ring), _ptr(kv), b, n, d, win_kv.shape[1], start_pos, dtype_code(kv, name),
          _stream(kv))


def window_idx(wp, n, window, device):
    name = "dsv41_window_idx"
    weff = min(window, wp + n)
    out = torch.empty(n, weff, dtype=torch.int32, device=device)
    if out.numel():
        _call(name, _ptr(out), wp, n, window, ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    return out


# ---------------------------------------------------------------------------- compressor


def compress_pool(kv, score, kv_state, score_state, norm_w, ratio, start_pos, eps, dtype):
    """Returns latents [b, g, d] in `dtype` (None when no group completes)."""
    name = "dsv41_compress_pool"
    _gpu(name, kv, score, kv_state, score_state, norm_w)
    _contig(name, kv, score, kv_state, score_state, norm_w)
    for t in (kv, score, kv_state, score_state):
        if t.dtype != torch.float32:
            raise ValueError(f"{name}: kv/score/state must be fp32")
    b, n, d = kv.shape
    if score.shape != kv.shape:
        raise ValueError(f"{name}: score {tuple(score.shape)} must match kv {tuple(kv.shape)}")
    for st in (kv_state, score_state):
        if st.dim() != 3 or st.shape[0] < b or st.shape[1:] != (ratio, d):
            raise ValueError(f"{name}: state {tuple(st.shape)} does not match [>={b}, {ratio}, {d}]")
    _vec(name, "norm weight", norm_w, d)
    g = (start_pos % ratio + n) // ratio
    lat = torch.empty(b, g, d, dtype=dtype, device=kv.device) if g else None
    code = _DTYPES.get(dtype)
    if code is None:
        raise ValueError(f"{name}: dtype {dtype} not supported")
    _call(name, _ptr(kv), _ptr(score), _ptr(kv_state), _ptr(score_state), _ptr(lat), _ptr(norm_w),
          b, n, d, ratio, start_pos, float(eps), code, _stream(kv))
    return lat


def comp_write(latents, comp_kv, g0, ratio, cos, sin, rd):
    name = "dsv41_comp_write"
    _gpu(name, latents, comp_kv, cos, sin)
    _contig(name, latents)
    _tables(name, cos, sin, rd)
    b, g, d = latents.shape
    if comp_kv.dtype != latents.dtype:
        raise ValueError(f"{name}: cache dtype {comp_kv.dtype} != latent dtype {latents.dtype}")
    _batch(name, "the compressed cache", comp_kv, b)
    if comp_kv.shape[1] < g0 + g or comp_kv.shape[2] != d:
        raise ValueError(f"{name}: cache {tuple(comp_kv.shape)} cannot take groups {g0}..{g0 + g}")
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(latents), _ptr(comp_kv), row_stride(comp_kv, name), _ptr(cos), _ptr(sin), b, g, d,
          rd, g0, ratio, dtype_code(latents, name), _stream(latents))


def index_key_publish(k_raw, index_k, g0, ratio, norm_w, cos, sin, rd, eps):
    name = "dsv41_index_key_publish"
    _gpu(name, k_raw, index_k, norm_w, cos, sin)
    _contig(name, k_raw)
    _tables(name, cos, sin, rd)
    b, g, d = k_raw.shape
    _vec(name, "k_norm weight", norm_w, d)
    if index_k.dtype != k_raw.dtype:
        raise ValueError(f"{name}: cache dtype {index_k.dtype} != key dtype {k_raw.dtype}")
    _batch(name, "the index-key cache", index_k, b)
    if index_k.shape[1] < g0 + g or index_k.shape[2] != d:
        raise ValueError(f"{name}: cache {tuple(index_k.shape)} cannot take groups {g0}..{g0 + g}")
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(k_raw), _ptr(index_k), row_stride(index_k, name), _ptr(norm_w), _ptr(cos),
          _ptr(sin), b, g, d, rd, g0, ratio, float(eps), dtype_code(k_raw, name), _stream(k_raw))


def _fp8_rows(name, src, codes, scales, g0, scale_rb=1):
    b, g, d = src.shape
    if scale_rb not in (1, 32):
        raise ValueError(f"{name}: scale_rb must be 1 or 32, got {scale_rb}")
    if codes.dtype != torch.uint8 or codes.shape[0] < b or codes.shape[2] != d or codes.shape[1] < g0 + g:
        raise ValueError(f"{name}: code cache {tuple(codes.shape)} cannot take groups {g0}..{g0 + g}")
    nblk = -(-(g0 + g) // scale_rb)
    if scales.dtype != torch.uint8 or scales.shape[0] < b or scales.shape[2] != d // 32 or scales.shape[1] < nblk:
        raise ValueError(f"{name}: scale cache {tuple(scales.shape)} cannot take groups {g0}..{g0 + g}")
    return b, g, d


def comp_write_fp8(latents, codes, scales, g0, ratio, cos, sin, rd, scale_rb=1):
    """comp_write into an fp8 cache: codes uint8 [b, >=g0+g, d] e4m3fn, scales uint8
    [b, >=ceil((g0+g)/scale_rb), d/32] ue8m0 (one per 32 channels of every scale_rb rows), values
    fq_fp8_ue8m0(rope(latent)); with scale_rb 32 the row opening a block sets its scale, later rows
    are rounded with it."""
    name = "dsv41_comp_write_fp8"
    _gpu(name, latents, codes, scales, cos, sin)
    _contig(name, latents)
    _tables(name, cos, sin, rd)
    b, g, d = _fp8_rows(name, latents, codes, scales, g0, scale_rb)
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(latents), _ptr(codes), row_stride(codes, name), _ptr(scales), row_stride(scales, name), scale_rb,
          _ptr(cos), _ptr(sin), b, g, d, rd, g0, ratio, dtype_code(latents, name), _stream(latents))


def mxfp8_row_bytes(d: int) -> int:
    """Bytes of one MXFP8 window-ring row: d e4m3fn codes, then d/32 ue8m0 scales."""
    return d + d // 32


def window_write_mxfp8(win_kv8, kv, start_pos):
    """window_write into an MXFP8 ring: win_kv8 uint8 [b, window, d + d/32], position p at slot
    p % window; each row stored as fake_quant_fp8_ue8m0's codes and block scales (exact for window
    KV that carries that QAT)."""
    name = "dsv41_window_write_mxfp8"
    _gpu(name, win_kv8, kv)
    _contig(name, kv)
    b, n, d = kv.shape
    if win_kv8.dtype != torch.uint8 or win_kv8.dim() != 3 or win_kv8.shape[2] != mxfp8_row_bytes(d):
        raise ValueError(f"{name}: ring {tuple(win_kv8.shape)} {win_kv8.dtype} does not hold {d}-channel MXFP8 rows")
    _batch(name, "the window ring", win_kv8, b)
    _call(name, _ptr(win_kv8), row_stride(win_kv8, name), _ptr(kv), b, n, d, win_kv8.shape[1], start_pos,
          dtype_code(kv, name), _stream(kv))


def fp4_row_bytes(d: int) -> int:
    """Bytes of one packed fp4 compressed-cache row: d/2 code bytes, then d/16 e4m3 scales."""
    return d // 2 + d // 16


def wo_a_grouped(o, wo_a, groups, out=None, out_dtype=None):
    """The grouped block-diagonal output LoRA (attention.py:176-179): o [..., groups*d] (the
    attention output; its leading dims are the rows), wo_a [groups*r, d] (the Linear weight,
    read in place), both bf16 or both float32. Returns [..., groups*r] in out_dtype (o's dtype
    by default, the reference's cast of its fp32 einsum; float32 gives the einsum itself)."""
    name = "dsv41_wo_a_grouped"
    _gpu(name, o, wo_a, out)
    _contig(name, o, wo_a)
    if o.dtype != wo_a.dtype:
        raise ValueError(f"{name}: o {o.dtype} and wo_a {wo_a.dtype} must share a dtype")
    if groups <= 0 or wo_a.dim() != 2 or wo_a.shape[0] % groups:
        raise ValueError(f"{name}: wo_a {tuple(wo_a.shape)} is not [groups * r, d] for {groups} groups")
    d, r = wo_a.shape[1], wo_a.shape[0] // groups
    if o.dim() < 1 or o.shape[-1] != groups * d:
        raise ValueError(f"{name}: o's last dim must be groups * d = {groups * d}, got {tuple(o.shape)}")
    out_dtype = o.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"{name}: out_dtype must be bf16 or float32")
    rows = o.numel() // (groups * d)
    out = _out(name, out, (*o.shape[:-1], groups * r), out_dtype, o.device)
    _call(name, _ptr(o), _ptr(wo_a), _ptr(out), rows, groups, d, r, dtype_code(o, name), dtype_code(out, name),
          _stream(o))
    return out


def linear_rows_wide_tile(rows: int, k: int, n: int, splits: int) -> int:
    """The weight rows of dsv41_linear_rows's wide tiles for this call, 0 when it takes the 32-row
    ones (the kernel's own rule, out_proj.hip wide_split_tile): 33-64 rows, each contraction range
    at least 1024 channels, and of 128- and 160-row tiles dividing n the one whose n / tile x splits
    workgroups is largest within 128-256."""
    if not 32 < rows <= 64 or k // splits < 1024:
        return 0
    best, best_t = 0, 0
    for tr in (128, 160):
        t = (n // tr) * splits
        if n % tr == 0 and 128 <= t <= 256 and t > best_t:
            best, best_t = tr, t
    return best


def linear_rows_wide(rows: int, k: int, n: int, splits: int) -> bool:
    """Whether dsv41_linear_rows takes its wide (128- or 160-row) weight tiles for this call."""
    return linear_rows_wide_tile(rows, k, n, splits) != 0


def linear_rows_splits(k: int, n: int, rows: int = 64) -> int:
    """Contraction ranges for dsv41_linear_rows (whole 64-channel steps, at most 64). At 33-64 rows
    the ranges whose wide tiles (linear_rows_wide) make the most workgroups when some do; otherwise the most
    that keep the n / 32 x ranges workgroups within one wave of the chip (256: one workgroup per
    CU; a 320-workgroup wq_a ran a second round of 64 and took 9.0 us)."""
    wide = [((n // linear_rows_wide_tile(rows, k, n, s)) * s, s) for s in range(1, 65)
            if k % (64 * s) == 0 and linear_rows_wide(rows, k, n, s)]
    if wide:
        return max(wide)[1]                    # the most workgroups, then the most ranges
    tiles = max(n // 32, 1)
    best = 1
    for s in range(1, 65):
        if k % (64 * s) == 0 and tiles * s <= 256:
            best = s
    return best


def _linear_args(name, x, *ws):
    _gpu(name, x, *ws)
    _contig(name, x, *ws)
    if x.dtype != torch.bfloat16 or any(w.dtype != torch.bfloat16 for w in ws):
        raise ValueError(f"{name}: x and w must be bfloat16")
    for w in ws:
        if w.dim() != 2 or x.shape[-1] != w.shape[1]:
            raise ValueError(f"{name}: x {tuple(x.shape)} and w {tuple(w.shape)} do not contract")
    return ws[0].shape[1], x.numel() // ws[0].shape[1]


def linear_rows(x, w, splits=None, out=None, workspace=None):
    """y = x @ w^T for decode row counts (at most 128 rows of x [..., k]; w [n, k] the Linear
    weight, read in place), bf16: the projections of attention.py:114-116 and :179 on the decode
    tile kernel with the contraction split over `splits` ranges (linear_rows_splits by default)."""
    name = "dsv41_linear_rows"
    k, rows = _linear_args(name, x, w)
    n = w.shape[0]
    if splits is None:
        splits = linear_rows_splits(k, n, rows)
    out = _out(name, out, (*x.shape[:-1], n), torch.bfloat16, x.device)
    need = lib().dsv41_linear_rows_workspace_bytes(rows, n, splits)
    ws = _ws(name, workspace, need, x.device)
    _call(name, _ptr(x), _ptr(w), _ptr(out), _ptr(ws) if ws is not None else None, need, rows, k, n, splits,
          dtype_code(x, name), _stream(x))
    return out


def linear_rows_pair(x, w0, w1, splits=None, out0=None, out1=None, workspace=None):
    """(x @ w0^T, x @ w1^T) in one launch for decode row counts -- wq_a(x) and wkv(x) of
    attention.py:114/:116 -- each weight read in place; every output equals linear_rows on its
    own weight with the same ranges (linear_rows_splits over the stacked width by default, at
    least 2)."""
    name = "dsv41_linear_rows_pair"
    k, rows = _linear_args(name, x, w0, w1)
    n0, n1 = w0.shape[0], w1.shape[0]
    if splits is None:
        splits = max(linear_rows_splits(k, n0 + n1, rows), 2)
    out0 = _out(name, out0, (*x.shape[:-1], n0), torch.bfloat16, x.device)
    out1 = _out(name, out1, (*x.shape[:-1], n1), torch.bfloat16, x.device)
    need = lib().dsv41_linear_rows_workspace_bytes(rows, n0 + n1, splits)
    ws = _ws(name, workspace, need, x.device)
    _call(name, _ptr(x), _ptr(w0), _ptr(w1), _ptr(out0), _ptr(out1), _ptr(ws) if ws is not None else None, need,
          rows, k, n0, n1, splits, dtype_code(x, name), _stream(x))
    return out0, out1


def comp_write_fp4(latents, comp_kv4, g0, ratio, cos, sin, rd):
    """comp_write into a packed fp4 cache: comp_kv4 uint8 [b, >=g0+g, d/2 + d/16], per row the
    e2m1 codes of fake_quant_fp4_e4m3(rope(latent), 16) (channel 2p in the low nibble of byte p)
    and then one e4m3 scale byte per 16 channels. Decoding e2m1(code) * scale gives exactly the
    values comp_write stores."""
    name = "dsv41_comp_write_fp4"
    _gpu(name, latents, comp_kv4, cos, sin)
    _contig(name, latents)
    _tables(name, cos, sin, rd)
    b, g, d = latents.shape
    if (comp_kv4.dtype != torch.uint8 or comp_kv4.dim() != 3 or comp_kv4.shape[2] != fp4_row_bytes(d)
            or comp_kv4.shape[1] < g0 + g):
        raise ValueError(f"{name}: packed cache {tuple(comp_kv4.shape)} {comp_kv4.dtype} cannot take "
                         f"groups {g0}..{g0 + g} of {d} channels")
    _batch(name, "the compressed cache", comp_kv4, b)
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(latents), _ptr(comp_kv4), row_stride(comp_kv4, name), _ptr(cos), _ptr(sin), b, g, d, rd, g0,
          ratio, dtype_code(latents, name), _stream(latents))


def index_key_publish_fp8(k_raw, codes, scales, g0, ratio, norm_w, cos, sin, rd, eps, scale_rb=1):
    """index_key_publish into an fp8 index cache (layout of comp_write_fp8), values
    fq_fp8_ue8m0(rope(k_norm(k_raw)))."""
    name = "dsv41_index_key_publish_fp8"
    _gpu(name, k_raw, codes, scales, norm_w, cos, sin)
    _contig(name, k_raw)
    _tables(name, cos, sin, rd)
    b, g, d = _fp8_rows(name, k_raw, codes, scales, g0, scale_rb)
    _vec(name, "k_norm weight", norm_w, d)
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(k_raw), _ptr(codes), row_stride(codes, name), _ptr(scales), row_stride(scales, name), scale_rb,
          _ptr(norm_w), _ptr(cos), _ptr(sin), b, g, d, rd, g0, ratio, float(eps), dtype_code(k_raw, name),
          _stream(k_raw))


def index_key_publish_mxfp4(k_raw, k_codes, k_scales, g0, ratio, norm_w, cos, sin, rd, eps):
    """index_key_publish into an MXFP4 index cache: k_codes uint8 [b, >=g0+g, d/2] e2m1 codes,
    k_scales uint8 [b, >=g0+g, d/32] ue8m0 exponents."""
    name = "dsv41_index_key_publish_mxfp4"
    _gpu(name, k_raw, k_codes, k_scales, norm_w, cos, sin)
    _contig(name, k_raw)
    _tables(name, cos, sin, rd)
    b, g, d = k_raw.shape
    _vec(name, "k_norm weight", norm_w, d)
    if k_codes.dtype != torch.uint8 or k_codes.shape[0] < b or k_codes.shape[2] != d // 2 or k_codes.shape[1] < g0 + g:
        raise ValueError(f"{name}: code cache {tuple(k_codes.shape)} cannot take groups {g0}..{g0 + g}")
    if k_scales.dtype != torch.uint8 or k_scales.shape[0] < b or k_scales.shape[2] != d // 32 or k_scales.shape[1] < g0 + g:
        raise ValueError(f"{name}: scale cache {tuple(k_scales.shape)} cannot take groups {g0}..{g0 + g}")
    if g and (g0 + g - 1) * ratio >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(k_raw), _ptr(k_codes), row_stride(k_codes, name), _ptr(k_scales), row_stride(k_scales, name),
          _ptr(norm_w), _ptr(cos), _ptr(sin), b, g, d, rd, g0, ratio, float(eps), dtype_code(k_raw, name),
          _stream(k_raw))


# ---------------------------------------------------------------------------- indexer


def index_q_prep(q, cos, sin, rd, start_pos):
    name = "dsv41_index_q_prep"
    _gpu(name, q, cos, sin)
    _contig(name, q)
    _tables(name, cos, sin, rd)
    b, n, h, d = q.shape
    if n and start_pos + n - 1 >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    _call(name, _ptr(q), _ptr(cos), _ptr(sin), b, n, h, d, rd, start_pos, dtype_code(q, name),
          _stream(q))
    return q


def indexer_score(q, w_raw, w_scale, index_k, start_pos, ratio, candidates=None, out=None):
    """q [b,n,h,d], w_raw [b,n,h], index_k view [b, nb, d] of the owner's cache."""
    name = "dsv41_indexer_score"
    _gpu(name, q, w_raw, index_k, candidates, out)
    _contig(name, q, w_raw, candidates)
    b, n, h, d = q.shape
    nb = index_k.shape[1]
    if w_raw.shape != (b, n, h) or w_raw.dtype != q.dtype:
        raise ValueError(f"{name}: w_raw must be {q.dtype} [{b}, {n}, {h}]")
    if index_k.shape[0] < b or index_k.shape[2] != d or index_k.dtype != q.dtype:
        raise ValueError(f"{name}: index_k {tuple(index_k.shape)} {index_k.dtype} does not match q")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    out = _out(name, out, (b, n, nb), torch.float32, q.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q), _ptr(w_raw), float(w_scale), _ptr(index_k), row_stride(index_k, name),
          _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio, dtype_code(q, name), _stream(q))
    return out


def indexer_topk_workspace_bytes(b, n, heads, dim, nb, topk, has_candidates=False) -> int:
    return int(lib().dsv41_indexer_topk_workspace_bytes(b, n, heads, dim, nb, topk, 1 if has_candidates else 0))


def indexer_topk(q, w_raw, w_scale, index_k, start_pos, ratio, topk, offset, candidates=None, out=None,
                 workspace=None):
    """indexer_score followed by topk_select in one fused decode form: int32 [b, n, min(topk, nb)],
    bit-equal to topk_select(indexer_score(...)) -- but the [b, n, nb] scores are never written:
    each row range keeps its best topk and a merge selects from those lists. Returns None when
    the shape is not one the fused form serves (the caller then makes the two calls)."""
    name = "dsv41_indexer_topk"
    _gpu(name, q, w_raw, index_k, candidates, out, workspace)
    _contig(name, q, w_raw, candidates)
    b, n, h, d = q.shape
    nb = index_k.shape[1]
    if q.dtype != torch.bfloat16 or w_raw.shape != (b, n, h) or w_raw.dtype != q.dtype:
        raise ValueError(f"{name}: q and w_raw must be bf16, w_raw [{b}, {n}, {h}]")
    if index_k.shape[0] < b or index_k.shape[2] != d or index_k.dtype != q.dtype:
        raise ValueError(f"{name}: index_k {tuple(index_k.shape)} {index_k.dtype} does not match q")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    ws_bytes = indexer_topk_workspace_bytes(b, n, h, d, nb, topk, candidates is not None)
    if ws_bytes == 0:
        return None
    k = min(topk, nb)
    out = _out(name, out, (b, n, k), torch.int32, q.device)
    ws = _ws(name, workspace, ws_bytes, q.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q), _ptr(w_raw), float(w_scale), _ptr(index_k), row_stride(index_k, name), _ptr(cand),
          _ptr(out), b, n, h, d, nb, start_pos, ratio, topk, offset, _ptr(ws), ws_bytes, _stream(q))
    return out


def indexer_score_fp8(q, w_raw, w_scale, index_k8, k_scale, scale_rb, nb, start_pos, ratio, candidates=None,
                      out=None):
    """indexer_score with fp8 keys: index_k8 uint8 [b, >=nb, 128] e4m3fn codes, k_scale uint8
    [b, >=ceil(nb / scale_rb), 4] ue8m0 exponents (one per 32 channels, every scale_rb = 1 or 32
    rows). q [b,n,h,128] and w_raw [b,n,h] bf16."""
    name = "dsv41_indexer_score_fp8"
    _gpu(name, q, w_raw, index_k8, k_scale, candidates, out)
    _contig(name, q, w_raw, candidates)
    b, n, h, d = q.shape
    if q.dtype != torch.bfloat16 or d != 128:
        raise ValueError(f"{name}: q must be bf16 with 128 channels")
    if w_raw.shape != (b, n, h) or w_raw.dtype != q.dtype:
        raise ValueError(f"{name}: w_raw must be {q.dtype} [{b}, {n}, {h}]")
    if index_k8.dtype != torch.uint8 or index_k8.shape[0] < b or index_k8.shape[2] != d or index_k8.shape[1] < nb:
        raise ValueError(f"{name}: fp8 keys {tuple(index_k8.shape)} {index_k8.dtype} do not match")
    if (k_scale.dtype != torch.uint8 or k_scale.shape[0] < b or k_scale.shape[2] != d // 32
            or k_scale.shape[1] < -(-nb // scale_rb)):
        raise ValueError(f"{name}: key scales {tuple(k_scale.shape)} do not match")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    out = _out(name, out, (b, n, nb), torch.float32, q.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q), _ptr(w_raw), float(w_scale), _ptr(index_k8), row_stride(index_k8, name), _ptr(k_scale),
          row_stride(k_scale, name), scale_rb, _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio, _stream(q))
    return out


def indexer_topk_fp8(q, w_raw, w_scale, index_k8, k_scale, scale_rb, nb, start_pos, ratio, topk, offset,
                     candidates=None, out=None, workspace=None):
    """indexer_topk over fp8 keys (the layouts of indexer_score_fp8): int32 [b, n, min(topk, nb)],
    bit-equal to topk_select(indexer_score_fp8(...)). Returns None when the fused form does not
    serve the shape or the layout (scales and both strides 16-byte aligned)."""
    name = "dsv41_indexer_topk_fp8"
    _gpu(name, q, w_raw, index_k8, k_scale, candidates, out, workspace)
    _contig(name, q, w_raw, candidates)
    b, n, h, d = q.shape
    if q.dtype != torch.bfloat16 or d != 128 or w_raw.shape != (b, n, h) or w_raw.dtype != q.dtype:
        raise ValueError(f"{name}: q must be bf16 [b, n, h, 128] and w_raw bf16 [{b}, {n}, {h}]")
    if index_k8.dtype != torch.uint8 or index_k8.shape[0] < b or index_k8.shape[2] != d or index_k8.shape[1] < nb:
        raise ValueError(f"{name}: fp8 keys {tuple(index_k8.shape)} {index_k8.dtype} do not match")
    if (k_scale.dtype != torch.uint8 or k_scale.shape[0] < b or k_scale.shape[2] != d // 32
            or k_scale.shape[1] < -(-nb // scale_rb)):
        raise ValueError(f"{name}: key scales {tuple(k_scale.shape)} do not match")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    ks_stride = row_stride(k_scale, name)
    ws_bytes = indexer_topk_workspace_bytes(b, n, h, d, nb, topk, candidates is not None)
    if ws_bytes == 0 or k_scale.data_ptr() % 16 or ks_stride % 16 or index_k8.data_ptr() % 16:
        return None
    k = min(topk, nb)
    out = _out(name, out, (b, n, k), torch.int32, q.device)
    ws = _ws(name, workspace, ws_bytes, q.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q), _ptr(w_raw), float(w_scale), _ptr(index_k8), row_stride(index_k8, name), _ptr(k_scale),
          ks_stride, scale_rb, _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio, topk, offset, _ptr(ws),
          ws_bytes, _stream(q))
    return out


def index_q_prep_mxfp4(q, cos, sin, rd, start_pos, out=None):
    """index_q_prep into MXFP4 form: q [b,n,h,d] (read only) -> (codes uint8 [b,n,h,d/2],
    scales uint8 [b,n,h,d/32]) of fake_quant_fp4_ue8m0(rope_tail(q))."""
    name = "dsv41_index_q_prep_mxfp4"
    _gpu(name, q, cos, sin)
    _contig(name, q)
    _tables(name, cos, sin, rd)
    b, n, h, d = q.shape
    if d % 32:
        raise ValueError(f"{name}: {d} channels is not a whole number of 32-channel blocks")
    if n and start_pos + n - 1 >= cos.shape[0]:
        raise ValueError(f"{name}: rope table too short")
    codes, scales = out if out is not None else (None, None)
    codes = _out(name, codes, (b, n, h, d // 2), torch.uint8, q.device)
    scales = _out(name, scales, (b, n, h, d // 32), torch.uint8, q.device)
    _call(name, _ptr(q), _ptr(codes), _ptr(scales), _ptr(cos), _ptr(sin), b, n, h, d, rd, start_pos,
          dtype_code(q, name), _stream(q))
    return codes, scales


def indexer_score_mxfp4(q_mx, w_raw, w_scale, k_codes, k_scales, nb, start_pos, ratio, candidates=None, out=None):
    """indexer_score with query and keys in MXFP4 form: q_mx = (codes uint8 [b,n,h,64], scales
    uint8 [b,n,h,4]) from index_q_prep_mxfp4; k_codes uint8 [b, >=nb, 64], k_scales uint8
    [b, >=nb, 4]; w_raw [b,n,h] bf16."""
    name = "dsv41_indexer_score_mxfp4"
    q_codes, q_scales = q_mx
    _gpu(name, q_codes, q_scales, w_raw, k_codes, k_scales, candidates, out)
    _contig(name, q_codes, q_scales, w_raw, candidates)
    b, n, h, d2 = q_codes.shape
    d = d2 * 2
    if q_codes.dtype != torch.uint8 or d != 128 or q_scales.shape != (b, n, h, d // 32) or q_scales.dtype != torch.uint8:
        raise ValueError(f"{name}: query must be uint8 codes [b, n, h, 64] with scales [b, n, h, 4]")
    if w_raw.shape != (b, n, h) or w_raw.dtype != torch.bfloat16:
        raise ValueError(f"{name}: w_raw must be bf16 [{b}, {n}, {h}]")
    if k_codes.dtype != torch.uint8 or k_codes.shape[0] < b or k_codes.shape[2] != d // 2 or k_codes.shape[1] < nb:
        raise ValueError(f"{name}: key codes {tuple(k_codes.shape)} {k_codes.dtype} do not match")
    if k_scales.dtype != torch.uint8 or k_scales.shape[0] < b or k_scales.shape[2] != d // 32 or k_scales.shape[1] < nb:
        raise ValueError(f"{name}: key scales {tuple(k_scales.shape)} do not match")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    out = _out(name, out, (b, n, nb), torch.float32, w_raw.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q_codes), _ptr(q_scales), _ptr(w_raw), float(w_scale), _ptr(k_codes), row_stride(k_codes, name),
          _ptr(k_scales), row_stride(k_scales, name), _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio,
          _stream(w_raw))
    return out


def indexer_topk_mxfp4(q_mx, w_raw, w_scale, k_codes, k_scales, nb, start_pos, ratio, topk, offset, candidates=None,
                       out=None, workspace=None):
    """indexer_topk over MXFP4 query and keys (the layouts of indexer_score_mxfp4): int32
    [b, n, min(topk, nb)], bit-equal to topk_select(indexer_score_mxfp4(...)). Returns None when
    the fused form does not serve the shape."""
    name = "dsv41_indexer_topk_mxfp4"
    q_codes, q_scales = q_mx
    _gpu(name, q_codes, q_scales, w_raw, k_codes, k_scales, candidates, out, workspace)
    _contig(name, q_codes, q_scales, w_raw, candidates)
    b, n, h, d2 = q_codes.shape
    d = d2 * 2
    if q_codes.dtype != torch.uint8 or d != 128 or q_scales.shape != (b, n, h, d // 32) or q_scales.dtype != torch.uint8:
        raise ValueError(f"{name}: query must be uint8 codes [b, n, h, 64] with scales [b, n, h, 4]")
    if w_raw.shape != (b, n, h) or w_raw.dtype != torch.bfloat16:
        raise ValueError(f"{name}: w_raw must be bf16 [{b}, {n}, {h}]")
    if k_codes.dtype != torch.uint8 or k_codes.shape[0] < b or k_codes.shape[2] != d // 2 or k_codes.shape[1] < nb:
        raise ValueError(f"{name}: key codes {tuple(k_codes.shape)} {k_codes.dtype} do not match")
    if k_scales.dtype != torch.uint8 or k_scales.shape[0] < b or k_scales.shape[2] != d // 32 or k_scales.shape[1] < nb:
        raise ValueError(f"{name}: key scales {tuple(k_scales.shape)} do not match")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    ws_bytes = indexer_topk_workspace_bytes(b, n, h, d, nb, topk, candidates is not None)
    if ws_bytes == 0:
        return None
    k = min(topk, nb)
    out = _out(name, out, (b, n, k), torch.int32, w_raw.device)
    ws = _ws(name, workspace, ws_bytes, w_raw.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q_codes), _ptr(q_scales), _ptr(w_raw), float(w_scale), _ptr(k_codes), row_stride(k_codes, name),
          _ptr(k_scales), row_stride(k_scales, name), _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio, topk,
          offset, _ptr(ws), ws_bytes, _stream(w_raw))
    return out


def _mxq_fp8_check(name, q_mx, w_raw, k_codes, k_scales, scale_rb, nb, candidates):
    q_codes, q_scales = q_mx
    _gpu(name, q_codes, q_scales, w_raw, k_codes, k_scales, candidates)
    _contig(name, q_codes, q_scales, w_raw, candidates)
    b, n, h, d2 = q_codes.shape
    d = d2 * 2
    if q_codes.dtype != torch.uint8 or d != 128 or q_scales.shape != (b, n, h, d // 32) or q_scales.dtype != torch.uint8:
        raise ValueError(f"{name}: query must be uint8 codes [b, n, h, 64] with scales [b, n, h, 4]")
    if w_raw.shape != (b, n, h) or w_raw.dtype != torch.bfloat16:
        raise ValueError(f"{name}: w_raw must be bf16 [{b}, {n}, {h}]")
    if scale_rb not in (1, 32):
        raise ValueError(f"{name}: scale_rb must be 1 or 32, got {scale_rb}")
    if k_codes.dtype != torch.uint8 or k_codes.shape[0] < b or k_codes.shape[2] != d or k_codes.shape[1] < nb:
        raise ValueError(f"{name}: fp8 keys {tuple(k_codes.shape)} {k_codes.dtype} do not match")
    if (k_scales.dtype != torch.uint8 or k_scales.shape[0] < b or k_scales.shape[2] != d // 32
            or k_scales.shape[1] < -(-nb // scale_rb)):
        raise ValueError(f"{name}: key scales {tuple(k_scales.shape)} do not match")
    if candidates is not None and (candidates.shape != (b, n, nb) or candidates.dtype not in (torch.uint8, torch.bool)):
        raise ValueError(f"{name}: candidates must be bool/uint8 [{b}, {n}, {nb}]")
    return q_codes, q_scales, b, n, h, d


def indexer_score_mxq_fp8(q_mx, w_raw, w_scale, k_codes, k_scales, scale_rb, nb, start_pos, ratio, candidates=None,
                          out=None):
    """indexer_score with the query in MXFP4 form (codes uint8 [b,n,h,64], scales uint8 [b,n,h,4])
    against fp8 keys: k_codes uint8 [b, >=nb, 128] e4m3fn, k_scales uint8 [b, >=ceil(nb/scale_rb), 4]
    ue8m0 (one per 32 channels of every scale_rb = 1 or 32 rows); block-scaled fp4 x fp8 MFMA."""
    name = "dsv41_indexer_score_mxq_fp8"
    q_codes, q_scales, b, n, h, d = _mxq_fp8_check(name, q_mx, w_raw, k_codes, k_scales, scale_rb, nb, candidates)
    out = _out(name, out, (b, n, nb), torch.float32, w_raw.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q_codes), _ptr(q_scales), _ptr(w_raw), float(w_scale), _ptr(k_codes), row_stride(k_codes, name),
          _ptr(k_scales), row_stride(k_scales, name), scale_rb, _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio,
          _stream(w_raw))
    return out


def indexer_topk_mxq_fp8(q_mx, w_raw, w_scale, k_codes, k_scales, scale_rb, nb, start_pos, ratio, topk, offset,
                         candidates=None, out=None, workspace=None):
    """indexer_topk over an MXFP4 query and fp8 keys (the layouts of indexer_score_mxq_fp8): int32
    [b, n, min(topk, nb)], bit-equal to topk_select(indexer_score_mxq_fp8(...)). Returns None when
    the fused form does not serve the shape."""
    name = "dsv41_indexer_topk_mxq_fp8"
    q_codes, q_scales, b, n, h, d = _mxq_fp8_check(name, q_mx, w_raw, k_codes, k_scales, scale_rb, nb, candidates)
    _gpu(name, out, workspace)
    ws_bytes = indexer_topk_workspace_bytes(b, n, h, d, nb, topk, candidates is not None)
    if ws_bytes == 0:
        return None
    k = min(topk, nb)
    out = _out(name, out, (b, n, k), torch.int32, w_raw.device)
    ws = _ws(name, workspace, ws_bytes, w_raw.device)
    cand = candidates.view(torch.uint8) if candidates is not None else None
    _call(name, _ptr(q_codes), _ptr(q_scales), _ptr(w_raw), float(w_scale), _ptr(k_codes), row_stride(k_codes, name),
          _ptr(k_scales), row_stride(k_scales, name), scale_rb, _ptr(cand), _ptr(out), b, n, h, d, nb, start_pos, ratio,
          topk, offset, _ptr(ws), ws_bytes, _stream(w_raw))
    return out


def topk_workspace_bytes(rows, nb, topk) -> int:
    return int(lib().dsv41_topk_workspace_bytes(rows, nb, topk))


def topk_select(scores, topk, start_pos, ratio, offset, workspace=None, out=None):
    """scores [b, n, nb] fp32 -> int32 [b, n, min(topk, nb)] (into `out` when given). Rows longer
    than 16384 scores (k <= 2048) are selected in two stages through a uint8 workspace of
    topk_workspace_bytes(...) bytes, allocated when it is omitted or too small."""
    name = "dsv41_topk_select_ws"
    _gpu(name, scores, workspace, out)
    _contig(name, scores)
    if scores.dtype != torch.float32 or scores.dim() != 3:
        raise ValueError(f"{name}: scores must be fp32 [b, n, nb]")
    b, n, nb = scores.shape
    k = min(topk, nb)
    out = _out(name, out, (b, n, k), torch.int32, scores.device)
    if out.numel():
        ws_bytes = topk_workspace_bytes(b * n, nb, topk)
        ws = _ws(name, workspace, ws_bytes, scores.device)
        _call(name, _ptr(scores), _ptr(out), b * n, n, nb, topk, start_pos, ratio, offset, _ptr(ws),
              ws_bytes, _stream(scores))
    return out


def candidate_blocks(scores, topk_blocks, block_size, lens=None, start_pos=0, ratio=1):
    """scores [b, n, nb] fp32 -> bool [b, n, nb]; lens optional int32 [n] on the GPU."""
    name = "dsv41_candidate_blocks"
    _gpu(name, scores, lens)
    _contig(name, scores, lens)
    if scores.dtype != torch.float32 or scores.dim() != 3:
        raise ValueError(f"{name}: scores must be fp32 [b, n, nb]")
    b, n, nb = scores.shape
    if lens is not None and (lens.dtype != torch.int32 or lens.numel() != n):
        raise ValueError(f"{name}: lens must be int32 [{n}]")
    keep = torch.empty(b, n, nb, dtype=torch.uint8, device=scores.device)
    if keep.numel():
        _call(name, _ptr(scores), _ptr(keep), b * n, n, nb, topk_blocks, block_size, _ptr(lens),
              start_pos, ratio, _stream(scores))
    return keep.view(torch.bool)


# ---------------------------------------------------------------------------- sparse MLA


def mla_workspace_bytes(b, m, heads, dim, rows_per_query, dtype) -> int:
    return int(lib().dsv41_sparse_mla_workspace_bytes(b, m, heads, dim, rows_per_query,
                                                      _DTYPES.get(dtype, -1)))


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale):
    name = "dsv41_sparse_attn"
    _gpu(name, q, kv, attn_sink, topk_idxs)
    _contig(name, q, kv, attn_sink, topk_idxs)
    b, m, h, d = q.shape
    if kv.dim() != 3 or kv.shape[0] != b or kv.shape[2] != d or kv.dtype != q.dtype:
        raise ValueError(f"{name}: kv {tuple(kv.shape)} {kv.dtype} does not match q")
    if topk_idxs.dtype != torch.int32 or topk_idxs.shape[:2] != (b, m):
        raise ValueError(f"{name}: topk_idxs must be int32 [{b}, {m}, k]")
    if attn_sink.dtype != torch.float32 or attn_sink.numel() != h:
        raise ValueError(f"{name}: attn_sink must be fp32 [{h}]")
    k = topk_idxs.shape[2]
    o = torch.empty_like(q)
    ws_bytes = mla_workspace_bytes(b, m, h, d, k, q.dtype)
    ws = _workspace(ws_bytes, q.device)
    _call(name, _ptr(q), _ptr(kv), _ptr(attn_sink), _ptr(topk_idxs), _ptr(o), b, m, h, d,
          kv.shape[1], k, float(softmax_scale), dtype_code(q, name), _ptr(ws), ws_bytes, _stream(q))
    return o


def sparse_mla(q, win_kv, chunk_kv, comp_kv, n_comp, attn_sink, idx, softmax_scale, window,
               start_pos, cos=None, sin=None, rd=0, out=None, workspace=None, write_ring=False, q_rd=0):
    """The layer form: window ring + this chunk's KV + the owner's compressed cache, all read
    in place. comp_kv: [b, >=n_comp, d] view (or None); idx [b, n, k] int32 or None.
    workspace: a uint8 scratch tensor of at least mla_workspace_bytes(...) bytes, allocated
    when it is omitted or too small. write_ring (one token per row): the same launch also
    stores chunk_kv into its ring slot, as LayerCache.write_window would afterwards.
    rd: width of the inverse rope on the output; q_rd > 0: q is given before its rope and the
    launch applies rope_tail(q, q_rd, cos, sin) at positions start_pos + s as it loads q."""
    name = "dsv41_sparse_mla_decode" if write_ring else "dsv41_sparse_mla"
    _gpu(name, q, win_kv, chunk_kv, comp_kv, attn_sink, idx, cos, sin, out)
    _contig(name, q, chunk_kv, attn_sink, idx)
    b, n, h, d = q.shape
    _vec(name, "attn_sink", attn_sink, h)
    wp = min(start_pos, window)
    if chunk_kv.shape != (b, n, d) or chunk_kv.dtype != q.dtype:
        raise ValueError(f"{name}: chunk kv must be {q.dtype} [{b}, {n}, {d}]")
    ring = None
    if win_kv is not None:
        if win_kv.shape[0] < b or win_kv.shape[1:] != (window, d) or win_kv.dtype != q.dtype:
            raise ValueError(f"{name}: window ring {tuple(win_kv.shape)} does not match")
        ring = win_kv[:b]
        _contig(name, ring)
    elif wp:
        raise ValueError(f"{name}: a window ring is needed once start_pos > 0")
    comp_bstride = 0
    if comp_kv is not None and n_comp:
        if (comp_kv.dim() != 3 or comp_kv.dtype != q.dtype or comp_kv.shape[2] != d
                or comp_kv.shape[1] < n_comp):
            raise ValueError(f"{name}: compressed cache {tuple(comp_kv.shape)} does not match")
        _batch(name, "the compressed cache", comp_kv, b)
        comp_bstride = row_stride(comp_kv, name)
    else:
        comp_kv, n_comp = None, 0
    k = 0
    if idx is not None:
        if idx.dtype != torch.int32 or idx.shape[:2] != (b, n):
            raise ValueError(f"{name}: idx must be int32 [{b}, {n}, k]")
        k = idx.shape[2]
    _attn_tables(name, cos, sin, rd, q_rd, start_pos, n)
    o = _out(name, out, q.shape, q.dtype, q.device)
    rows = min(window, wp + n) + k
    ws_bytes = mla_workspace_bytes(b, n, h, d, rows, q.dtype)
    workspace = _ws(name, workspace, ws_bytes, q.device)
    tail = (_ptr(cos) if rd or q_rd else None, _ptr(sin) if rd or q_rd else None, rd, q_rd, dtype_code(q, name),
            _ptr(workspace) if ws_bytes else None, ws_bytes, _stream(q))
    if write_ring:
        if n != 1 or ring is None:
            raise ValueError(f"{name}: the ring store needs one token per row and a window ring")
        _call(name, _ptr(q), _ptr(ring), _ptr(chunk_kv), _ptr(comp_kv), comp_bstride, n_comp, _ptr(attn_sink),
              _ptr(idx), k, _ptr(o), b, h, d, window, start_pos, float(softmax_scale), *tail)
    else:
        _call(name, _ptr(q), _ptr(ring), _ptr(chunk_kv), _ptr(comp_kv), comp_bstride, n_comp, _ptr(attn_sink),
              _ptr(idx), k, _ptr(o), b, n, h, d, window, start_pos, float(softmax_scale), *tail)
    return o


def _packed_mla_sources(name, q, win_kv, chunk_kv, attn_sink, idx, window, start_pos, cos, sin, rd, q_rd,
                        write_ring, ring_mxfp8=False):
    """Checks shared by the packed-cache sparse_mla forms (bf16 q and chunk, a bf16 or MXFP8
    ring; 512 channels): returns (b, n, h, d, ring view, k)."""
    _contig(name, q, chunk_kv, attn_sink, idx)
    b, n, h, d = q.shape
    if q.dtype != torch.bfloat16 or d != 512:
        raise ValueError(f"{name}: q must be bf16 with 512 channels")
    _vec(name, "attn_sink", attn_sink, h)
    wp = min(start_pos, window)
    if chunk_kv.shape != (b, n, d) or chunk_kv.dtype != q.dtype:
        raise ValueError(f"{name}: chunk kv must be {q.dtype} [{b}, {n}, {d}]")
    ring = None
    row, rdt = (mxfp8_row_bytes(d), torch.uint8) if ring_mxfp8 else (d, q.dtype)
    if win_kv is not None:
        if win_kv.dim() != 3 or win_kv.shape[0] < b or win_kv.shape[1:] != (window, row) or win_kv.dtype != rdt:
            raise ValueError(f"{name}: window ring {tuple(win_kv.shape)} {win_kv.dtype} does not match")
        ring = win_kv[:b]
        _contig(name, ring)
    elif wp:
        raise ValueError(f"{name}: a window ring is needed once start_pos > 0")
    k = 0
    if idx is not None:
        if idx.dtype != torch.int32 or idx.shape[:2] != (b, n):
            raise ValueError(f"{name}: idx must be int32 [{b}, {n}, k]")
        k = idx.shape[2]
    _attn_tables(name, cos, sin, rd, q_rd, start_pos, n)
    if write_ring and (n != 1 or ring is None):
        raise ValueError(f"{name}: the ring store needs one token per row and a window ring")
    return b, n, h, d, ring, k


def sparse_mla_fp4(q, win_kv, chunk_kv, comp_kv4, n_comp, attn_sink, idx, softmax_scale, window, start_pos,
                   cos=None, sin=None, rd=0, out=None, workspace=None, write_ring=False, q_rd=0):
    """sparse_mla with a packed fp4 compressed cache (comp_write_fp4's layout): comp_kv4 uint8
    [b, >=n_comp, 288] rows of 512 e2m1 codes and 32 e4m3 scales. q, the window ring, chunk and
    output are bf16; the result equals sparse_mla's on the decoded cache.
    write_ring (one token per row): the launch also stores chunk_kv into its ring slot."""
    name = "dsv41_sparse_mla_fp4_decode" if write_ring else "dsv41_sparse_mla_fp4"
    return _sparse_mla_fp4_rows(name, q, win_kv, chunk_kv, comp_kv4, n_comp, attn_sink, idx, softmax_scale, window,
                                start_pos, cos, sin, rd, q_rd, out, workspace, write_ring, False)


def sparse_mla_packed(q, win_kv8, chunk_kv, comp_kv4, n_comp, attn_sink, idx, softmax_scale, window, start_pos,
                      cos=None, sin=None, rd=0, out=None, workspace=None, write_ring=False, q_rd=0):
    """sparse_mla over the packed cache: the window ring as MXFP8 rows (win_kv8 uint8
    [b, window, 528]: 512 e4m3fn codes, 16 ue8m0 scales; window_write_mxfp8's layout) and the
    compressed KV as packed fp4 rows (comp_kv4, or None for a window-only layer). q, chunk and
    output are bf16; the result equals sparse_mla's on the decoded caches. write_ring (one token
    per row): the launch also stores chunk_kv, MXFP8-encoded, into its ring slot."""
    name = "dsv41_sparse_mla_packed_decode" if write_ring else "dsv41_sparse_mla_packed"
    return _sparse_mla_fp4_rows(name, q, win_kv8, chunk_kv, comp_kv4, n_comp, attn_sink, idx, softmax_scale, window,
                                start_pos, cos, sin, rd, q_rd, out, workspace, write_ring, True)


def _sparse_mla_fp4_rows(name, q, win_kv, chunk_kv, comp_kv4, n_comp, attn_sink, idx, softmax_scale, window,
                         start_pos, cos, sin, rd, q_rd, out, workspace, write_ring, ring_mxfp8):
    _gpu(name, q, win_kv, chunk_kv, comp_kv4, attn_sink, idx, cos, sin, out)
    b, n, h, d, ring, k = _packed_mla_sources(name, q, win_kv, chunk_kv, attn_sink, idx, window, start_pos, cos,
                                              sin, rd, q_rd, write_ring, ring_mxfp8)
    comp_bstride = 0
    if comp_kv4 is not None and n_comp:
        if (comp_kv4.dtype != torch.uint8 or comp_kv4.dim() != 3 or comp_kv4.shape[2] != fp4_row_bytes(d)
                or comp_kv4.shape[1] < n_comp):
            raise ValueError(f"{name}: packed fp4 cache {tuple(comp_kv4.shape)} {comp_kv4.dtype} does not match")
        _batch(name, "the compressed cache", comp_kv4, b)
        comp_bstride = row_stride(comp_kv4, name)
    else:
        comp_kv4, n_comp = None, 0
    o = _out(name, out, q.shape, q.dtype, q.device)
    wp = min(start_pos, window)
    ws_bytes = mla_workspace_bytes(b, n, h, d, min(window, wp + n) + k, q.dtype)
    workspace = _ws(name, workspace, ws_bytes, q.device)
    tail = (_ptr(cos) if rd or q_rd else None, _ptr(sin) if rd or q_rd else None, rd, q_rd,
            _ptr(workspace) if ws_bytes else None, ws_bytes, _stream(q))
    if ring_mxfp8:
        if ring is None:
            raise ValueError(f"{name}: the MXFP8 ring is required")
        ring_part = (_ptr(ring), row_stride(ring, name))
    else:
        ring_part = (_ptr(ring),)
    head = (_ptr(q), *ring_part, _ptr(chunk_kv), _ptr(comp_kv4), comp_bstride, n_comp, _ptr(attn_sink), _ptr(idx),
            k, _ptr(o), b)
    if write_ring:
        _call(name, *head, h, d, window, start_pos, float(softmax_scale), *tail)
    else:
        _call(name, *head, n, h, d, window, start_pos, float(softmax_scale), *tail)
    return o


def sparse_mla_fp8(q, win_kv, chunk_kv, comp8, comp_scale, scale_rb, n_comp, attn_sink, idx, softmax_scale,
                   window, start_pos, cos=None, sin=None, rd=0, out=None, workspace=None, write_ring=False, q_rd=0):
    """sparse_mla with an fp8 compressed cache: comp8 uint8 [b, >=n_comp, 512] e4m3fn codes,
    comp_scale uint8 [b, >=ceil(n_comp / scale_rb), 16] ue8m0 exponents (one per 32 channels
    for every scale_rb = 1 or 32 rows). q, the window ring, chunk and output are bf16.
    write_ring (one token per row): the launch also stores chunk_kv into its ring slot."""
    name = "dsv41_sparse_mla_fp8_decode" if write_ring else "dsv41_sparse_mla_fp8"
    _gpu(name, q, win_kv, chunk_kv, comp8, comp_scale, attn_sink, idx, cos, sin, out)
    b, n, h, d, ring, k = _packed_mla_sources(name, q, win_kv, chunk_kv, attn_sink, idx, window, start_pos, cos,
                                              sin, rd, q_rd, write_ring)
    wp = min(start_pos, window)
    comp_bstride = sc_bstride = 0
    if comp8 is not None and n_comp:
        if comp8.dtype != torch.uint8 or comp8.shape[2] != d or comp8.shape[1] < n_comp or comp8.shape[0] < b:
            raise ValueError(f"{name}: fp8 cache {tuple(comp8.shape)} {comp8.dtype} does not match")
        nblk = -(-n_comp // scale_rb)
        if (comp_scale is None or comp_scale.dtype != torch.uint8 or comp_scale.shape[2] != d // 32
                or comp_scale.shape[1] < nblk or comp_scale.shape[0] < b):
            raise ValueError(f"{name}: scale tensor does not match the cache")
        comp_bstride = row_stride(comp8, name)
        sc_bstride = row_stride(comp_scale, name)
    else:
        comp8, comp_scale, n_comp = None, None, 0
    o = _out(name, out, q.shape, q.dtype, q.device)
    rows = min(window, wp + n) + k
    ws_bytes = mla_workspace_bytes(b, n, h, d, rows, q.dtype)
    workspace = _ws(name, workspace, ws_bytes, q.device)
    tail = (_ptr(cos) if rd or q_rd else None, _ptr(sin) if rd or q_rd else None, rd, q_rd,
            _ptr(workspace) if ws_bytes else None, ws_bytes, _stream(q))
    if write_ring:
        _call(name, _ptr(q), _ptr(ring), _ptr(chunk_kv), _ptr(comp8), comp_bstride, n_comp, _ptr(comp_scale),
              sc_bstride, scale_rb, _ptr(attn_sink), _ptr(idx), k, _ptr(o), b, h, d, window, start_pos,
              float(softmax_scale), *tail)
    else:
        _call(name, _ptr(q), _ptr(ring), _ptr(chunk_kv), _ptr(comp8), comp_bstride, n_comp, _ptr(comp_scale),
              sc_bstride, scale_rb, _ptr(attn_sink), _ptr(idx), k, _ptr(o), b, n, h, d, window, start_pos,
              float(softmax_scale), *tail)
    return o
