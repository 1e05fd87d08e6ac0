"""Drop-in for the native ``kernel`` module that DeepSeek's reference model imports
(docs/reference/model.py:12-19; its TileLang wrappers live in docs/reference/kernel.py).

The reference's own tests replace that module by ``sys.modules["kernel"] = kernel_stub``
(tests/test_parity.py:57-58); this module fills the same seam with the gfx950 kernels:

    import sys, dsv41.kernel
    sys.modules["kernel"] = dsv41.kernel

Covered (the attention path): the in-place QAT round trips of ``act_quant`` /
``fp4_act_quant`` and ``sparse_attn``. The weight GEMMs (``fp8_gemm``, ``fp4_gemm``) and the
hyper-connection Sinkhorn are outside the attention path and raise, like the reference's
test stub (tests/kernel_stub.py:127-134).
"""

from __future__ import annotations

import torch

from . import _abi


def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt=None, scale_dtype=None,
              inplace: bool = False):
    """kernel.py:98-124. Only the fused quant->dequant form with power-of-two scales
    (``scale_fmt="ue8m0"``, ``inplace=True``) is on the attention path."""
    if not inplace or scale_fmt is None:
        raise NotImplementedError("dsv41.kernel.act_quant implements the inplace ue8m0 round trip only")
    _abi.fq_fp8_ue8m0(x, block_size, out=x)
    return x


def fp4_act_quant(x: torch.Tensor, block_size: int = 32, inplace: bool = False,
                  scale_dtype=torch.float8_e8m0fnu):
    """kernel.py:184-204: e8m0 (power-of-two) scales, or e4m3 scales (compressed KV)."""
    if not inplace:
        raise NotImplementedError("dsv41.kernel.fp4_act_quant implements the inplace round trip only")
    if scale_dtype == torch.float8_e4m3fn:
        _abi.fq_fp4_e4m3(x, block_size, out=x)
    else:
        _abi.fq_fp4_ue8m0(x, block_size, out=x)
    return x


def sparse_attn(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor,
                softmax_scale: float) -> torch.Tensor:
    """kernel.py:392-403 (no head padding needed: partial head tiles are masked in-kernel)."""
    return _abi.sparse_attn(q.contiguous(), kv.contiguous(), attn_sink.float().contiguous(),
                            topk_idxs.to(torch.int32).contiguous(), softmax_scale)


def _outside_path(name):
    def f(*args, **kwargs):
        raise RuntimeError(f"{name} is outside the attention path; dsv41 does not implement it")
    return f


fp8_gemm = _outside_path("fp8_gemm")
fp4_gemm = _outside_path("fp4_gemm")
hc_split_sinkhorn = _outside_path("hc_split_sinkhorn")
