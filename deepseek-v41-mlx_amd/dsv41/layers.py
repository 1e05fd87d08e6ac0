"""RMSNorm and YaRN rope on the GPU (deepseek_v41_mlx/layers.py:20-84).

* ``RMSNorm`` computes in fp32 and returns the input dtype; eps is 1e-20 in the release.
* Rope pairs *adjacent* channels (real, imag) and acts on the last ``rope_head_dim``
  channels only; ``inverse=True`` conjugates (used on the attention output).
* ``precompute_freqs_cis`` returns device (cos, sin) tables ``[seqlen, rd/2]`` fp32: the
  YaRN-ramped inverse frequencies are configuration (rd/2 numbers, computed here in fp32
  exactly as the reference's formula does), the table itself is built by a HIP kernel.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _abi


class RMSNorm(torch.nn.Module):
    def __init__(self, dim: int, eps: float = 1e-20, device=None):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim, dtype=torch.float32, device=device),
                                         requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _abi.rmsnorm(x.contiguous(), self.weight, self.eps)


# Decode row counts (at most 128 rows of bf16 activations): the projections that take
# decode_linear run on dsv41_linear_rows -- the weight streamed once through the decode tile
# kernel's LDS copy ring, the contraction split so that small outputs still fill the chip --
# instead of torch's linear, whose library kernels for these shapes run ~17 us even for a 5 MB
# weight. Other shapes, dtypes and row counts take torch's linear.
DECODE_ROWS = 128


def _decode_ok(lin: torch.nn.Linear, x: torch.Tensor) -> bool:
    w = lin.weight
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.is_cuda and lin.bias is None
            and x.numel() // x.shape[-1] <= DECODE_ROWS and w.dim() == 2 and w.is_contiguous()
            and w.shape[1] % 64 == 0 and w.shape[0] % 32 == 0)


def decode_linear(lin: torch.nn.Linear, x: torch.Tensor, wide_only: bool = False) -> torch.Tensor:
    """lin(x) on dsv41_linear_rows at decode row counts, else torch's linear. wide_only: only where
    the 128-row tiles apply (the large projections wq_b and wo_b, 84 MB each at the release's
    widths, where the 32-row tiles lose to the library: wo_b 32.8 against 29.0 us at 64 rows)."""
    if _decode_ok(lin, x):
        k, n = lin.weight.shape[1], lin.weight.shape[0]
        rows = x.numel() // k
        splits = _abi.linear_rows_splits(k, n, rows)
        if not wide_only or _abi.linear_rows_wide(rows, k, n, splits):
            return _abi.linear_rows(x.contiguous(), lin.weight, splits)
    return lin(x)


def decode_linear_pair(lin0: torch.nn.Linear, lin1: torch.nn.Linear, x: torch.Tensor):
    """(lin0(x), lin1(x)) in one dsv41_linear_rows_pair launch at decode row counts (wq_a and wkv of
    attention.py:114/:116: 10.9 us at 64 rows against 10.2 + 8.4 us for the two calls), else the two
    decode_linear calls."""
    k = x.shape[-1]
    if (_decode_ok(lin0, x) and _decode_ok(lin1, x) and lin0.weight.shape[1] == lin1.weight.shape[1]
            and k % 128 == 0):
        return _abi.linear_rows_pair(x.contiguous(), lin0.weight, lin1.weight)
    return decode_linear(lin0, x), decode_linear(lin1, x)

def yarn_inv_freqs(dim: int, original_seq_len: int, base: float, factor: float,
                   beta_fast: int, beta_slow: int) -> np.ndarray:
    """[dim/2] fp32 inverse frequencies; ``original_seq_len == 0`` disables YaRN (layers.py:36-52)."""
    f32 = np.float32
    freqs = (f32(1.0) / (f32(base) ** (np.arange(0, dim, 2, dtype=f32) / f32(dim)))).astype(f32)
    if original_seq_len > 0:
        def corr(rot):
            return dim * math.log(original_seq_len / (rot * 2 * math.pi)) / (2 * math.log(base))
        lo = max(math.floor(corr(beta_fast)), 0)
        hi = min(math.ceil(corr(beta_slow)), dim - 1)
        ramp = np.clip((np.arange(dim // 2, dtype=f32) - f32(lo)) / f32(max(hi - lo, 1e-3)),
                       f32(0), f32(1)).astype(f32)
        smooth = (f32(1) - ramp).astype(f32)
        freqs = (freqs / f32(factor) * (f32(1) - smooth) + freqs * smooth).astype(f32)
    return freqs


def precompute_freqs_cis(dim: int, seqlen: int, original_seq_len: int, base: float,
                         factor: float, beta_fast: int, beta_slow: int, device="cuda"):
    """(cos, sin) tables [seqlen, dim//2] of the fp32 angles t * freqs (layers.py:36-56)."""
    freqs = torch.from_numpy(yarn_inv_freqs(dim, original_seq_len, base, factor, beta_fast,
                                            beta_slow)).to(device)
    return _abi.rope_table(freqs, seqlen)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     inverse: bool = False) -> torch.Tensor:
    """Rotate all of x [b, s, (h,) d] by tables already sliced to x's positions (layers.py:59-79)."""
    return _abi.rope_tail(x.contiguous(), x.shape[-1], cos.contiguous(), sin.contiguous(), 0, 1,
                          inverse)


def rope_tail(x: torch.Tensor, rd: int, cos: torch.Tensor, sin: torch.Tensor,
              inverse: bool = False) -> torch.Tensor:
    """Rope on the last rd channels, tables sliced to x's positions (layers.py:82-84)."""
    return _abi.rope_tail(x.contiguous(), rd, cos.contiguous(), sin.contiguous(), 0, 1, inverse)
