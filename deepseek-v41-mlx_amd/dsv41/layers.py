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


def decode_linear(lin: torch.nn.Linear, x: torch.Tensor) -> torch.Tensor:
    w = lin.weight
    rows = x.numel() // x.shape[-1]
    if (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.is_cuda and lin.bias is None
            and rows <= DECODE_ROWS and w.shape[1] % 64 == 0 and w.shape[0] % 32 == 0):
        return _abi.linear_rows(x.contiguous(), w)
    return lin(x)

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
