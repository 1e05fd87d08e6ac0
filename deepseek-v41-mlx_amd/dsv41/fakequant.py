"""The QAT activation fake-quants on the GPU (deepseek_v41_mlx/fakequant.py).

* window KV: fp8 e4m3, blocks of 32, ue8m0 (power-of-two) scales;
* compressed KV latents: fp4 e2m1, blocks of 16, e4m3 scales;
* indexer queries and keys: fp4 e2m1, blocks of 32, ue8m0 scales.

Each returns a new tensor of the input dtype. ``DISABLE`` is the reference's test hook
(fakequant.py:33-37): with it set, the attention path skips every fake-quant.
"""

from __future__ import annotations

import torch

from . import _abi

DISABLE = False


def fake_quant_fp8_ue8m0(x: torch.Tensor, block: int = 32) -> torch.Tensor:
    if DISABLE:
        return x
    return _abi.fq_fp8_ue8m0(x.contiguous(), block)


def fake_quant_fp4_ue8m0(x: torch.Tensor, block: int = 32) -> torch.Tensor:
    if DISABLE:
        return x
    return _abi.fq_fp4_ue8m0(x.contiguous(), block)


def fake_quant_fp4_e4m3(x: torch.Tensor, block: int = 16) -> torch.Tensor:
    if DISABLE:
        return x
    return _abi.fq_fp4_e4m3(x.contiguous(), block)
