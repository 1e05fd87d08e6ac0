"""dsv41: the DeepSeek-V4.1 sparse-attention hot path on MI355X (gfx950).

Same module layout and call surface as the reference's ``deepseek_v41_mlx`` attention
modules (config, layers, fakequant, sparse_attention, indexer, compressor, cache,
attention, model), on torch device tensors, with every in-scope step running in the
hand-written HIP kernels of ``libdsv41.so`` (C ABI: include/dsv41.h).
"""

from .config import ModelArgs

__all__ = ["ModelArgs"]
