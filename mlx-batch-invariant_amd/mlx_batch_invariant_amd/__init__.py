"""Batch-invariant inference kernels for MI355X (gfx950), on PyTorch-ROCm tensors.

    import mlx_batch_invariant_amd as bi
    with bi.set_batch_invariant_mode():
        logits = model(tokens)          # same bits at batch 1 and batch 256
    print(bi.stats())                   # which ops were handled / fell back

Drop-in counterpart of mlx-batch-invariant's Python surface
(mlx_batch_invariant/__init__.py:9-32) for torch models.
"""

from ._mode import is_batch_invariant_mode_enabled, set_batch_invariant_mode
from .ops import reset_stats, stats
from .kernels import (
    batch_invariant_attention,
    batch_invariant_decode_attention,
    batch_invariant_paged_attention,
    batch_invariant_prefill_attention,
    batch_invariant_bmm,
    batch_invariant_layer_norm,
    batch_invariant_matmul,
    batch_invariant_quantized_matmul,
    batch_invariant_rms_norm,
)
from .kernels.quantized import (quantize, dequantize, pack, unpack, cache_dequantized, drop_dequantized,
                                cache_packed, drop_packed)
from .kernels.matmul import cache_packed_weight, drop_packed_weight
from . import library  # registers torch.ops.mlx_bi.*

__all__ = [
    "set_batch_invariant_mode",
    "is_batch_invariant_mode_enabled",
    "stats",
    "reset_stats",
    "batch_invariant_matmul",
    "batch_invariant_bmm",
    "batch_invariant_rms_norm",
    "batch_invariant_layer_norm",
    "batch_invariant_quantized_matmul",
    "batch_invariant_decode_attention",
    "batch_invariant_prefill_attention",
    "batch_invariant_attention",
    "batch_invariant_paged_attention",
    "quantize",
    "dequantize",
    "cache_dequantized",
    "drop_dequantized",
    "cache_packed",
    "drop_packed",
    "cache_packed_weight",
    "drop_packed_weight",
    "pack",
    "unpack",
]
__version__ = "0.1.0"
