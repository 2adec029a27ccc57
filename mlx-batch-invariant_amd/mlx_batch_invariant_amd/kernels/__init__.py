"""Batch-invariant gfx950 kernels (hand-written HIP, C ABI in include/bi_kernels.h).

Every kernel obeys one rule (reference: mlx_batch_invariant/kernels/__init__.py:1-17):
the floating-point reduction order of an output element never depends on how many
*other* rows or sequences share the launch.

* matmul / quantized matmul: fixed 256-wide K groups, one MFMA instruction and one
  k-slot map for every tile shape, group partials folded left to right in fp32;
* rmsnorm / layernorm: one workgroup per row, fixed-stride partials, fixed-shape
  wave/LDS tree (layernorm: a mean pass, then a squared-deviation pass);
* attention: fixed 256-key splits folded in index order, one shared per-split
  sequence (split maximum, exp2 weights, MFMA P.V) for decode and prefill.

Only the launch shape adapts to the batch. Division and sqrt are correctly
rounded, exp is either the full-precision device expf or the hardware exp2
(attention), always the same one for a given quantity, every fma is explicit and
the build forbids fp contraction and fast math, so compiler choices cannot make
two kernels disagree.
"""

from .matmul import batch_invariant_bmm, batch_invariant_matmul
from .rmsnorm import batch_invariant_rms_norm
from .layernorm import batch_invariant_layer_norm
from .quantized import batch_invariant_quantized_matmul
from .attention import (
    batch_invariant_attention,
    batch_invariant_decode_attention,
    batch_invariant_paged_attention,
    batch_invariant_prefill_attention,
)

__all__ = [
    "batch_invariant_matmul",
    "batch_invariant_bmm",
    "batch_invariant_rms_norm",
    "batch_invariant_layer_norm",
    "batch_invariant_quantized_matmul",
    "batch_invariant_decode_attention",
    "batch_invariant_prefill_attention",
    "batch_invariant_attention",
    "batch_invariant_paged_attention",
]
