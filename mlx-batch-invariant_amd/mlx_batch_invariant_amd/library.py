"""The batch-invariant kernels as dispatcher operators: ``torch.ops.mlx_bi.*``.

Registered with ``torch.library.custom_op`` when the package is imported, each
with a fake (shape / dtype) implementation, so code that goes through the
dispatcher reaches the HIP kernels by name: ``torch.compile`` graphs (the op
stays one opaque node; no generated kernel replaces it), ``torch.export``, and
C++ code in the same process through ``c10::Dispatcher``
(``findSchemaOrThrow("mlx_bi::matmul", "")``). The mode's monkey-patching
cannot reach callers that captured the stock functions before it was entered
(the reference's limitation, README.md:252-253); an explicit
``torch.ops.mlx_bi.*`` call is bound to the kernel whatever the mode.

Operators (each the same computation, and bits, as the Python function named):

* ``matmul(a, b)``: ``batch_invariant_matmul`` for 2-D ``b``, else
  ``batch_invariant_bmm``;
* ``quantized_matmul(x, w, scales, biases, group_size, bits)``;
* ``rms_norm(x, weight, eps)``; ``layer_norm(x, weight, bias, eps)``;
* ``attention(q, k, v, scale, causal, kv_lens)``: decode for one query token,
  prefill otherwise (``mask="causal"`` is bottom-right aligned);
* ``paged_attention(q, k_pages, v_pages, block_table, kv_lens, scale, causal)``:
  the same over a paged K/V pool (``batch_invariant_paged_attention``).

The ops have no autograd formula (inference kernels, as in the reference).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import kernels as _k

NAMESPACE = "mlx_bi"


@torch.library.custom_op(f"{NAMESPACE}::matmul", mutates_args=())
def matmul(a: Tensor, b: Tensor) -> Tensor:
    return _k.batch_invariant_matmul(a, b) if b.ndim == 2 else _k.batch_invariant_bmm(a, b)


@matmul.register_fake
def _matmul_fake(a, b):
    dt = torch.result_type(a, b)
    if b.ndim == 2:
        return a.new_empty((*a.shape[:-1], b.shape[1]), dtype=dt)
    batch = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    return a.new_empty((*batch, a.shape[-2], b.shape[-1]), dtype=dt)


@torch.library.custom_op(f"{NAMESPACE}::quantized_matmul", mutates_args=())
def quantized_matmul(x: Tensor, w: Tensor, scales: Tensor, biases: Tensor, group_size: int, bits: int) -> Tensor:
    return _k.batch_invariant_quantized_matmul(x, w, scales, biases, group_size=group_size, bits=bits)


@quantized_matmul.register_fake
def _quantized_matmul_fake(x, w, scales, biases, group_size, bits):
    return x.new_empty((*x.shape[:-1], w.shape[0]))


@torch.library.custom_op(f"{NAMESPACE}::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Optional[Tensor], eps: float) -> Tensor:
    return _k.batch_invariant_rms_norm(x, weight, eps)


@rms_norm.register_fake
def _rms_norm_fake(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op(f"{NAMESPACE}::layer_norm", mutates_args=())
def layer_norm(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float) -> Tensor:
    return _k.batch_invariant_layer_norm(x, weight, bias, eps)


@layer_norm.register_fake
def _layer_norm_fake(x, weight, bias, eps):
    return torch.empty_like(x)


@torch.library.custom_op(f"{NAMESPACE}::attention", mutates_args=())
def attention(q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool, kv_lens: Optional[Tensor]) -> Tensor:
    return _k.batch_invariant_attention(q, k, v, scale=scale, mask="causal" if causal else None, kv_lens=kv_lens)


@attention.register_fake
def _attention_fake(q, k, v, scale, causal, kv_lens):
    return q.new_empty((*q.shape[:-1], v.shape[-1]))


@torch.library.custom_op(f"{NAMESPACE}::paged_attention", mutates_args=())
def paged_attention(q: Tensor, k_pages: Tensor, v_pages: Tensor, block_table: Tensor, kv_lens: Optional[Tensor],
                    scale: float, causal: bool) -> Tensor:
    return _k.batch_invariant_paged_attention(q, k_pages, v_pages, block_table, kv_lens, scale=scale,
                                              mask="causal" if causal else None)


@paged_attention.register_fake
def _paged_attention_fake(q, k_pages, v_pages, block_table, kv_lens, scale, causal):
    return q.new_empty((*q.shape[:-1], v_pages.shape[-1]))
