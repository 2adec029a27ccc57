"""Batch-invariant LayerNorm over the last dimension on gfx950.

The reference has no LayerNorm kernel (roadmap item "a batch-invariant
mx.fast.layer_norm", README.md:257-260; GPT-2 runs the stock op,
README.md:250-251). This one follows the RMSNorm contract
(kernels/rmsnorm.py:19-47 there): one 256-thread workgroup per row, thread t
owns 8-element chunks t, t+256, ...; pass 1 sums x, pass 2 sums
``fmaf(d, d, ss)`` with ``d = x - mean``, each through the fixed wave butterfly
and a left-to-right fold of the four wave sums; ``mean = S / D``,
``var = SS / D``, ``inv = 1 / sqrtf(var + eps)`` (correctly rounded), then
``out = T(((x - mean) * inv) * w + b)``. The order depends on D only.
"""

from __future__ import annotations

import torch

from .. import _lib


def _vec(t, D, dtype, name):
    if t is None:
        return None
    if t.numel() != D:
        raise ValueError(f"batch_invariant_layer_norm: {name} has {t.numel()} elements, expected {D}")
    if t.ndim != 1:
        t = t.reshape(D)
    if t.dtype != dtype:
        t = t.to(dtype)
    return t if t.is_contiguous() else t.contiguous()


def batch_invariant_layer_norm(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                               eps: float) -> torch.Tensor:
    if x.dtype not in _lib.FLOAT_DTYPES:
        raise ValueError(f"batch_invariant_layer_norm: unsupported dtype {x.dtype}")
    _lib.require_gpu("batch_invariant_layer_norm", x, weight, bias)
    D = x.shape[-1]
    weight = _vec(weight, D, x.dtype, "weight")
    bias = _vec(bias, D, x.dtype, "bias")
    rows = x.numel() // D if D else 0
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if rows == 0 or D == 0:
        return out
    x2 = x if x.ndim == 2 else x.reshape(rows, D)
    if x2.stride(-1) != 1 or x2.stride(0) < D:
        x2 = x2.contiguous()
    lib = _lib.load()
    rc = lib.bi_layer_norm(x2.data_ptr(), x2.stride(0), _lib.ptr(weight), _lib.ptr(bias), out.data_ptr(), rows, D,
                           float(eps), _lib.DTYPE_CODE[x.dtype], _lib.stream_of(x))
    _lib.check(rc, "bi_layer_norm")
    return out
