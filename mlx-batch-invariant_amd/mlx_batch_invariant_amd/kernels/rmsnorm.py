"""Batch-invariant RMSNorm on gfx950.

One 256-thread workgroup per row, whatever the row count (reference:
mlx_batch_invariant/kernels/rmsnorm.py:1-79). The row is read as 8-element
chunks; thread t owns chunks t, t+256, ... and sums ``fmaf(v, v, ss)`` over
them in order; each wave64 folds its partials with a fixed xor butterfly and
the four wave sums are added left to right. ``inv = 1 / sqrtf(ss / D + eps)``
with correctly rounded division and square root, then
``out = T((x * inv) * w)``. The reduction order depends on D only.
"""

from __future__ import annotations

import torch

from .. import _lib

TG = 256


def batch_invariant_rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    if x.dtype not in _lib.FLOAT_DTYPES:
        raise ValueError(f"batch_invariant_rms_norm: unsupported dtype {x.dtype}")
    _lib.require_gpu("batch_invariant_rms_norm", x, weight)
    D = x.shape[-1]
    if weight is not None:
        if weight.numel() != D:
            raise ValueError(f"batch_invariant_rms_norm: weight has {weight.numel()} elements, expected {D}")
        if weight.ndim != 1:
            weight = weight.reshape(D)
        if weight.dtype != x.dtype:
            weight = weight.to(x.dtype)
        if not weight.is_contiguous():
            weight = weight.contiguous()
    rows = x.numel() // D if D else 0
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if rows == 0 or D == 0:
        return out
    x2 = x if x.ndim == 2 else x.reshape(rows, D)
    if x2.stride(-1) != 1 or x2.stride(0) < D:
        x2 = x2.contiguous()
    _lib.load()
    rc = _lib.rms_norm_call(x2.data_ptr(), x2.stride(0), _lib.ptr(weight), out.data_ptr(), rows, D,
                            float(eps), _lib.DTYPE_CODE[x.dtype], _lib.stream_of(x))
    _lib.check(rc, "bi_rms_norm")
    return out
