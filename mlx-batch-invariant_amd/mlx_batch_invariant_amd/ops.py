"""Functional entry points with explicit fallback accounting.

Torch counterpart of mlx_batch_invariant/ops.py:1-104. Each op has the
signature of the stock torch op it stands in for and returns the
batch-invariant result when a kernel supports the inputs; otherwise it calls
the stock op (captured at import, so patching never recurses) and records a
fallback under ``"op:reason"``, or raises ``RuntimeError`` when the mode is
strict. "Deterministic" with ten silent fallbacks is not deterministic, so the
counters are public through ``stats()``.

Counter keys (same as the reference): handled ``matmul``, ``addmm``,
``quantized_matmul``, ``rms_norm``, ``sdpa_decode``, ``sdpa_prefill``;
fallbacks ``matmul:non-2d-rhs-or-non-float``, ``addmm:non-2d-rhs-or-non-float``,
``quantized_matmul:{mode}-{bits}bit-g{gs}-{T|N}``, ``rms_norm:non-float``,
``sdpa:array-mask``, ``sdpa:sinks-or-shape``. One reason is new: inputs
that are not GPU tensors fall back as ``{op}:non-gpu-tensor``.

Beyond the reference's op set: right-hand sides with batch dims (``torch.matmul``
of 2+-D operands, ``torch.bmm``) run the batched kernel and count as
``matmul`` (the reference falls back there, ``matmul:non-2d-rhs-or-non-float``;
a 1-D operand still does); ``F.layer_norm`` over the last dim counts as
``layer_norm`` (fallbacks ``layer_norm:non-float``, ``layer_norm:non-last-dim``).
"""

from __future__ import annotations

import math
from collections import Counter

import torch
import torch.nn.functional as F
from torch.nn.attention.bias import CausalBias as _CausalBias
from torch.nn.attention.bias import CausalVariant as _CausalVariant

from . import _lib
from .kernels import (
    batch_invariant_attention,
    batch_invariant_bmm,
    batch_invariant_layer_norm,
    batch_invariant_matmul,
    batch_invariant_quantized_matmul,
    batch_invariant_rms_norm,
)
from .kernels import attention as _attn
from .kernels import quantized as _quant

# Stock implementations, captured at import so patching never recurses.
_orig_matmul = torch.matmul
_orig_mm = torch.mm
_orig_bmm = torch.bmm
_orig_addmm = torch.addmm
_orig_tensor_matmul = torch.Tensor.__matmul__
_orig_linear = F.linear
_orig_rms_norm = F.rms_norm
_orig_layer_norm = F.layer_norm
_orig_sdpa = F.scaled_dot_product_attention

handled: Counter = Counter()
fallbacks: Counter = Counter()
strict: bool = False
attention_order: str = "mfma"   # "per_key": the reference's own attention order


def _fallback(op: str, reason: str):
    fallbacks[f"{op}:{reason}"] += 1
    if strict:
        raise RuntimeError(f"batch-invariant mode: no kernel for {op} ({reason})")


def _is_float(x) -> bool:
    return isinstance(x, torch.Tensor) and x.dtype in _lib.FLOAT_DTYPES


def _on_gpu(*ts) -> bool:
    return all(_lib.is_gpu_tensor(t) for t in ts if t is not None)


def _mm_reason(a, b, batched_ok: bool = False) -> str | None:
    """None if the dense kernel takes (a, b); else the fallback reason. With
    ``batched_ok`` a right-hand side with batch dims is taken too (both
    operands 2+-D)."""
    if not (_is_float(a) and _is_float(b)):
        return "non-2d-rhs-or-non-float"
    two_d = b.ndim == 2 and a.ndim >= 1
    batched = batched_ok and b.ndim >= 3 and a.ndim >= 2
    if not (two_d or batched):
        return "non-2d-rhs-or-non-float"
    if not _on_gpu(a, b) or a.device != b.device:
        return "non-gpu-tensor"
    return None


def _matmul_any(a, b):
    return batch_invariant_matmul(a, b) if b.ndim == 2 else batch_invariant_bmm(a, b)


def matmul(a, b, *, out=None):
    reason = "out-argument" if out is not None else _mm_reason(a, b, batched_ok=True)
    if reason is None:
        handled["matmul"] += 1
        return _matmul_any(a, b)
    _fallback("matmul", reason)
    return _orig_matmul(a, b) if out is None else _orig_matmul(a, b, out=out)


def bmm(a, b, *, out=None):
    reason = "out-argument" if out is not None else _mm_reason(a, b, batched_ok=True)
    if reason is None and not (a.ndim == 3 and b.ndim == 3 and a.shape[0] == b.shape[0]):
        reason = "non-2d-rhs-or-non-float"     # let the stock op raise its own shape error
    if reason is None:
        handled["matmul"] += 1
        return batch_invariant_bmm(a, b)
    _fallback("matmul", reason)
    return _orig_bmm(a, b) if out is None else _orig_bmm(a, b, out=out)


def mm(a, b, *, out=None):
    reason = "out-argument" if out is not None else _mm_reason(a, b)
    if reason is None and a.ndim == 2:
        handled["matmul"] += 1
        return batch_invariant_matmul(a, b)
    _fallback("matmul", reason or "non-2d-rhs-or-non-float")
    return _orig_mm(a, b) if out is None else _orig_mm(a, b, out=out)


def tensor_matmul(self, other):
    reason = _mm_reason(self, other, batched_ok=True)
    if reason is None:
        handled["matmul"] += 1
        return _matmul_any(self, other)
    _fallback("matmul", reason)
    return _orig_tensor_matmul(self, other)


def addmm(c, a, b, *, beta=1, alpha=1, out=None):
    reason = "out-argument" if out is not None else _mm_reason(a, b)
    if reason is None and a.ndim != 2:
        reason = "non-2d-rhs-or-non-float"
    if reason is None and isinstance(c, torch.Tensor) and not _on_gpu(c):
        reason = "non-gpu-tensor"
    if reason is None and isinstance(c, torch.Tensor) and c.dtype != torch.result_type(a, b):
        reason = "dtype-mismatch"              # the stock op raises its own error for mixed dtypes
    if reason is None:
        handled["addmm"] += 1
        prod = batch_invariant_matmul(a, b)
        if alpha != 1:
            prod = prod * alpha
        if beta == 0:                          # as torch.addmm: c is ignored, NaN/Inf in it do not propagate
            return prod.expand(torch.broadcast_shapes(prod.shape, c.shape)).clone() if isinstance(
                c, torch.Tensor) else prod
        return prod + (c if beta == 1 else c * beta)
    _fallback("addmm", reason)
    kw = {"beta": beta, "alpha": alpha}
    return _orig_addmm(c, a, b, **kw) if out is None else _orig_addmm(c, a, b, out=out, **kw)


def linear(input, weight, bias=None):
    """``F.linear``: ``input @ weight.T (+ bias)``. Counted as ``matmul`` without
    bias and ``addmm`` with bias, like MLX's nn.Linear (x @ W.T / mx.addmm)."""
    op = "matmul" if bias is None else "addmm"
    reason = _mm_reason(input, weight.t() if isinstance(weight, torch.Tensor) and weight.ndim == 2 else weight)
    if reason is None and bias is not None and not _on_gpu(bias):
        reason = "non-gpu-tensor"
    if reason is None:
        handled[op] += 1
        prod = batch_invariant_matmul(input, weight.t())
        return prod if bias is None else prod + bias
    _fallback(op, reason)
    return _orig_linear(input, weight, bias)


def quantized_matmul(x, w, scales, biases=None, transpose: bool = True, group_size=None,
                     bits=None, mode: str = "affine"):
    """Signature of mx.quantized_matmul (reference ops.py:65-77). There is no
    stock torch op for the MLX affine format; the stock path is dequantize +
    torch.matmul."""
    gs = 64 if group_size is None else group_size
    b = 4 if bits is None else bits
    if _quant.supports(x, w, scales, biases, transpose, gs, b, mode):
        handled["quantized_matmul"] += 1
        return batch_invariant_quantized_matmul(x, w, scales, biases, group_size=gs, bits=b)
    _fallback("quantized_matmul", f"{mode}-{b}bit-g{gs}-{'T' if transpose else 'N'}")
    if mode != "affine" or biases is None:
        raise NotImplementedError(f"quantized_matmul: no stock path for mode={mode!r} without biases")
    W = _quant.dequantize(w, scales, biases, gs, b, dtype=x.dtype)
    return _orig_matmul(x, W.t() if transpose else W)


def rms_norm(input, normalized_shape, weight=None, eps=None):
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    shape_ok = (isinstance(input, torch.Tensor)
                and tuple(input.shape[input.ndim - len(normalized_shape):]) == tuple(normalized_shape))
    if _is_float(input) and shape_ok and (weight is None or _is_float(weight)):
        if _on_gpu(input, weight):
            handled["rms_norm"] += 1
            D = math.prod(normalized_shape)
            e = torch.finfo(input.dtype).eps if eps is None else eps
            x2 = input.reshape(*input.shape[:input.ndim - len(normalized_shape)], D)
            w2 = None if weight is None else weight.reshape(D)
            return batch_invariant_rms_norm(x2, w2, e).reshape(input.shape)
        _fallback("rms_norm", "non-gpu-tensor")
    else:
        _fallback("rms_norm", "non-float")
    return _orig_rms_norm(input, normalized_shape, weight, eps)


def layer_norm(input, normalized_shape, weight=None, bias=None, eps=1e-5):
    """``F.layer_norm``; the kernel normalises over the last dim, so a
    multi-dim ``normalized_shape`` is taken by flattening those dims."""
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    nd = len(normalized_shape)
    shape_ok = (isinstance(input, torch.Tensor) and nd >= 1
                and tuple(input.shape[input.ndim - nd:]) == tuple(normalized_shape))
    if not (_is_float(input) and (weight is None or _is_float(weight)) and (bias is None or _is_float(bias))):
        _fallback("layer_norm", "non-float")
    elif not shape_ok:
        _fallback("layer_norm", "non-last-dim")
    elif not _on_gpu(input, weight, bias):
        _fallback("layer_norm", "non-gpu-tensor")
    else:
        handled["layer_norm"] += 1
        D = math.prod(normalized_shape)
        x2 = input.reshape(*input.shape[:input.ndim - nd], D)
        w2 = None if weight is None else weight.reshape(D)
        b2 = None if bias is None else bias.reshape(D)
        return batch_invariant_layer_norm(x2, w2, b2, eps).reshape(input.shape)
    return _orig_layer_norm(input, normalized_shape, weight, bias, eps)


def _causal_variant(attn_mask, is_causal, Tq, L):
    """(supported, variant) for the mask arguments: variant None, "upper_left"
    (torch's ``is_causal`` / ``causal_upper_left``) or "lower_right"
    (``causal_lower_right``, MLX's ``mask="causal"``)."""
    if isinstance(attn_mask, _CausalBias):
        if is_causal or (attn_mask.seq_len_q, attn_mask.seq_len_kv) != (Tq, L):
            return False, None
        if attn_mask.variant == _CausalVariant.LOWER_RIGHT:
            return True, "lower_right"
        return True, "upper_left"
    if attn_mask is not None:
        return False, None
    return True, ("upper_left" if is_causal else None)


def scaled_dot_product_attention(query, key, value, attn_mask=None, dropout_p=0.0,
                                 is_causal=False, scale=None, enable_gqa=False, **kwargs):
    """``F.scaled_dot_product_attention``. The kernel's causal mask is
    bottom-right aligned (query t of T_q sees ``L - T_q + t + 1`` keys): that is
    what ``attn_mask=causal_lower_right(T_q, L)`` asks for (chunked prefill
    over a KV cache). ``is_causal`` / ``causal_upper_left`` follow torch's
    top-left alignment; for T_q <= L that equals the bottom-right mask on the
    first T_q keys, so that is what is run."""
    q, k, v = query, key, value
    shapes = (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor)
              and q.ndim == 4 and k.ndim == 4)
    mask_ok, variant = (_causal_variant(attn_mask, is_causal, q.shape[2], k.shape[2]) if shapes
                        else (False, None))
    ok = (shapes and mask_ok and dropout_p == 0.0 and not kwargs
          and (q.shape[1] == k.shape[1] or enable_gqa)
          and not (variant is not None and q.shape[2] > k.shape[2]))
    if ok:
        if variant == "upper_left" and q.shape[2] < k.shape[2]:
            k = k[:, :, : q.shape[2]]
            v = v[:, :, : q.shape[2]]
        mask = None if variant is None else "causal"
        if _attn.supports(q, k, v, mask):
            handled["sdpa_decode" if q.shape[2] == 1 else "sdpa_prefill"] += 1
            sc = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
            # head dims only the per-key kernels take run there whatever the mode's order
            order = attention_order if q.shape[-1] in _attn.MFMA_HEAD_DIMS else "per_key"
            return batch_invariant_attention(q, k, v, scale=sc, mask=mask, order=order)
    if isinstance(attn_mask, torch.Tensor) and not (mask_ok and isinstance(attn_mask, _CausalBias)):
        reason = "array-mask"
    elif ok and not _on_gpu(q, k, v):
        reason = "non-gpu-tensor"
    else:
        reason = "sinks-or-shape"
    _fallback("sdpa", reason)
    if isinstance(attn_mask, _CausalBias):
        # CausalBias dispatches through __torch_function__ only when it sees
        # torch's own F.scaled_dot_product_attention, which is patched here:
        # hand the stock op the equivalent boolean mask instead.
        Tq, L = attn_mask.seq_len_q, attn_mask.seq_len_kv
        diag = L - Tq if attn_mask.variant == _CausalVariant.LOWER_RIGHT else 0
        attn_mask = torch.ones((Tq, L), dtype=torch.bool, device=query.device).tril(diag)
    extra = {"enable_gqa": enable_gqa} if enable_gqa else {}
    return _orig_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                      is_causal=is_causal, scale=scale, **extra, **kwargs)


def reset_stats():
    handled.clear()
    fallbacks.clear()


def stats() -> dict:
    return {"handled": dict(handled), "fallbacks": dict(fallbacks)}
