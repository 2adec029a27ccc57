"""The override mechanism (reference: mlx_batch_invariant/_mode.py:1-91).

Torch resolves ``torch.matmul``, ``F.linear``, ``F.rms_norm``,
``F.layer_norm`` and ``F.scaled_dot_product_attention`` by attribute lookup at
call time, and
``a @ b`` through ``torch.Tensor.__matmul__``. So, like the reference does for
MLX, the mode swaps those module attributes (plus ``torch.mm``,
``torch.addmm`` and this package's own ``nn.quantized_matmul``, which
``nn.QuantizedLinear`` calls) for the wrappers in ``ops`` while any ``with``
block is open (and ``torch.bmm``, ``F.layer_norm``, which the reference has no
kernel for), and restores them on exit. ``nn.Linear`` reaches ``F.linear``,
``nn.RMSNorm`` reaches ``F.rms_norm``, ``nn.LayerNorm`` reaches
``F.layer_norm``, attention code reaches ``F.scaled_dot_product_attention``:
all are covered.

Not covered (falls back, counted): 1-D matmul operands, attention with tensor
masks or dropout, non-affine quantization. Code that captured a
stock function object before the mode was entered keeps calling it.
"""

from __future__ import annotations

import contextlib
import threading

import torch
import torch.nn.functional as F

from . import nn as _bnn
from . import ops

# (owner object, attribute, replacement): every entry point the mode swaps.
_PATCHES = (
    (torch, "matmul", ops.matmul),
    (torch, "mm", ops.mm),
    (torch, "bmm", ops.bmm),
    (torch, "addmm", ops.addmm),
    (torch.Tensor, "__matmul__", ops.tensor_matmul),
    (F, "linear", ops.linear),
    (F, "rms_norm", ops.rms_norm),
    (F, "layer_norm", ops.layer_norm),
    (F, "scaled_dot_product_attention", ops.scaled_dot_product_attention),
    (_bnn, "quantized_matmul", ops.quantized_matmul),
)

_lock = threading.Lock()   # guards _depth, the patch state and ops.strict
_depth = 0                 # open `with` blocks, process-wide
_originals: list = []      # what _PATCHES replaced, in the same order


def _apply():
    """Swap every patched attribute for its wrapper, remembering the original."""
    _originals[:] = [getattr(owner, name) for owner, name, _ in _PATCHES]
    for owner, name, repl in _PATCHES:
        setattr(owner, name, repl)


def _restore():
    for (owner, name, _), orig in zip(_PATCHES, _originals):
        setattr(owner, name, orig)
    _originals.clear()


def is_batch_invariant_mode_enabled() -> bool:
    return _depth > 0


@contextlib.contextmanager
def set_batch_invariant_mode(enabled: bool = True, *, strict: bool = False, attention_order: str = "mfma"):
    """Inside the block, matmul / mm / bmm / addmm / ``@`` / linear / the
    package's quantized matmul / rms_norm / layer_norm / sdpa resolve to the
    batch-invariant kernels (reference: _mode.py:66-91).

    With ``strict`` an input no kernel handles raises ``RuntimeError``; without
    it the stock op runs and the fallback is counted. ``attention_order``
    picks the attention kernels: "mfma" (matrix cores, the default) or
    "per_key" (the reference's own order of operations, slower). Blocks nest:
    the swap happens when the first one opens and is undone when the last one
    closes, and each block's ``strict`` and ``attention_order`` hold until it
    closes. ``enabled=False`` is a
    no-op block. The swap is process-wide, since torch looks these attributes
    up at call time; a lock serialises opening and closing.
    """
    global _depth
    if not enabled:
        yield
        return
    from .kernels.attention import ORDERS
    if attention_order not in ORDERS:
        raise ValueError(f"attention_order must be one of {ORDERS}; got {attention_order!r}")
    with _lock:
        outer = (ops.strict, ops.attention_order)
        if _depth == 0:
            _apply()
        _depth += 1
        ops.strict, ops.attention_order = strict, attention_order
    try:
        yield
    finally:
        with _lock:
            _depth -= 1
            ops.strict, ops.attention_order = outer
            if _depth == 0:
                _restore()
