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

_lock = threading.Lock()
_depth = 0
_saved: dict = {}


def _apply():
    global _saved
    _saved = {
        "matmul": torch.matmul,
        "mm": torch.mm,
        "bmm": torch.bmm,
        "addmm": torch.addmm,
        "tensor_matmul": torch.Tensor.__matmul__,
        "linear": F.linear,
        "rms_norm": F.rms_norm,
        "layer_norm": F.layer_norm,
        "sdpa": F.scaled_dot_product_attention,
        "quantized_matmul": _bnn.quantized_matmul,
    }
    torch.matmul = ops.matmul
    torch.mm = ops.mm
    torch.bmm = ops.bmm
    torch.addmm = ops.addmm
    torch.Tensor.__matmul__ = ops.tensor_matmul
    F.linear = ops.linear
    F.rms_norm = ops.rms_norm
    F.layer_norm = ops.layer_norm
    F.scaled_dot_product_attention = ops.scaled_dot_product_attention
    _bnn.quantized_matmul = ops.quantized_matmul


def _restore():
    torch.matmul = _saved["matmul"]
    torch.mm = _saved["mm"]
    torch.bmm = _saved["bmm"]
    torch.addmm = _saved["addmm"]
    torch.Tensor.__matmul__ = _saved["tensor_matmul"]
    F.linear = _saved["linear"]
    F.rms_norm = _saved["rms_norm"]
    F.layer_norm = _saved["layer_norm"]
    F.scaled_dot_product_attention = _saved["sdpa"]
    _bnn.quantized_matmul = _saved["quantized_matmul"]


def is_batch_invariant_mode_enabled() -> bool:
    return _depth > 0


@contextlib.contextmanager
def set_batch_invariant_mode(enabled: bool = True, *, strict: bool = False):
    """Route matmul / bmm / linear / addmm / quantized matmul / rms_norm /
    layer_norm / sdpa through
    the batch-invariant kernels for the duration of the block.

    ``strict=True`` raises instead of silently falling back to a stock kernel
    for unsupported inputs. Re-entrant; process-global (torch dispatch by
    attribute lookup is), guarded by a lock.
    """
    global _depth
    if not enabled:
        yield
        return
    with _lock:
        if _depth == 0:
            _apply()
        _depth += 1
        prev_strict = ops.strict
        ops.strict = strict
    try:
        yield
    finally:
        with _lock:
            ops.strict = prev_strict
            _depth -= 1
            if _depth == 0:
                _restore()
