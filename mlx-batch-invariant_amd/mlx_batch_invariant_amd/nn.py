"""Torch modules for the MLX affine quantized format.

``QuantizedLinear`` holds a packed uint32 weight ``[N, K*bits/32]`` with
scales/biases ``[N, K/group_size]`` (MLX's layout) and calls the module-level
``quantized_matmul`` through attribute lookup at call time, exactly as MLX's
``nn.QuantizedLinear`` calls ``mx.quantized_matmul``. Outside the mode that is
the stock path (dequantize + torch.matmul); inside ``set_batch_invariant_mode``
the mode swaps in the batch-invariant kernel.
"""

from __future__ import annotations

import sys

import torch

from .kernels import quantized as _quant


def quantized_matmul(x, w, scales, biases=None, transpose: bool = True, group_size=None,
                     bits=None, mode: str = "affine"):
    """Stock (non-invariant) path: dequantize, then torch.matmul."""
    gs = 64 if group_size is None else group_size
    b = 4 if bits is None else bits
    if mode != "affine" or biases is None:
        raise NotImplementedError(f"quantized_matmul: mode={mode!r} without biases is not supported")
    W = _quant.dequantize(w, scales, biases, gs, b, dtype=x.dtype)
    return torch.matmul(x, W.t() if transpose else W)


_this = sys.modules[__name__]


class QuantizedLinear(torch.nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = True, group_size: int = 64,
                 bits: int = 4, device=None, dtype=torch.bfloat16):
        super().__init__()
        if in_features % group_size:
            raise ValueError("in_features must be a multiple of group_size")
        self.in_features, self.out_features = in_features, out_features
        self.group_size, self.bits = group_size, bits
        W = torch.randn(out_features, in_features, device=device) * (in_features ** -0.5)
        wq, s, b = _quant.quantize(W, group_size, bits, dtype=dtype)
        self.register_buffer("weight", wq.view(torch.int32))  # same bits as MLX's uint32
        self.register_buffer("scales", s)
        self.register_buffer("biases", b)
        self.bias = torch.nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype)) if bias else None

    @classmethod
    def from_linear(cls, lin: torch.nn.Linear, group_size: int = 64, bits: int = 4):
        q = cls.__new__(cls)
        torch.nn.Module.__init__(q)
        q.in_features, q.out_features = lin.in_features, lin.out_features
        q.group_size, q.bits = group_size, bits
        wq, s, b = _quant.quantize(lin.weight.detach(), group_size, bits, dtype=lin.weight.dtype)
        q.register_buffer("weight", wq.view(torch.int32))
        q.register_buffer("scales", s)
        q.register_buffer("biases", b)
        q.bias = None if lin.bias is None else torch.nn.Parameter(lin.bias.detach().clone())
        return q

    def cache_dequantized(self):
        """Keep the weight dequantized once (``kernels.quantized.cache_dequantized``):
        under the mode, calls with at least ``DEQUANTIZED_MIN_M`` rows (prefill)
        then skip the per-call dequantization, with the same bits. Costs
        out_features * in_features * 2 bytes of device memory."""
        _quant.cache_dequantized(self.weight, self.scales, self.biases, group_size=self.group_size, bits=self.bits)
        return self

    def cache_packed(self):
        """Keep a repacked copy of the codes (``kernels.quantized.cache_packed``):
        under the mode, calls with at most ``PACKED_MAX_M`` rows (decode) then
        read it in the decode GEMV's layout, with the same bits. Costs about
        the codes' size again in device memory."""
        _quant.cache_packed(self.weight, self.scales, self.biases, group_size=self.group_size, bits=self.bits)
        return self

    def forward(self, x):
        y = _this.quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                                   group_size=self.group_size, bits=self.bits)
        return y if self.bias is None else y + self.bias


def cache_packed_linears(module: torch.nn.Module) -> torch.nn.Module:
    """Repack every linear weight of ``module`` once for the decode GEMV:
    ``QuantizedLinear.cache_packed()`` for the quantized ones (in_features a
    multiple of 256) and ``cache_packed_weight`` for each ``nn.Linear`` whose
    weight qualifies (bf16 / fp16, in_features a multiple of 8). Decode calls
    (at most 16 rows) under the mode then read the copies, with the same bits."""
    from .kernels.matmul import cache_packed_weight
    for m in module.modules():
        if isinstance(m, QuantizedLinear):
            if m.in_features % 256 == 0 and m.scales.dtype in (torch.bfloat16, torch.float16):
                m.cache_packed()
        elif isinstance(m, torch.nn.Linear):
            w = m.weight
            if w.is_cuda and w.dtype in (torch.bfloat16, torch.float16) and w.shape[1] % 8 == 0:
                cache_packed_weight(w)     # the parameter itself: the cache holds a weak reference to it
    return module
