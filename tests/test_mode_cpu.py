"""Mode and dispatch contract on the CPU (reference tests
tests/test_batch_invariance.py:50-70 and :91-105 restated for torch). CPU
tensors are inputs the kernels do not take, so they exercise fallback counting
and strict raising without a GPU."""

import threading

import pytest
import torch
import torch.nn.functional as F

import mlx_batch_invariant_amd as bi
from mlx_batch_invariant_amd import nn as bnn
from mlx_batch_invariant_amd import ops


def _symbols():
    return (torch.matmul, torch.mm, torch.bmm, torch.addmm, torch.Tensor.__matmul__, F.linear, F.rms_norm,
            F.layer_norm, F.scaled_dot_product_attention, bnn.quantized_matmul)


def test_mode_patches_and_restores():
    orig = _symbols()
    assert not bi.is_batch_invariant_mode_enabled()
    with bi.set_batch_invariant_mode():
        assert bi.is_batch_invariant_mode_enabled()
        assert torch.matmul is ops.matmul and F.linear is ops.linear
        assert torch.Tensor.__matmul__ is ops.tensor_matmul
        assert torch.bmm is ops.bmm and F.layer_norm is ops.layer_norm
        with bi.set_batch_invariant_mode():  # re-entrant
            assert bi.is_batch_invariant_mode_enabled()
        assert bi.is_batch_invariant_mode_enabled()
        assert torch.matmul is ops.matmul
    assert not bi.is_batch_invariant_mode_enabled()
    assert _symbols() == orig


def test_disabled_mode_does_not_patch():
    orig = _symbols()
    with bi.set_batch_invariant_mode(enabled=False):
        assert _symbols() == orig
        assert not bi.is_batch_invariant_mode_enabled()


def test_strict_is_saved_and_restored_per_level():
    assert ops.strict is False
    with bi.set_batch_invariant_mode(strict=True):
        assert ops.strict is True
        with bi.set_batch_invariant_mode(strict=False):
            assert ops.strict is False
        assert ops.strict is True
    assert ops.strict is False


def test_restores_after_exception():
    orig = _symbols()
    with pytest.raises(KeyError):
        with bi.set_batch_invariant_mode():
            raise KeyError("boom")
    assert _symbols() == orig and not bi.is_batch_invariant_mode_enabled()


def test_strict_mode_raises_on_unsupported():
    q = torch.randn((1, 4, 7, 32))
    m = torch.zeros((7, 7), dtype=torch.bool)
    with bi.set_batch_invariant_mode(strict=True):
        with pytest.raises(RuntimeError, match="no kernel for sdpa"):
            F.scaled_dot_product_attention(q, q, q, attn_mask=m)


def test_non_strict_counts_fallbacks():
    q = torch.randn((1, 4, 7, 32))
    m = torch.zeros((7, 7), dtype=torch.bool)
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        F.scaled_dot_product_attention(q, q, q, attn_mask=m)
    assert bi.stats()["fallbacks"].get("sdpa:array-mask") == 1


def test_fallback_returns_stock_result_and_counts():
    torch.manual_seed(0)
    x = torch.randn(3, 16)
    W = torch.randn(8, 16)
    b = torch.randn(8)
    ref_mm = torch.matmul(x, W.T)
    ref_lin = F.linear(x, W, b)
    ref_norm = F.rms_norm(x, (16,), None, 1e-6)
    ref_bmm = torch.bmm(x[None], W.T[None])
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        assert torch.equal(x @ W.T, ref_mm)
        assert torch.equal(torch.matmul(x, W.T), ref_mm)
        assert torch.equal(F.linear(x, W, b), ref_lin)
        assert torch.equal(F.rms_norm(x, (16,), None, 1e-6), ref_norm)
        torch.matmul(torch.ones(2, 3, dtype=torch.int64), torch.ones(3, 2, dtype=torch.int64))
        torch.matmul(x, torch.randn(2, 16, 4))      # 3-D rhs: the batched kernel's (GPU only)
        torch.matmul(x, torch.randn(16))            # 1-D rhs: no kernel
        assert torch.equal(torch.bmm(x[None], W.T[None]), ref_bmm)
        ref_ln = torch.nn.LayerNorm(16)(x)
        assert torch.equal(torch.nn.LayerNorm(16)(x), ref_ln)
        F.layer_norm(x, (3, 16))                    # trailing dims flattened: still the kernel's
    st = bi.stats()
    assert st["handled"] == {}
    assert st["fallbacks"] == {"matmul:non-gpu-tensor": 4, "addmm:non-gpu-tensor": 1,
                               "rms_norm:non-gpu-tensor": 1, "matmul:non-2d-rhs-or-non-float": 2,
                               "layer_norm:non-gpu-tensor": 3}


def test_quantized_fallback_key_and_stock_path():
    W = torch.randn(16, 64)
    wq, s, b = bi.quantize(W, group_size=32, bits=4, dtype=torch.float32)
    x = torch.randn(2, 64)
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        y = bnn.quantized_matmul(x, wq, s, b, transpose=True, group_size=32, bits=4)
    assert bi.stats()["fallbacks"] == {"quantized_matmul:affine-4bit-g32-T": 1}
    ref = torch.matmul(x, bi.dequantize(wq, s, b, 32, 4, dtype=torch.float32).T)
    assert torch.equal(y, ref)
    with bi.set_batch_invariant_mode(strict=True):
        with pytest.raises(RuntimeError, match="quantized_matmul"):
            bnn.quantized_matmul(x, wq, s, b, group_size=32, bits=4)


def test_quantized_linear_calls_module_level_function():
    lin = bnn.QuantizedLinear(64, 16, bias=True, group_size=64, bits=4, dtype=torch.float32)
    x = torch.randn(3, 64)
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        y = lin(x)
    assert y.shape == (3, 16)
    assert bi.stats()["fallbacks"] == {"quantized_matmul:affine-4bit-g64-T": 1}


def test_mode_is_thread_safe():
    orig = _symbols()
    errors = []

    def worker():
        try:
            for _ in range(50):
                with bi.set_batch_invariant_mode():
                    assert bi.is_batch_invariant_mode_enabled()
        except Exception as e:  # pragma: no cover
            errors.append(e)

    ts = [threading.Thread(target=worker) for _ in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    assert _symbols() == orig and not bi.is_batch_invariant_mode_enabled()


def test_direct_kernel_calls_reject_cpu_tensors():
    with pytest.raises(ValueError, match="GPU"):
        bi.batch_invariant_matmul(torch.randn(2, 8), torch.randn(8, 4))
    with pytest.raises(ValueError, match="GPU"):
        bi.batch_invariant_rms_norm(torch.randn(2, 8), None, 1e-6)


def test_split_size_other_than_256_needs_the_per_key_order():
    """split_size is the reference's keyword: the per-key kernels take any
    size; the matrix-core kernels only the contract's 256, and an invalid size
    is rejected before any device check."""
    q = torch.randn(1, 2, 1, 64)
    with pytest.raises(ValueError, match="matrix-core kernels use 256-key splits"):
        bi.batch_invariant_decode_attention(q, q, q, scale=1.0, split_size=128, order="mfma")
    with pytest.raises(ValueError, match="split_size must be"):
        bi.batch_invariant_prefill_attention(q, q, q, scale=1.0, causal=True, split_size=0)


def test_causal_bias_masks_are_not_array_masks():
    """torch's CausalBias (causal_lower_right / causal_upper_left) maps to the
    kernel's causal mask; on CPU tensors it falls back as non-gpu-tensor and
    the stock result is returned unchanged."""
    from torch.nn.attention.bias import causal_lower_right, causal_upper_left
    torch.manual_seed(1)
    q = torch.randn((1, 2, 3, 32))
    kv = torch.randn((1, 2, 7, 32))
    lr, ul = causal_lower_right(3, 7), causal_upper_left(3, 7)
    ref_lr = F.scaled_dot_product_attention(q, kv, kv, attn_mask=lr)
    ref_ul = F.scaled_dot_product_attention(q, kv, kv, attn_mask=ul)
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        assert torch.equal(F.scaled_dot_product_attention(q, kv, kv, attn_mask=lr), ref_lr)
        assert torch.equal(F.scaled_dot_product_attention(q, kv, kv, attn_mask=ul), ref_ul)
        F.scaled_dot_product_attention(q, kv, kv, attn_mask=torch.ones((3, 7), dtype=torch.bool))
    assert bi.stats()["fallbacks"] == {"sdpa:non-gpu-tensor": 2, "sdpa:array-mask": 1}
    assert ops._causal_variant(lr, False, 3, 7) == (True, "lower_right")
    assert ops._causal_variant(ul, False, 3, 7) == (True, "upper_left")
    assert ops._causal_variant(None, True, 3, 7) == (True, "upper_left")
    assert ops._causal_variant(lr, True, 3, 7) == (False, None)
    assert ops._causal_variant(causal_lower_right(3, 6), False, 3, 7) == (False, None)


def test_dequantized_cache_follows_the_weight_tensor():
    """The dequantize-once cache entry matches only its own weight tensor and
    the scales / biases it was made from, goes with drop_dequantized, and goes
    when the weight tensor is collected (bookkeeping only: no GPU call)."""
    import gc
    import weakref
    from mlx_batch_invariant_amd.kernels import quantized as kq
    w = torch.zeros((4, 32), dtype=torch.int32)
    s, b = torch.zeros((4, 4)), torch.zeros((4, 4))
    key = id(w)

    def put():
        ref = weakref.ref(w, lambda _r, k=key: kq._DEQUANTIZED.pop(k, None)
                          if kq._DEQUANTIZED.get(k, (None,))[0] is _r else None)
        kq._DEQUANTIZED[key] = (ref, w.data_ptr(), s.data_ptr(), b.data_ptr(), 64, 4, torch.float32, "copy")

    put()
    assert kq._dequantized_for(w, s, b, 64, 4, torch.float32) == "copy"
    assert kq._dequantized_for(w, s.clone(), b, 64, 4, torch.float32) is None
    assert kq._dequantized_for(w, s, b, 32, 4, torch.float32) is None
    assert kq._dequantized_for(w.clone(), s, b, 64, 4, torch.float32) is None
    kq.drop_dequantized(w)
    assert key not in kq._DEQUANTIZED
    put()
    del w
    gc.collect()
    assert key not in kq._DEQUANTIZED
