"""The mode on GPU tensors: torch modules route through the kernels, with no
fallbacks in strict mode, and give the direct kernels' bits."""

import pytest
import torch
import torch.nn.functional as F

from helpers import bits, gen, randn

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def test_modules_route_through_mode():
    bi = _bi()
    torch.manual_seed(0)
    lin = torch.nn.Linear(896, 4864, bias=True).to(torch.bfloat16).cuda()
    lin_nb = torch.nn.Linear(896, 256, bias=False).to(torch.bfloat16).cuda()
    norm = torch.nn.RMSNorm(896, eps=1e-6).to(torch.bfloat16).cuda()
    x = randn((5, 896), torch.bfloat16, gen(1))
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        h = norm(x)
        y = lin(h)
        z = lin_nb(h)
        w = h @ lin_nb.weight.T
        q = randn((2, 8, 33, 64), torch.bfloat16, gen(2))
        kv = randn((2, 2, 33, 64), torch.bfloat16, gen(3))
        a = F.scaled_dot_product_attention(q, kv, kv, is_causal=True, enable_gqa=True)
        d = F.scaled_dot_product_attention(q[:, :, -1:], kv, kv, enable_gqa=True)
    st = bi.stats()
    assert st["fallbacks"] == {}
    assert st["handled"] == {"rms_norm": 1, "addmm": 1, "matmul": 2, "sdpa_prefill": 1, "sdpa_decode": 1}
    assert bits(h) == bits(bi.batch_invariant_rms_norm(x, norm.weight, 1e-6))
    assert bits(y) == bits(bi.batch_invariant_matmul(h, lin.weight.T) + lin.bias)
    assert bits(z) == bits(w)
    assert bits(a[:, :, -1:]) == bits(d)


def test_quantized_linear_routes_through_mode():
    bi = _bi()
    from mlx_batch_invariant_amd.nn import QuantizedLinear
    lin = QuantizedLinear(256, 64, bias=False, group_size=64, bits=4).cuda()
    x = randn((3, 256), torch.float16, gen(4))
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        y = lin(x)
    assert bi.stats()["handled"].get("quantized_matmul") == 1
    assert y.shape == (3, 64)


def test_strict_mode_raises_on_array_mask():
    bi = _bi()
    q = torch.randn((1, 4, 7, 64), device="cuda")
    m = torch.zeros((7, 7), dtype=torch.bool, device="cuda")
    with bi.set_batch_invariant_mode(strict=True):
        with pytest.raises(RuntimeError):
            F.scaled_dot_product_attention(q, q, q, attn_mask=m)


def test_causal_lower_right_is_the_kernel_causal_mask():
    """``attn_mask=causal_lower_right(T_q, L)`` (chunked prefill over a cache)
    runs the kernel's bottom-right causal mask; ``is_causal`` with T_q < L is
    top-left, i.e. the kernel on the first T_q keys."""
    bi = _bi()
    from torch.nn.attention.bias import causal_lower_right
    q = randn((2, 8, 5, 128), torch.bfloat16, gen(5))
    kv = randn((2, 2, 300, 128), torch.bfloat16, gen(6))
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        lr = F.scaled_dot_product_attention(q, kv, kv, attn_mask=causal_lower_right(5, 300), enable_gqa=True)
        ul = F.scaled_dot_product_attention(q, kv, kv, is_causal=True, enable_gqa=True)
    assert bi.stats()["handled"] == {"sdpa_prefill": 2}
    assert bits(lr) == bits(bi.batch_invariant_attention(q, kv, kv, mask="causal"))
    assert bits(ul) == bits(bi.batch_invariant_attention(q, kv[:, :, :5], kv[:, :, :5], mask="causal"))
    stock = F.scaled_dot_product_attention(q.float(), kv.float(), kv.float(),
                                           attn_mask=causal_lower_right(5, 300), enable_gqa=True)
    assert torch.allclose(lr.float(), stock, atol=2e-2, rtol=2e-2)


def test_addmm_beta_zero_ignores_c_and_mixed_dtype_falls_back():
    """As stock torch.addmm: with beta = 0, c is not read (NaN / Inf in it do
    not propagate) and the result is alpha * (a @ b) broadcast to c's shape; a
    c whose dtype differs from the product goes to the stock op (counted),
    which raises its own error."""
    bi = _bi()
    a = randn((4, 256), torch.bfloat16, gen(7))
    b = randn((256, 96), torch.bfloat16, gen(8))
    c = torch.full((4, 96), float("nan"), dtype=torch.bfloat16, device="cuda")
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        y = torch.addmm(c, a, b, beta=0)
        y2 = torch.addmm(c[0], a, b, beta=0, alpha=2)
    assert bi.stats()["handled"] == {"addmm": 2}
    prod = bi.batch_invariant_matmul(a, b)
    assert bits(y) == bits(prod)
    assert bits(y2) == bits(prod * 2)
    bi.reset_stats()
    with bi.set_batch_invariant_mode():
        with pytest.raises(RuntimeError):
            torch.addmm(c.float(), a, b)
    assert bi.stats()["fallbacks"] == {"addmm:dtype-mismatch": 1}
