"""LayerNorm on the GPU: bit-exact parity with the oracle, batch invariance,
interception of nn.LayerNorm by the mode."""

import numpy as np
import pytest
import torch

from helpers import DT, bits, gen, randn, to_np
from oracle import bi_oracle as ora
from sweep import sweep

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _params(D, dt, g):
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(DT[dt]).cuda()
    b = (0.1 * torch.randn(D, generator=g)).to(DT[dt]).cuda()
    return w, b


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D,rows", [(896, 64), (4096, 9), (100, 7), (2048, 3), (5000, 5), (9000, 3), (8, 2),
                                    (1, 4), (768, 5)])
def test_layer_norm_bit_exact_vs_oracle(dt, D, rows):
    g = gen(D + rows)
    x = (randn((rows, D), DT[dt], g) + 2.0).to(DT[dt])      # mean away from 0
    w, b = _params(D, dt, g)
    got = _bi().batch_invariant_layer_norm(x, w, b, 1e-5)
    want = ora.layer_norm(to_np(x), to_np(w), to_np(b), 1e-5, dt)
    np.testing.assert_array_equal(to_np(got), want)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_layer_norm_without_weight_or_bias(dt):
    g = gen(3)
    x = randn((7, 1000), DT[dt], g)
    w, b = _params(1000, dt, g)
    for ww, bb in ((None, None), (w, None), (None, b)):
        got = _bi().batch_invariant_layer_norm(x, ww, bb, 1e-5)
        want = ora.layer_norm(to_np(x), None if ww is None else to_np(ww), None if bb is None else to_np(bb),
                              1e-5, dt)
        np.testing.assert_array_equal(to_np(got), want)


def test_layer_norm_strided_rows_and_leading_dims():
    g = gen(2)
    base = randn((6, 1024), torch.bfloat16, g)
    x = base[:, :896]                                  # row stride 1024
    w, b = _params(896, "bf16", g)
    got = _bi().batch_invariant_layer_norm(x, w, b, 1e-5)
    assert bits(got) == bits(_bi().batch_invariant_layer_norm(x.contiguous(), w, b, 1e-5))
    x3 = randn((2, 3, 896), torch.bfloat16, g)
    got3 = _bi().batch_invariant_layer_norm(x3, w, b, 1e-5)
    assert bits(got3.reshape(6, 896)) == bits(_bi().batch_invariant_layer_norm(x3.reshape(6, 896), w, b, 1e-5))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [768, 4096])
def test_layer_norm_batch_invariant(dt, D):
    g = gen(0)
    w, b = _params(D, dt, g)
    probe = randn((1, D), DT[dt], g)
    fails = sweep(probe, lambda n, gg: randn((n, D), DT[dt], gg),
                  lambda x: _bi().batch_invariant_layer_norm(x, w, b, 1e-5))
    assert not fails, fails


def test_nn_layernorm_is_intercepted():
    bi = _bi()
    g = gen(4)
    ln = torch.nn.LayerNorm(768, eps=1e-5).to(torch.bfloat16).cuda()
    with torch.no_grad():
        ln.weight.copy_((1 + 0.1 * torch.randn(768, generator=g)).to(torch.bfloat16))
        ln.bias.copy_((0.1 * torch.randn(768, generator=g)).to(torch.bfloat16))
    x = randn((4, 5, 768), torch.bfloat16, g)
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        with torch.no_grad():
            y = ln(x)
    assert bi.stats()["handled"] == {"layer_norm": 1}
    assert bits(y) == bits(bi.batch_invariant_layer_norm(x, ln.weight, ln.bias, 1e-5))
    ref = torch.nn.functional.layer_norm(x.float(), (768,), ln.weight.float(), ln.bias.float(), 1e-5)
    assert torch.allclose(y.float(), ref, atol=2e-2, rtol=2e-2)
