"""RMSNorm on the GPU: bit-exact parity with the oracle, batch invariance."""

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


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D,rows", [(896, 64), (4096, 9), (100, 7), (2048, 3), (5000, 5), (9000, 3), (8, 2), (1, 4)])
def test_rms_norm_bit_exact_vs_oracle(dt, D, rows):
    g = gen(D + rows)
    x = randn((rows, D), DT[dt], g)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(DT[dt]).cuda()
    got = _bi().batch_invariant_rms_norm(x, w, 1e-6)
    want = ora.rms_norm(to_np(x), to_np(w), 1e-6, dt)
    np.testing.assert_array_equal(to_np(got), want)


def test_rms_norm_weight_none_and_fp32():
    g = gen(1)
    x = randn((5, 4096), torch.float32, g)
    got = _bi().batch_invariant_rms_norm(x, None, 1e-5)
    want = ora.rms_norm(to_np(x), None, 1e-5, "f32")
    # the oracle's fma is correctly rounded for any fp32 operands: bit-exact
    np.testing.assert_array_equal(to_np(got), want)


def test_rms_norm_strided_rows():
    g = gen(2)
    base = randn((6, 1024), torch.bfloat16, g)
    x = base[:, :896]                                  # row stride 1024
    got = _bi().batch_invariant_rms_norm(x, None, 1e-6)
    want = _bi().batch_invariant_rms_norm(x.contiguous(), None, 1e-6)
    assert bits(got) == bits(want)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [896, 4096])
def test_rms_norm_batch_invariant(dt, D):
    g = gen(0)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(DT[dt]).cuda()
    probe = randn((1, D), DT[dt], g)
    fails = sweep(probe, lambda n, gg: randn((n, D), DT[dt], gg),
                  lambda x: _bi().batch_invariant_rms_norm(x, w, 1e-6))
    assert not fails, fails
