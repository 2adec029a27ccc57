"""The default (matrix-core) attention kernels against the oracle's emulation
of their own order (oracle attention_mfma: MFMA score chains, split maximum,
hi/lo P, P.V and weight-sum MFMA chains, base-2 merge), bit for bit. The one
piece the emulation does not model, the hardware exp2 (v_exp_f32), is taken
from the GPU through bi_exp2_f32 and pinned here against the correctly
rounded exp2 (within one ulp, exact where the result is a power of two)."""

import math

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, gen, gpu_exp2, randn, to_np
from oracle import bi_oracle as ora

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _qkv(B, Hq, Hkv, Tq, L, D, dt, seed):
    g = gen(seed)
    return (randn((B, Hq, Tq, D), DT[dt], g), randn((B, Hkv, L, D), DT[dt], g),
            randn((B, Hkv, L, D), DT[dt], g))


def test_hardware_exp2_within_one_ulp_of_correctly_rounded():
    """v_exp_f32 against the correctly rounded exp2: exact at integer
    arguments with a normal result, within one ulp elsewhere in the normal
    range, and results below the normal range flushed to zero (measured: the
    instruction does not produce subnormals), which the oracle's default
    exp2_f32 follows."""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-30, 0, 200000), rng.uniform(-150, -120, 20000), rng.uniform(-1, 1, 50000),
                        -np.arange(0, 160, dtype=np.float64), [0.0, -0.0, -np.inf]]).astype(np.float32)
    got = gpu_exp2(x)
    want = ora.exp2_f32(x)
    exact64 = np.exp2(x.astype(np.float64))
    normal = exact64 >= 2.0 ** -126
    ints = np.isfinite(x) & (x == np.round(x)) & normal
    assert np.array_equal(got[ints], want[ints])          # powers of two exactly
    assert got[-1] == 0.0 and got[-3] == 1.0 and got[-2] == 1.0
    assert not got[~normal].any()                         # no subnormal results: flushed to +0
    assert np.array_equal(got[~normal], want[~normal])
    fin = np.isfinite(x) & normal
    ulps = np.abs(got[fin].astype(np.float64) - want[fin]) / ora.ulp(want[fin], "f32")
    assert ulps.max() <= 1.0, ulps.max()
    print(f"v_exp_f32: {np.mean(got[fin] != want[fin]):.4%} of normal results differ from correctly rounded "
          f"(max {ulps.max():.0f} ulp)")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,L,D", [(8, 2, 1000, 128), (4, 4, 300, 64), (32, 8, 513, 128), (8, 1, 256, 128),
                                         (4, 2, 700, 32), (4, 2, 300, 96), (4, 1, 520, 192), (2, 1, 600, 256)])
def test_decode_bitwise_equals_matrix_core_emulation(dt, Hq, Hkv, L, D):
    q, k, v = _qkv(2, Hq, Hkv, 1, L, D, dt, seed=L + D + Hq)
    sc = 1 / math.sqrt(D)
    got = to_np(_bi().batch_invariant_decode_attention(q, k, v, scale=sc))
    want = ora.attention_mfma(to_np(q), to_np(k), to_np(v), sc, False, dt, exp2=gpu_exp2)
    assert_bits_equal(got, want, f"decode {dt} Hq={Hq} Hkv={Hkv} L={L} D={D}")


def test_decode_ragged_config3_heads_bitwise_equals_emulation():
    """Config-3 heads (32 / 8, D = 128) with ragged lengths through split edges."""
    lens = np.array([1, 255, 256, 257, 1000, 2100])
    q, k, v = _qkv(len(lens), 32, 8, 1, int(lens.max()), 128, "bf16", seed=21)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    got = to_np(_bi().batch_invariant_decode_attention(q, k, v, scale=128 ** -0.5, kv_lens=kl))
    want = ora.attention_mfma(to_np(q), to_np(k), to_np(v), 128 ** -0.5, False, "bf16", kv_lens=lens, exp2=gpu_exp2)
    assert_bits_equal(got, want, "ragged decode")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Tq,L,D", [(37, 300, 64), (64, 600, 128), (5, 257, 32)])
def test_prefill_bitwise_equals_matrix_core_emulation(dt, causal, Tq, L, D):
    q, k, v = _qkv(2, 8, 2, Tq, L, D, dt, seed=Tq + L + D)
    sc = D ** -0.5
    got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=sc, causal=causal))
    want = ora.attention_mfma(to_np(q), to_np(k), to_np(v), sc, causal, dt, exp2=gpu_exp2)
    assert_bits_equal(got, want, f"prefill {dt} causal={causal} Tq={Tq} L={L} D={D}")


def test_prefill_kv_lens_bitwise_equals_emulation():
    """Per-sequence lengths with a causal chunk longer than one sequence (rows
    with no visible key give 0)."""
    lens = np.array([300, 20, 0])
    q, k, v = _qkv(3, 8, 2, 48, 300, 64, "bf16", seed=31)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=True, kv_lens=kl))
    want = ora.attention_mfma(to_np(q), to_np(k), to_np(v), 0.125, True, "bf16", kv_lens=lens, exp2=gpu_exp2)
    assert_bits_equal(got, want, "prefill kv_lens")


def test_emulation_with_correctly_rounded_exp2_stays_within_the_exp_error():
    """Without the hardware's exp2 values (correctly rounded exp2 instead,
    which v_exp_f32 differs from by at most one fp32 ulp) the emulation stays
    within half an output ulp of each side plus 4 * 2^-23 * sum p|v| / sum p
    of the GPU (each weight and its normalisation move by at most 2^-23
    relative, twice); most elements are still bit-equal."""
    q, k, v = _qkv(2, 8, 2, 40, 500, 128, "bf16", seed=41)
    sc = 128 ** -0.5
    got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=sc, causal=True))
    want = ora.attention_mfma(to_np(q), to_np(k), to_np(v), sc, True, "bf16")
    A = ora.attention_float64(to_np(q), to_np(k), np.abs(to_np(v)), sc, True)
    allow = 0.5 * (ora.ulp(got, "bf16") + ora.ulp(want, "bf16")) + 4 * 2.0 ** -23 * A
    assert (np.abs(got.astype(np.float64) - want) <= allow).all()
    assert np.mean(got == want) > 0.99
