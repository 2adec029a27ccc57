"""Attention in the reference's own per-key order (bi_attn_decode_per_key /
bi_attn_prefill_per_key) on the GPU: bit for bit equal to the oracle, which
restates the reference kernels' order (kernels/attention.py:1-85), and the
same invariance properties as the reference's tests check
(tests/test_batch_invariance.py: batch sweep, decode == prefill, chunked ==
one-shot)."""

import json
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, attn_bound_check, bits, gen, randn, to_np
from oracle import bi_oracle as ora
from sweep import sweep

pytestmark = pytest.mark.gpu

OUT = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"
PK = {"order": "per_key"}


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _qkv(B, Hq, Hkv, Tq, L, D, dt, seed):
    g = gen(seed)
    return (randn((B, Hq, Tq, D), DT[dt], g), randn((B, Hkv, L, D), DT[dt], g),
            randn((B, Hkv, L, D), DT[dt], g))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,L,D", [(8, 2, 1000, 128), (4, 4, 300, 64), (32, 8, 513, 128), (8, 1, 256, 32)])
def test_decode_equals_oracle_bitwise(dt, Hq, Hkv, L, D):
    q, k, v = _qkv(2, Hq, Hkv, 1, L, D, dt, seed=L + D)
    sc = D ** -0.5
    got = to_np(_bi().batch_invariant_decode_attention(q, k, v, scale=sc, **PK))
    want = ora.attention(to_np(q), to_np(k), to_np(v), sc, False, dt)
    assert_bits_equal(got, want, f"decode {dt} {Hq}/{Hkv} L={L} D={D}")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [64, 96, 256])
def test_prefill_equals_oracle_bitwise(dt, causal, D):
    q, k, v = _qkv(2, 8, 2, 37, 300, D, dt, seed=3 + D)
    got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=causal, **PK))
    want = ora.attention(to_np(q), to_np(k), to_np(v), 0.125, causal, dt)
    assert_bits_equal(got, want, f"prefill {dt} causal={causal} D={D}")


def test_long_fp32_decode_over_nine_splits_equals_oracle():
    q, k, v = _qkv(1, 8, 2, 1, 2304, 128, "f32", seed=23)
    sc = 128 ** -0.5
    got = to_np(_bi().batch_invariant_decode_attention(q, k, v, scale=sc, **PK))
    assert_bits_equal(got, ora.attention(to_np(q), to_np(k), to_np(v), sc, False, "f32"), "f32 L=2304")
    ref = ora.attention_float64(to_np(q), to_np(k), to_np(v), sc, False)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


def test_shared_head_units_equal_single_head_units():
    """At B * Hq * splits >= 16384 a decode unit scores 4 query heads of a kv
    head together; each sequence's rows equal its batch-1 call (one head per
    unit) and the oracle, bit for bit."""
    B, Hq, Hkv, L, D = 64, 32, 8, 2048, 128
    q, k, v = _qkv(B, Hq, Hkv, 1, L, D, "bf16", seed=41)
    sc = D ** -0.5
    out = _bi().batch_invariant_decode_attention(q, k, v, scale=sc, **PK)
    for b in (0, 37, B - 1):
        alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], scale=sc, **PK)
        assert bits(out[b:b + 1]) == bits(alone), b
    want = ora.attention(to_np(q[:1]), to_np(k[:1]), to_np(v[:1]), sc, False, "bf16")
    assert_bits_equal(to_np(out[:1]), want, "B=64 row 0")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_decode_batch_invariant(dt):
    Hq, Hkv, L, D = 8, 2, 600, 128
    q0, k0, v0 = _qkv(1, Hq, Hkv, 1, L, D, dt, seed=0)
    filler = lambda n, g: (randn((n, Hq, 1, D), DT[dt], g), randn((n, Hkv, L, D), DT[dt], g),
                           randn((n, Hkv, L, D), DT[dt], g))
    run = lambda t: _bi().batch_invariant_decode_attention(t[0], t[1], t[2], scale=D ** -0.5, **PK)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 3, 4, 8, 16, 32, 64])
    assert not fails, fails


def test_prefill_batch_invariant():
    Hq, Hkv, Tq, L, D = 8, 2, 48, 300, 128
    q0, k0, v0 = _qkv(1, Hq, Hkv, Tq, L, D, "bf16", seed=0)
    filler = lambda n, g: (randn((n, Hq, Tq, D), torch.bfloat16, g), randn((n, Hkv, L, D), torch.bfloat16, g),
                           randn((n, Hkv, L, D), torch.bfloat16, g))
    run = lambda t: _bi().batch_invariant_prefill_attention(t[0], t[1], t[2], scale=D ** -0.5, causal=True, **PK)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 3, 8, 16])
    assert not fails, fails


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [32, 128, 192])
def test_decode_equals_prefill_and_chunked_equals_one_shot(dt, D):
    """Reference tests test_decode_matches_prefill_position and the chunked
    prefill test: a prefill token equals the decode step for its position,
    and prefill in chunks over the growing cache equals one shot."""
    Hq, Hkv, T = 8, 2, 300
    q, k, v = _qkv(2, Hq, Hkv, T, T, D, dt, seed=D + len(dt))
    sc = D ** -0.5
    att = _bi().batch_invariant_attention
    full = att(q, k, v, scale=sc, mask="causal", **PK)
    for t in (0, 1, 255, 256, T - 1):
        dec = att(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=sc, **PK)
        assert bits(dec) == bits(full[:, :, t:t + 1]), t
    parts = [att(q[:, :, s:e], k[:, :, :e], v[:, :, :e], scale=sc, mask="causal", **PK)
             for s, e in ((0, 100), (100, 257), (257, T))]
    assert bits(torch.cat(parts, 2)) == bits(full)


def test_ragged_kv_lens_equal_alone_and_empty_rows_are_zero():
    Hq, Hkv, D, L = 8, 2, 128, 700
    q, k, v = _qkv(4, Hq, Hkv, 1, L, D, "bf16", seed=9)
    lens = [1, 256, 0, 700]
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    out = _bi().batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=kl, **PK)
    for b, n in enumerate(lens):
        if n == 0:
            assert not out[b].any()
            continue
        alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                       scale=D ** -0.5, **PK)
        assert bits(out[b:b + 1]) == bits(alone), b
    qp, kp, vp = _qkv(3, Hq, Hkv, 40, L, 64, "bf16", seed=10)
    plens = [40, 511, 20]          # the third: causal rows t < 20 see no key
    pout = _bi().batch_invariant_prefill_attention(qp, kp, vp, scale=0.125, causal=True,
                                                   kv_lens=torch.tensor(plens, dtype=torch.int32).cuda(), **PK)
    want = ora.attention(to_np(qp), to_np(kp), to_np(vp), 0.125, True, "bf16", kv_lens=plens)
    assert_bits_equal(to_np(pout), want, "prefill kv_lens")


def test_mode_runs_the_per_key_kernels_through_sdpa():
    import torch.nn.functional as F
    bi = _bi()
    q, k, v = _qkv(2, 8, 2, 33, 200, 64, "bf16", seed=12)
    want = bi.batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=True, **PK)
    with bi.set_batch_invariant_mode(strict=True, attention_order="per_key"):
        got = F.scaled_dot_product_attention(q, k[:, :, :33].repeat_interleave(4, 1),
                                             v[:, :, :33].repeat_interleave(4, 1), is_causal=True, scale=0.125)
        dec = F.scaled_dot_product_attention(q[:, :, -1:], k, v, enable_gqa=True, scale=0.125)
    alone = bi.batch_invariant_prefill_attention(q, k[:, :, :33].repeat_interleave(4, 1),
                                                 v[:, :, :33].repeat_interleave(4, 1), scale=0.125, causal=True, **PK)
    assert bits(got) == bits(alone)
    assert bits(dec) == bits(bi.batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=0.125, **PK))
    assert bits(dec) == bits(want[:, :, -1:])
    assert bi.ops.attention_order == "mfma"      # restored on exit


def test_matrix_core_order_within_stated_error_of_per_key_order():
    """The default (matrix-core) kernels against the reference order on the
    same inputs, config-3-like GQA decode and a full causal prefill: element
    by element within the bound the two orders imply (helpers.attn_bound:
    hi + lo weights of 16 significant bits, the per-key order's rescaling,
    score rounding, each scaled by sum p|v| / sum p) plus half a bf16 ulp of
    each side. The measured differences and the worst ratio are written out."""
    bi = _bi()
    sc = 128 ** -0.5
    report = {}
    for name, (B, Tq, L, causal, seed) in {"decode": (4, 1, 1500, False, 31),
                                           "prefill": (1, 256, 256, True, 32)}.items():
        q, k, v = _qkv(B, 32, 8, Tq, L, 128, "bf16", seed=seed)
        att = bi.batch_invariant_prefill_attention if Tq > 1 else (
            lambda *a, causal, **kw: bi.batch_invariant_decode_attention(*a, **kw))
        a = to_np(att(q, k, v, scale=sc, causal=causal))
        b = to_np(att(q, k, v, scale=sc, causal=causal, **PK))
        ratio = attn_bound_check(a, b, to_np(q), to_np(k), to_np(v), sc, causal, "bf16")
        report[name] = {"max_abs": float(np.abs(a - b).max()), "frac_equal": float(np.mean(a == b)),
                        "max_ulp_excess_no_allowance": ora.max_ulp_excess(a, b, "bf16"),
                        "worst_ratio_to_stated_bound": ratio}
    if OUT.is_dir():
        (OUT / "attn_mfma_vs_per_key.json").write_text(json.dumps(report))


@pytest.mark.parametrize("split", [1, 37, 128, 512])
def test_split_size_equals_oracle_and_keeps_invariance(split):
    """The reference's split_size keyword (attention.py:326-327, :368-370): any
    split size runs the per-key kernels, bitwise equal to the oracle at that
    split, with decode == prefill and chunked == one-shot at the same split."""
    Hq, Hkv, T, D = 8, 2, 300, 64
    q, k, v = _qkv(2, Hq, Hkv, T, T, D, "bf16", seed=split)
    sc = D ** -0.5
    att = _bi().batch_invariant_attention
    full = att(q, k, v, scale=sc, mask="causal", split_size=split)
    want = ora.attention(to_np(q[:1, :, -24:]), to_np(k[:1]), to_np(v[:1]), sc, True, "bf16", split=split)
    assert_bits_equal(to_np(full[:1, :, -24:]), want, f"prefill split={split}")
    dec = _bi().batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=sc, split_size=split)
    assert bits(dec) == bits(full[:, :, -1:])
    assert_bits_equal(to_np(dec[:1]), ora.attention(to_np(q[:1, :, -1:]), to_np(k[:1]), to_np(v[:1]), sc, False,
                                                     "bf16", split=split), f"decode split={split}")
    for t in (0, split - 1, split, T - 2):
        if 0 <= t < T:
            d = att(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=sc, split_size=split)
            assert bits(d) == bits(full[:, :, t:t + 1]), t
    parts = [att(q[:, :, s:e], k[:, :, :e], v[:, :, :e], scale=sc, mask="causal", split_size=split)
             for s, e in ((0, 90), (90, T))]
    assert bits(torch.cat(parts, 2)) == bits(full)
    if split != 256:
        with pytest.raises(ValueError):
            att(q, k, v, scale=sc, mask="causal", split_size=split, order="mfma")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("D", [160, 224, 320, 512])
def test_per_key_head_dims_beyond_the_matrix_core_set(dt, D):
    """Head dims only the per-key kernels take (any multiple of 32 up to 512,
    as the reference accepts): decode and causal prefill bitwise equal to the
    oracle, decode == prefill, ragged lengths equal alone; order=None and the
    mode pick these kernels for such a head dim."""
    bi = _bi()
    Hq, Hkv, T = 4, 2, 300
    g = gen(D + len(dt))
    q, k, v = (randn((2, Hq, T, D), DT[dt], g), randn((2, Hkv, T, D), DT[dt], g), randn((2, Hkv, T, D), DT[dt], g))
    sc = D ** -0.5
    full = bi.batch_invariant_prefill_attention(q, k, v, scale=sc, causal=True)        # order=None: per-key
    want = ora.attention(to_np(q[:1, :, -24:]), to_np(k[:1]), to_np(v[:1]), sc, True, dt)
    assert_bits_equal(to_np(full[:1, :, -24:]), want, f"prefill D={D}")
    dec = bi.batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=sc)
    assert bits(dec) == bits(full[:, :, -1:])
    lens = torch.tensor([T, 45], dtype=torch.int32).cuda()
    rag = bi.batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=sc, kv_lens=lens)
    alone = bi.batch_invariant_decode_attention(q[1:, :, -1:], k[1:, :, :45], v[1:, :, :45], scale=sc)
    assert bits(rag[1:]) == bits(alone)
    with pytest.raises(ValueError):
        bi.batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=sc, order="mfma")
    bi.reset_stats()
    with bi.set_batch_invariant_mode(strict=True):
        y = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=sc, enable_gqa=True)
    assert bi.stats()["handled"] == {"sdpa_prefill": 1}
    assert bits(y) == bits(full)
