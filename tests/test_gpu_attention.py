"""Attention on the GPU: parity with the oracle and the float64 closed form,
known answers, batch invariance (also with ragged kv_lens), chunked prefill ==
one-shot prefill, decode == prefill for the same position."""

import math

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, attn_bound_check, bits, gen, gpu_exp2, randn, to_np
from oracle import bi_oracle as ora
from sweep import sweep

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _qkv(B, Hq, Hkv, Tq, L, D, dt, seed):
    g = gen(seed)
    return (randn((B, Hq, Tq, D), DT[dt], g), randn((B, Hkv, L, D), DT[dt], g),
            randn((B, Hkv, L, D), DT[dt], g))


def _tol_check(got, want, dt, q, k, v, scale, causal, kv_lens=None):
    """The matrix-core kernels against the per-key (reference-order) oracle:
    element by element within half a storage ulp of each side plus the bound
    the two orders imply (helpers.attn_bound: hi/lo weights, per-key
    rescaling, score rounding, each scaled by sum p|v| / sum p). Returns the
    worst ratio of difference to allowance (<= 1)."""
    f = lambda t: to_np(t) if isinstance(t, torch.Tensor) else t
    return attn_bound_check(got, want, f(q), f(k), f(v), scale, causal, dt, kv_lens)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Hq,Hkv,L,D", [(8, 2, 1000, 128), (4, 4, 300, 64), (32, 8, 513, 128), (8, 1, 256, 128)])
def test_decode_matches_oracle(dt, Hq, Hkv, L, D):
    q, k, v = _qkv(2, Hq, Hkv, 1, L, D, dt, seed=L + D)
    sc = 1 / math.sqrt(D)
    got = to_np(_bi().batch_invariant_decode_attention(q, k, v, scale=sc))
    want = ora.attention(to_np(q), to_np(k), to_np(v), sc, False, dt)
    _tol_check(got, want, dt, q, k, v, sc, False)
    ref64 = ora.attention_float64(to_np(q), to_np(k), to_np(v), sc, False)
    assert np.abs(got - ref64).max() < (2e-2 if dt == "bf16" else 4e-3)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_oracle(dt, causal):
    q, k, v = _qkv(2, 8, 2, 37, 300, 64, dt, seed=3)
    got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=causal))
    want = ora.attention(to_np(q), to_np(k), to_np(v), 0.125, causal, dt)
    _tol_check(got, want, dt, q, k, v, 0.125, causal)


def test_prefill_matches_float64_closed_form():
    """Reference test_prefill_matches_stock_causal_with_cache, against float64."""
    q, k, v = _qkv(2, 8, 2, 37, 150, 64, "f32", seed=3)
    for causal in (True, False):
        got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=causal))
        ref = ora.attention_float64(to_np(q), to_np(k), to_np(v), 0.125, causal)
        assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-4


def test_single_key_returns_v_exactly():
    q, k, v = _qkv(3, 8, 2, 1, 1, 128, "bf16", seed=4)
    got = _bi().batch_invariant_decode_attention(q, k, v, scale=0.1)
    want = v[:, :, 0:1, :].repeat_interleave(4, dim=1)
    assert bits(got) == bits(want)


def test_equal_scores_give_mean_of_v():
    """scale = 0 makes every score 0: out = mean of V (exact for a power-of-2 count
    of V rows that are small integers)."""
    g = gen(5)
    L = 256
    q = randn((1, 4, 1, 128), torch.bfloat16, g)
    k = randn((1, 4, L, 128), torch.bfloat16, g)
    v = torch.randint(-4, 5, (1, 4, L, 128), generator=g).to(torch.bfloat16).cuda()
    got = _bi().batch_invariant_decode_attention(q, k, v, scale=0.0)
    want = v.float().mean(dim=2, keepdim=True)
    np.testing.assert_allclose(to_np(got), to_np(want), rtol=0, atol=to_np(want).__abs__().max() * 2 ** -7)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_decode_batch_invariant(dt):
    Hq, Hkv, L, D = 8, 2, 1000, 128
    q0, k0, v0 = _qkv(1, Hq, Hkv, 1, L, D, dt, seed=0)
    filler = lambda n, g: (randn((n, Hq, 1, D), DT[dt], g), randn((n, Hkv, L, D), DT[dt], g),
                           randn((n, Hkv, L, D), DT[dt], g))
    run = lambda t: _bi().batch_invariant_decode_attention(t[0], t[1], t[2], scale=D ** -0.5)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 3, 4, 8, 16, 32, 64])
    assert not fails, fails


def test_decode_ragged_kv_lens_equal_alone():
    """per-sequence lengths in one batch; each sequence's
    output equals running it alone with K/V cut to its own length."""
    Hq, Hkv, D, L = 32, 8, 128, 2100
    rng = np.random.default_rng(0)
    B = 12
    lens = rng.integers(1, L + 1, size=B)
    lens[0], lens[1], lens[2], lens[3] = 1, 256, 257, L
    q, k, v = _qkv(B, Hq, Hkv, 1, L, D, "bf16", seed=8)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    out = _bi().batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=kl)
    for b in range(B):
        n = int(lens[b])
        alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                       scale=D ** -0.5)
        assert bits(out[b:b + 1]) == bits(alone), (b, n)


def test_decode_dynamic_items_equal_alone_and_replay():
    """A ragged batch with many more split items than the resident grid takes
    the dynamic item order (a counter in the workspace, zeroed by a fill
    kernel per call). Each sequence must equal running it alone (the static
    order), on repeated calls and on replays of a captured graph."""
    Hq, Hkv, D, L = 32, 8, 128, 4096
    rng = np.random.default_rng(3)
    B = 48
    lens = rng.integers(1, L + 1, size=B)
    lens[0], lens[1], lens[2], lens[-1] = 1, 256, 257, L
    q, k, v = _qkv(B, Hq, Hkv, 1, L, D, "bf16", seed=9)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    run = lambda: _bi().batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=kl)
    out = run()
    for b in range(B):
        n = int(lens[b])
        alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                       scale=D ** -0.5)
        assert bits(out[b:b + 1]) == bits(alone), (b, n)
    assert bits(run()) == bits(out)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gout = run()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert bits(gout) == bits(out)
        assert bits(run()) == bits(out)   # eager work between replays


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_chunked_prefill_and_decode_equivalence(dt):
    """Reference attention_structure_checks (harness/sweep.py:188-207): T=600,
    chunk at T1=257 (off the 256 split), decode(last) == prefill(last)."""
    Hq, Hkv, D, T, T1 = 8, 2, 128, 600, 257
    q, k, v = _qkv(2, Hq, Hkv, T, T, D, dt, seed=0)
    sc = D ** -0.5
    att = _bi().batch_invariant_attention
    full = att(q, k, v, scale=sc, mask="causal")
    part1 = att(q[:, :, :T1], k[:, :, :T1], v[:, :, :T1], scale=sc, mask="causal")
    part2 = att(q[:, :, T1:], k, v, scale=sc, mask="causal")
    assert bits(torch.cat([part1, part2], 2)) == bits(full)
    dec = att(q[:, :, T - 1:T], k, v, scale=sc)
    assert bits(dec) == bits(full[:, :, T - 1:T])
    for t in (0, 1, 255, 256, 300, 511, 512, 599):
        d = att(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=sc)
        assert bits(d) == bits(full[:, :, t:t + 1]), t


def test_prefill_chunks_128_512_llama_gqa():
    """BASELINE config 4 shape (GQA 32/8, D=128) at T=2048: chunks of 128 and
    512 against the cache equal one-shot prefill."""
    Hq, Hkv, D, T = 32, 8, 128, 2048
    q, k, v = _qkv(1, Hq, Hkv, T, T, D, "bf16", seed=2)
    sc = D ** -0.5
    att = _bi().batch_invariant_prefill_attention
    full = att(q, k, v, scale=sc, causal=True)
    for C in (128, 512):
        parts = [att(q[:, :, s:s + C], k[:, :, :s + C], v[:, :, :s + C], scale=sc, causal=True)
                 for s in range(0, T, C)]
        assert bits(torch.cat(parts, 2)) == bits(full), C


def test_prefill_batch_invariant():
    Hq, Hkv, Tq, L, D = 8, 2, 48, 300, 128
    q0, k0, v0 = _qkv(1, Hq, Hkv, Tq, L, D, "bf16", seed=0)
    filler = lambda n, g: (randn((n, Hq, Tq, D), torch.bfloat16, g), randn((n, Hkv, L, D), torch.bfloat16, g),
                           randn((n, Hkv, L, D), torch.bfloat16, g))
    run = lambda t: _bi().batch_invariant_prefill_attention(t[0], t[1], t[2], scale=D ** -0.5, causal=True)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 3, 8, 16])
    assert not fails, fails


def test_prefill_batch_invariant_config4_size():
    """BASELINE config 4 at its size: causal T = 2048, GQA 32 / 8, D = 128,
    bf16; the probe sequence at the first and the last position of batches
    of 1 to 16 (the benchmarked B = 16 launch included) gives the batch-1
    bits (fillers drawn on the device)."""
    Hq, Hkv, T, D = 32, 8, 2048, 128
    q0, k0, v0 = _qkv(1, Hq, Hkv, T, T, D, "bf16", seed=12)

    def filler(n, g):
        gd = torch.Generator(device="cuda").manual_seed(int(torch.randint(0, 2 ** 31, (1,), generator=g)))
        r = lambda *s: torch.randn(s, generator=gd, device="cuda").to(torch.bfloat16)
        return r(n, Hq, T, D), r(n, Hkv, T, D), r(n, Hkv, T, D)

    run = lambda t: _bi().batch_invariant_prefill_attention(t[0], t[1], t[2], scale=D ** -0.5, causal=True)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 4, 8, 16])
    assert not fails, fails


def test_prefill_kv_lens_equal_alone():
    Hq, Hkv, D, L, Tq = 8, 2, 64, 700, 40
    q, k, v = _qkv(3, Hq, Hkv, Tq, L, D, "bf16", seed=9)
    lens = [40, 511, 700]
    out = _bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=True,
                                                  kv_lens=torch.tensor(lens, dtype=torch.int32).cuda())
    for b, n in enumerate(lens):
        alone = _bi().batch_invariant_prefill_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                        scale=0.125, causal=True)
        assert bits(out[b:b + 1]) == bits(alone), b


def test_strided_kv_cache_view():
    """K/V read through strides: a cache preallocated for 1024 positions and
    viewed at 600 gives the same bits as a compact copy."""
    Hq, Hkv, D = 8, 2, 128
    q, k, v = _qkv(2, Hq, Hkv, 1, 1024, D, "bf16", seed=10)
    a = _bi().batch_invariant_decode_attention(q, k[:, :, :600], v[:, :, :600], scale=0.1)
    b = _bi().batch_invariant_decode_attention(q, k[:, :, :600].contiguous(), v[:, :, :600].contiguous(), scale=0.1)
    assert bits(a) == bits(b)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_zero_length_sequences_give_zeros(dt):
    """kv_lens[b] = 0 (and negative lengths, clamped to 0) has no key and no
    softmax: the output is defined as 0, and the other sequences of the batch
    still equal themselves run alone."""
    Hq, Hkv, D, L = 32, 8, 128, 600
    q, k, v = _qkv(5, Hq, Hkv, 1, L, D, dt, seed=12)
    lens = [0, 300, -4, 1, 600]
    out = _bi().batch_invariant_decode_attention(q, k, v, scale=D ** -0.5,
                                                 kv_lens=torch.tensor(lens, dtype=torch.int32).cuda())
    assert torch.isfinite(out).all()
    for b, n in enumerate(lens):
        if n <= 0:
            assert bits(out[b]) == bits(torch.zeros_like(out[b])), b
        else:
            alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                           scale=D ** -0.5)
            assert bits(out[b:b + 1]) == bits(alone), b


def test_causal_prefill_kv_lens_shorter_than_chunk():
    """A causal chunk of T_q tokens against a sequence with fewer than T_q
    keys: query t sees len - T_q + t + 1 keys; rows that see none are 0 (not
    0/0), the others equal the oracle and a decode step over their keys."""
    Hq, Hkv, D, L, Tq = 8, 2, 64, 300, 40
    q, k, v = _qkv(2, Hq, Hkv, Tq, L, D, "bf16", seed=13)
    lens = [10, 300]
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    out = _bi().batch_invariant_prefill_attention(q, k, v, scale=0.125, causal=True, kv_lens=kl)
    assert torch.isfinite(out).all()
    got = to_np(out)
    want = ora.attention(to_np(q), to_np(k), to_np(v), 0.125, True, "bf16", kv_lens=lens)
    _tol_check(got, want, "bf16", q, k, v, 0.125, True, kv_lens=lens)
    n0 = lens[0]
    for t in range(Tq):
        nk = n0 - Tq + t + 1
        if nk <= 0:
            assert not got[0, :, t].any(), t
        else:
            d = _bi().batch_invariant_decode_attention(q[0:1, :, t:t + 1], k[0:1, :, :nk], v[0:1, :, :nk],
                                                       scale=0.125)
            assert bits(d) == bits(out[0:1, :, t:t + 1]), t


def _report(name, payload):
    import json
    import os
    from pathlib import Path
    out = Path(os.environ.get("GRAFT_REPO_ROOT", Path(__file__).resolve().parent.parent)) / "gpurun_out"
    if out.is_dir():
        (out / name).write_text(json.dumps(payload, indent=1))


def _ulp_err(got, want, dt):
    """max |got - want| in storage ulps of want, and max |got - want|."""
    d = np.abs(got.astype(np.float64) - want)
    return float(np.max(d / ora.ulp(want, dt))), float(d.max())


def test_decode_config3_full_size():
    """BASELINE config 3 at its size: B = 256 sequences with lengths drawn from
    U{1..8192} (the bench's batch), GQA 32/8, D = 128, bf16. Sampled sequences
    equal themselves run alone, bit for bit; three of them match the per-key
    oracle within one bf16 ulp after the stated allowance."""
    Hq, Hkv, D, L, B = 32, 8, 128, 8192, 256
    lens = np.random.default_rng(B).integers(1, L + 1, size=B)
    g = torch.Generator(device="cuda").manual_seed(77)      # 2 x 2 GiB of K/V: drawn on the device
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, L, D), generator=g, device="cuda", dtype=torch.bfloat16)
    v = torch.randn((B, Hkv, L, D), generator=g, device="cuda", dtype=torch.bfloat16)
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    out = _bi().batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=kl)
    picks = sorted({0, B - 1, int(np.argmax(lens)), int(np.argmin(lens)), 17, 100, 200})
    for b in picks:
        n = int(lens[b])
        alone = _bi().batch_invariant_decode_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                                                       scale=D ** -0.5)
        assert bits(out[b:b + 1]) == bits(alone), (b, n)
    errs, ratios = {}, {}
    for b in (int(np.argmax(lens)), int(np.argmin(lens)), 100):
        n = int(lens[b])
        qb, kb, vb = to_np(q[b:b + 1]), to_np(k[b:b + 1, :, :n]), to_np(v[b:b + 1, :, :n])
        got = to_np(out[b:b + 1])
        # bit for bit against the emulation of the kernels' own order (hardware exp2)
        assert_bits_equal(got, ora.attention_mfma(qb, kb, vb, D ** -0.5, False, "bf16", exp2=gpu_exp2),
                          f"config 3, sequence {b} (len {n})")
        want = ora.attention(qb, kb, vb, D ** -0.5, False, "bf16")
        ratios[n] = _tol_check(got, want, "bf16", qb, kb, vb, D ** -0.5, False)
        errs[n] = _ulp_err(got, want, "bf16")
    _report("attn_err_config3.json", {"max_err_vs_per_key_oracle (ulps, abs) by length": errs,
                                      "worst ratio to the stated bound by length": ratios,
                                      "bitwise_vs_matrix_core_emulation": True})


def test_prefill_config4_tokens_equal_decode_steps():
    """BASELINE config 4 shape (GQA 32/8, D = 128, T = 2048, bf16, causal):
    each sampled token of a one-shot prefill equals a later single-token decode
    step for that position, bit for bit, and the per-key oracle within one bf16
    ulp after the stated allowance."""
    Hq, Hkv, D, T = 32, 8, 128, 2048
    q, k, v = _qkv(2, Hq, Hkv, T, T, D, "bf16", seed=21)
    sc = D ** -0.5
    full = _bi().batch_invariant_prefill_attention(q, k, v, scale=sc, causal=True)
    errs, ratios = {}, {}
    for t in (0, 1, 255, 256, 511, 1023, 1500, 2047):
        dec = _bi().batch_invariant_decode_attention(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=sc)
        assert bits(dec) == bits(full[:, :, t:t + 1]), t
        qt, kt, vt = to_np(q[:1, :, t:t + 1]), to_np(k[:1, :, :t + 1]), to_np(v[:1, :, :t + 1])
        got = to_np(full[:1, :, t:t + 1])
        assert_bits_equal(got, ora.attention_mfma(qt, kt, vt, sc, False, "bf16", exp2=gpu_exp2), f"config 4, token {t}")
        want = ora.attention(qt, kt, vt, sc, False, "bf16")
        ratios[t] = _tol_check(got, want, "bf16", qt, kt, vt, sc, False)
        errs[t] = _ulp_err(got, want, "bf16")
    _report("attn_err_config4.json", {"max_err_vs_per_key_oracle (ulps, abs) by token": errs,
                                      "worst ratio to the stated bound by token": ratios,
                                      "bitwise_vs_matrix_core_emulation": True})


def test_fp32_prefill_closed_form_d128_long():
    """fp32 at D = 128 over 2304 keys (nine splits), causal and not: within a
    relative 1e-5 of the float64 softmax closed form (the in-split order, the
    hardware exp2 and the split merge together)."""
    q, k, v = _qkv(1, 8, 2, 64, 2304, 128, "f32", seed=23)
    sc = 128 ** -0.5
    for causal in (True, False):
        got = to_np(_bi().batch_invariant_prefill_attention(q, k, v, scale=sc, causal=causal))
        ref = ora.attention_float64(to_np(q), to_np(k), to_np(v), sc, causal)
        rel = float(np.abs(got - ref).max() / np.abs(ref).max())
        _report(f"attn_fp32_closed_form_causal{int(causal)}.json", {"max_rel_err": rel})
        assert rel < 1e-5, (causal, rel)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [32, 96, 192, 256])
def test_every_head_dim_matches_oracle_and_decode_equals_prefill(dt, D):
    """Head dims the reference accepts (any D % 32 == 0, attention.py:299-310)
    beyond 64 / 128: decode and causal prefill match the per-key oracle within
    one storage ulp after the stated allowance, a prefill token equals the
    decode step for its position bit for bit, and chunked prefill equals
    one-shot (fp32 at D > 128 stages V in two dim slices in decode and runs a
    two-buffer K/V ring in prefill)."""
    Hq, Hkv, T = 8, 2, 300
    q, k, v = _qkv(2, Hq, Hkv, T, T, D, dt, seed=D + len(dt))
    sc = D ** -0.5
    att = _bi().batch_invariant_attention
    full = att(q, k, v, scale=sc, mask="causal")
    want = ora.attention(to_np(q[:1, :, -40:]), to_np(k[:1]), to_np(v[:1]), sc, True, dt)
    _tol_check(to_np(full[:1, :, -40:]), want, dt, q[:1, :, -40:], k[:1], v[:1], sc, True)
    assert_bits_equal(to_np(full[:1, :, -40:]),
                      ora.attention_mfma(to_np(q[:1, :, -40:]), to_np(k[:1]), to_np(v[:1]), sc, True, dt, exp2=gpu_exp2),
                      f"{dt} D={D}")
    for t in (0, 255, 256, T - 1):
        dec = att(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1], scale=sc)
        assert bits(dec) == bits(full[:, :, t:t + 1]), t
    part1 = att(q[:, :, :100], k[:, :, :100], v[:, :, :100], scale=sc, mask="causal")
    part2 = att(q[:, :, 100:], k, v, scale=sc, mask="causal")
    assert bits(torch.cat([part1, part2], 2)) == bits(full)
    lens = torch.tensor([T, 37], dtype=torch.int32).cuda()
    rag = _bi().batch_invariant_decode_attention(q[:, :, -1:], k, v, scale=sc, kv_lens=lens)
    alone = _bi().batch_invariant_decode_attention(q[1:, :, -1:], k[1:, :, :37], v[1:, :, :37], scale=sc)
    assert bits(rag[1:]) == bits(alone)


@pytest.mark.parametrize("D", [96, 256])
def test_every_head_dim_batch_invariant(D):
    Hq, Hkv, L = 8, 2, 700
    q0, k0, v0 = _qkv(1, Hq, Hkv, 1, L, D, "bf16", seed=D)
    filler = lambda n, g: (randn((n, Hq, 1, D), torch.bfloat16, g), randn((n, Hkv, L, D), torch.bfloat16, g),
                           randn((n, Hkv, L, D), torch.bfloat16, g))
    run = lambda t: _bi().batch_invariant_decode_attention(t[0], t[1], t[2], scale=D ** -0.5)
    fails = sweep((q0, k0, v0), filler, run, batches=[1, 2, 5, 16])
    assert not fails, fails
