"""Paged K/V attention on the GPU: the output over a shuffled page pool equals
the contiguous call on the same keys, bit for bit (paging changes addresses
only), for decode and causal prefill, several page sizes and both pool
layouts; and against the oracle on the K/V gathered from the pool."""

import math

import numpy as np
import pytest
import torch

from helpers import DT, assert_bits_equal, attn_bound_check, bits, gen, gpu_exp2, randn, to_np
from oracle import bi_oracle as ora

pytestmark = pytest.mark.gpu


def _bi():
    import mlx_batch_invariant_amd as bi
    return bi


def _paginate(k, v, page_size, g, token_major=False):
    """Scatter contiguous [B, Hkv, L, D] caches into a shuffled pool with spare
    pages of noise (a wrong page read shows). Returns (k_pool, v_pool, table)."""
    B, Hkv, L, D = k.shape
    npg = -(-L // page_size)
    total = B * npg + 5
    table = torch.randperm(total, generator=g)[:B * npg].reshape(B, npg)
    pools = []
    for src in (k, v):
        pool = (torch.randn((total, Hkv, page_size, D), generator=g) * 100).to(src.dtype).cuda()
        pad = torch.zeros((B, Hkv, npg * page_size, D), dtype=src.dtype, device=src.device)
        pad[:, :, :L] = src
        pages = pad.reshape(B, Hkv, npg, page_size, D).permute(0, 2, 1, 3, 4)    # [B, npg, Hkv, ps, D]
        pool[table.reshape(-1).cuda()] = pages.reshape(B * npg, Hkv, page_size, D)
        if token_major:                     # [pages, page_size, Hkv, D] storage, passed as a permuted view
            pool = pool.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        pools.append(pool)
    return pools[0], pools[1], table.to(torch.int32).cuda()


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("page_size", [1, 16, 64, 256, 1024])
def test_paged_decode_equals_contiguous(dt, page_size):
    bi = _bi()
    g = gen(page_size + len(dt))
    B, Hq, Hkv, L, D = 5, 32, 8, 1500, 128
    q = randn((B, Hq, 1, D), DT[dt], g)
    k = randn((B, Hkv, L, D), DT[dt], g)
    v = randn((B, Hkv, L, D), DT[dt], g)
    lens = torch.tensor([1, 255, 256, 1000, 1500], dtype=torch.int32).cuda()
    want = bi.batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=lens)
    kp, vp, table = _paginate(k, v, page_size, g)
    got = bi.batch_invariant_paged_attention(q, kp, vp, table, lens, scale=D ** -0.5)
    assert bits(got) == bits(want)


@pytest.mark.parametrize("page_size", [16, 256])
@pytest.mark.parametrize("token_major", [False, True])
def test_paged_prefill_equals_contiguous(page_size, token_major):
    bi = _bi()
    g = gen(page_size + 7 * token_major)
    B, Hq, Hkv, Tq, L, D = 3, 8, 2, 37, 700, 64
    q = randn((B, Hq, Tq, D), torch.bfloat16, g)
    k = randn((B, Hkv, L, D), torch.bfloat16, g)
    v = randn((B, Hkv, L, D), torch.bfloat16, g)
    lens = torch.tensor([37, 300, 700], dtype=torch.int32).cuda()
    want = bi.batch_invariant_prefill_attention(q, k, v, scale=D ** -0.5, causal=True, kv_lens=lens)
    kp, vp, table = _paginate(k, v, page_size, g, token_major=token_major)
    got = bi.batch_invariant_paged_attention(q, kp, vp, table, lens, scale=D ** -0.5, mask="causal")
    assert bits(got) == bits(want)
    got_nc = bi.batch_invariant_paged_attention(q, kp, vp, table, lens, scale=D ** -0.5)
    assert bits(got_nc) == bits(bi.batch_invariant_prefill_attention(q, k, v, scale=D ** -0.5, causal=False,
                                                                     kv_lens=lens))


def test_paged_decode_batch_invariant_and_errors():
    """A sequence's paged decode output does not depend on its batch
    companions or on where its pages sit in the pool."""
    bi = _bi()
    g = gen(3)
    B, Hq, Hkv, L, D = 4, 8, 2, 600, 128
    q = randn((B, Hq, 1, D), torch.bfloat16, g)
    k = randn((B, Hkv, L, D), torch.bfloat16, g)
    v = randn((B, Hkv, L, D), torch.bfloat16, g)
    lens = torch.tensor([600, 17, 333, 512], dtype=torch.int32).cuda()
    kp, vp, table = _paginate(k, v, 32, g)
    full = bi.batch_invariant_paged_attention(q, kp, vp, table, lens)
    for b in range(B):
        one = bi.batch_invariant_paged_attention(q[b:b + 1], kp, vp, table[b:b + 1], lens[b:b + 1])
        assert bits(one) == bits(full[b:b + 1]), b
    with pytest.raises(ValueError, match="power of two"):
        bi.batch_invariant_paged_attention(q, kp[:, :, :24], vp[:, :, :24], table, lens)


@pytest.mark.parametrize("page_size", [16, 64])
def test_paged_table_entries_are_clamped_into_the_pool(page_size):
    """A table entry outside [0, num_pages) is clamped into the pool by the
    kernels (a stale table reads wrong pages, never memory outside the pool):
    the output equals the call with the table clamped on the host."""
    bi = _bi()
    g = gen(40 + page_size)
    B, Hq, Hkv, L, D = 3, 8, 2, 400, 128
    q = randn((B, Hq, 1, D), torch.bfloat16, g)
    k = randn((B, Hkv, L, D), torch.bfloat16, g)
    v = randn((B, Hkv, L, D), torch.bfloat16, g)
    kp, vp, table = _paginate(k, v, page_size, g)
    npages = kp.shape[0]
    bad = table.clone()
    bad[0, 1] = -7
    bad[1, 0] = npages + 100
    bad[2, -1] = 2 ** 31 - 1
    lens = torch.tensor([400, 390, 400], dtype=torch.int32).cuda()
    clamped = bad.clamp(0, npages - 1)
    for Tq, mask in ((1, None), (9, "causal")):
        qq = randn((B, Hq, Tq, D), torch.bfloat16, g)
        got = bi.batch_invariant_paged_attention(qq, kp, vp, bad, lens, scale=D ** -0.5, mask=mask)
        want = bi.batch_invariant_paged_attention(qq, kp, vp, clamped, lens, scale=D ** -0.5, mask=mask)
        assert bits(got) == bits(want), Tq


@pytest.mark.parametrize("dt,D", [("bf16", 96), ("bf16", 256), ("f32", 256)])
def test_paged_other_head_dims_equal_contiguous(dt, D):
    bi = _bi()
    g = gen(D)
    B, Hq, Hkv, L = 3, 8, 2, 500
    q = randn((B, Hq, 1, D), DT[dt], g)
    k = randn((B, Hkv, L, D), DT[dt], g)
    v = randn((B, Hkv, L, D), DT[dt], g)
    lens = torch.tensor([500, 1, 300], dtype=torch.int32).cuda()
    want = bi.batch_invariant_decode_attention(q, k, v, scale=D ** -0.5, kv_lens=lens)
    for ps in (16, 128):
        kp, vp, table = _paginate(k, v, ps, g)
        got = bi.batch_invariant_paged_attention(q, kp, vp, table, lens, scale=D ** -0.5)
        assert bits(got) == bits(want), ps


def _gather(pool, table, L):
    """Host-side gather of a paged pool [pages, Hkv, page_size, D] (any
    strides) into contiguous [B, Hkv, L, D] through the block table: key p of
    sequence b is row p % page_size of page table[b, p // page_size]."""
    pool = pool.float().cpu().numpy()
    tab = table.cpu().numpy()
    ps = pool.shape[2]
    pos = np.arange(L)
    pages = tab[:, pos // ps]                                    # [B, L]
    return pool[pages, :, (pos % ps)[None, :], :].transpose(0, 2, 1, 3)   # [B, L, Hkv, D] -> [B, Hkv, L, D]


@pytest.mark.parametrize("page_size,token_major", [(16, False), (64, True), (256, False)])
def test_paged_decode_and_prefill_match_oracle_on_gathered_cache(page_size, token_major):
    """The paged kernels against the oracle run on K/V gathered from the pool
    on the host through the table: bit for bit against the emulation of the
    matrix-core order (hardware exp2), and within the stated bound of the
    reference's per-key order."""
    bi = _bi()
    g = gen(90 + page_size)
    B, Hq, Hkv, L, D = 3, 8, 2, 600, 128
    k = randn((B, Hkv, L, D), torch.bfloat16, g)
    v = randn((B, Hkv, L, D), torch.bfloat16, g)
    lens = np.array([600, 257, 1])
    kl = torch.tensor(lens, dtype=torch.int32).cuda()
    kp, vp, table = _paginate(k, v, page_size, g, token_major=token_major)
    kg, vg = _gather(kp, table, L), _gather(vp, table, L)
    sc = D ** -0.5
    for Tq, mask in ((1, None), (24, "causal")):
        q = randn((B, Hq, Tq, D), torch.bfloat16, g)
        lq = np.maximum(lens, Tq) if mask else lens            # causal chunks need len >= Tq
        klq = torch.tensor(lq, dtype=torch.int32).cuda()
        got = to_np(bi.batch_invariant_paged_attention(q, kp, vp, table, klq, scale=sc, mask=mask))
        want = ora.attention_mfma(to_np(q), kg, vg, sc, mask == "causal", "bf16", kv_lens=lq, exp2=gpu_exp2)
        assert_bits_equal(got, want, f"paged Tq={Tq} page={page_size}")
        ref = ora.attention(to_np(q), kg, vg, sc, mask == "causal", "bf16", kv_lens=lq)
        attn_bound_check(got, ref, to_np(q), kg, vg, sc, mask == "causal", "bf16", kv_lens=lq)
